"""GPU parity of the decode step (aq_decode.hip, alpacca_amd/model.py) with
the oracle (oracle/model_ref.py), through the C ABI.

Bars: RoPE and the KV store bit-identical to the reference's NumPy rotation;
argmax exact (first maximum); RMSNorm, SwiGLU and attention within a few
float32 ulps of the oracle (stated per test); model logits within the
matvec bar (2e-5 of ||W_r||*||x||, per layer, compounding over the layers:
1e-4 relative to the largest logit here); greedy tokens identical.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from alpacca_amd import _lib
from alpacca_amd.model import Hyperparams, Model, synthetic_llama_1b
from oracle import model_ref as MR

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev():
    _lib.ensure_device()
    return torch.device("cuda", 0)


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def state_tensor(token=0, pos=0, fed=0, count=0):
    st = np.zeros(8, np.int32)
    st[0:2] = np.array([token], np.int64).view(np.int32)
    st[4], st[5], st[6] = pos, fed, count
    return torch.from_numpy(st).to(dev())


def read_state(st):
    a = st.cpu().numpy()
    return {"token": int(a[0:2].view(np.int64)[0]), "key": int(a[2:4].view(np.uint64)[0]),
            "pos": int(a[4]), "fed": int(a[5]), "count": int(a[6])}


def _hp(style, n_head, n_kv, hd, n_rot):
    return Hyperparams(arch="llama", n_layer=1, n_embd=n_head * hd, n_head=n_head, n_kv=n_kv,
                       n_ff=64, n_vocab=64, n_ctx_train=4096, head_dim=hd, n_rot=n_rot,
                       rms_eps=1e-5, rope_base=500000.0, rope_style=style)


@pytest.mark.parametrize("rows,n", [(1, 2048), (3, 4096), (2, 333)])
def test_rmsnorm(rows, n):
    print(f"rmsnorm rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(rows + n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    xd, wd = torch.from_numpy(x).to(dev()), torch.from_numpy(w).to(dev())
    out = torch.empty_like(xd)
    _lib.check(_lib.load().aq_rmsnorm(P(xd), P(wd), rows, n, ctypes.c_float(1e-5), P(out), None))
    got = out.cpu().numpy()
    ref = MR.rmsnorm(x if rows > 1 else x[0], w, 1e-5).reshape(rows, n)
    assert np.abs(got - ref).max() <= 4e-7 * np.abs(ref).max()
    # in place
    _lib.check(_lib.load().aq_rmsnorm(P(xd), P(wd), rows, n, ctypes.c_float(1e-5), P(xd), None))
    assert np.array_equal(xd.cpu().numpy(), got)


@pytest.mark.parametrize("rows,n", [(1, 2048), (5, 4096), (3, 333), (2048, 2048)])
def test_add_rmsnorm_equals_add_then_rmsnorm(rows, n):
    """aq_add_rmsnorm (the batched step's residual add and the next RMSNorm
    in one launch) stores the same x and out bits as aq_add followed by
    aq_rmsnorm, and out is the oracle's rmsnorm of x + y (float32 adds)."""
    print(f"add_rmsnorm rows={rows} n={n}", flush=True)
    lib = _lib.load()
    rng = np.random.default_rng(7 * rows + n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    y = rng.standard_normal((rows, n)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    d = dev()
    xa, ya, wd = (torch.from_numpy(a).to(d) for a in (x, y, w))
    xb = xa.clone()
    out_a, out_b = torch.empty_like(xa), torch.empty_like(xa)
    eps = ctypes.c_float(1e-5)
    _lib.check(lib.aq_add_rmsnorm(P(xa), P(ya), P(wd), rows, n, eps, P(out_a), None))
    _lib.check(lib.aq_add(P(xb), P(ya), rows * n, None))
    _lib.check(lib.aq_rmsnorm(P(xb), P(wd), rows, n, eps, P(out_b), None))
    assert np.array_equal(xa.cpu().numpy(), xb.cpu().numpy())
    assert np.array_equal(out_a.cpu().numpy(), out_b.cpu().numpy())
    s = x + y
    assert np.array_equal(xa.cpu().numpy(), s)
    ref = np.stack([MR.rmsnorm(s[r], w, 1e-5) for r in range(min(rows, 8))])
    got = out_a.cpu().numpy()[:len(ref)]
    assert np.abs(got - ref).max() <= 4e-7 * np.abs(ref).max()
    # out may not alias x or y
    with pytest.raises(ValueError, match="aliases"):
        _lib.check(lib.aq_add_rmsnorm(P(xa), P(ya), P(wd), rows, n, eps, P(xa), None))


@pytest.mark.parametrize("style,n_head,n_kv,hd,n_rot",
                         [("norm", 32, 8, 64, 64), ("neox", 8, 2, 128, 128),
                          ("norm", 4, 4, 64, 32), ("neox", 4, 1, 64, 48)])
def test_rope_kv_bit_exact(style, n_head, n_kv, hd, n_rot):
    print(f"rope {style} {n_head}/{n_kv} hd={hd} n_rot={n_rot}", flush=True)
    hp = _hp(style, n_head, n_kv, hd, n_rot)
    n_ctx, T, pos0 = 300, 5, 290
    cos, sin = MR.rope_tables(hp, n_ctx)
    rng = np.random.default_rng(hd + n_rot)
    q = rng.standard_normal((T, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    d = dev()
    qd, kd, vd = (torch.from_numpy(a).to(d) for a in (q, k, v))
    cd, sd = torch.from_numpy(cos).to(d), torch.from_numpy(sin).to(d)
    kc = torch.zeros((n_kv, n_ctx, hd), device=d)
    vc = torch.zeros((n_kv, n_ctx, hd), device=d)
    lib = _lib.load()
    _lib.check(lib.aq_rope_kv(P(qd), P(kd), P(vd), T, n_head, n_kv, hd, n_rot,
                              1 if style == "neox" else 0, P(cd), P(sd), None, pos0, n_ctx,
                              P(kc), P(vc), None))
    pos = np.arange(pos0, pos0 + T)
    qr = MR.rope_batch_np(q, n_head, pos, hp, cos, sin)
    kr = MR.rope_batch_np(k, n_kv, pos, hp, cos, sin).reshape(T, n_kv, hd)
    assert np.array_equal(qd.cpu().numpy(), qr)
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    assert np.array_equal(kcn[:, pos0:pos0 + T].transpose(1, 0, 2), kr)
    assert np.array_equal(vcn[:, pos0:pos0 + T].transpose(1, 0, 2), v.reshape(T, n_kv, hd))
    assert not kcn[:, :pos0].any() and not vcn[:, :pos0].any()
    # the device-state position gives the same result (decode form, T = 1)
    st = state_tensor(pos=7)
    q1 = torch.from_numpy(q[:1].copy()).to(d)
    _lib.check(lib.aq_rope_kv(P(q1), P(kd), P(vd), 1, n_head, n_kv, hd, n_rot,
                              1 if style == "neox" else 0, P(cd), P(sd), P(st), 0, n_ctx,
                              P(kc), P(vc), None))
    assert np.array_equal(q1.cpu().numpy()[0], MR.rope_np(q[0], n_head, 7, hp, cos, sin))
    # a host position past the cache is rejected before any launch
    assert lib.aq_rope_kv(P(qd), P(kd), P(vd), T, n_head, n_kv, hd, n_rot, 0, P(cd), P(sd),
                          None, n_ctx - 2, n_ctx, P(kc), P(vc), None) == _lib.AQ_ERR_VALUE


@pytest.mark.parametrize("n_head,n_kv,hd", [(32, 8, 64), (8, 8, 64), (16, 8, 64), (16, 2, 64),
                                            (8, 2, 128), (4, 4, 128), (16, 2, 128)])
@pytest.mark.parametrize("pos", [0, 1, 63, 64, 65, 1000, 2303])
def test_attention(n_head, n_kv, hd, pos):
    print(f"attention {n_head}/{n_kv} hd={hd} pos={pos}", flush=True)
    hp = _hp("norm", n_head, n_kv, hd, hd)
    n_ctx = 2304
    rng = np.random.default_rng(pos * 7 + hd + n_head)
    q = (rng.standard_normal(n_head * hd) * 2).astype(np.float32)
    K = rng.standard_normal((n_ctx, n_kv, hd)).astype(np.float32)
    V = rng.standard_normal((n_ctx, n_kv, hd)).astype(np.float32)
    d = dev()
    kc = torch.from_numpy(np.ascontiguousarray(K.transpose(1, 0, 2))).to(d)
    vc = torch.from_numpy(np.ascontiguousarray(V.transpose(1, 0, 2))).to(d)
    qd = torch.from_numpy(q).to(d)
    out = torch.empty(n_head * hd, device=d)
    lib = _lib.load()
    _lib.check(lib.aq_attention(P(qd), P(kc), P(vc), n_head, n_kv, hd, n_ctx, None, pos,
                                P(out), None))
    ref = MR.attention_np(q, K[:pos + 1], V[:pos + 1], hp, n_head // n_kv, 1.0 / math.sqrt(hd))
    got = out.cpu().numpy().reshape(n_head, hd)
    assert np.abs(got - ref).max() < 2e-6 * np.abs(V).max()
    st = state_tensor(pos=pos)
    out2 = torch.empty_like(out)
    _lib.check(lib.aq_attention(P(qd), P(kc), P(vc), n_head, n_kv, hd, n_ctx, P(st), 0,
                                P(out2), None))
    assert torch.equal(out, out2)


def test_attention_rejects_unsupported():
    lib = _lib.load()
    d = dev()
    t = torch.zeros(64 * 64 * 12, device=d)
    assert lib.aq_attention(P(t), P(t), P(t), 12, 4, 32, 16, None, 0, P(t), None) == \
        _lib.AQ_ERR_VALUE
    assert lib.aq_attention(P(t), P(t), P(t), 12, 5, 64, 16, None, 0, P(t), None) == \
        _lib.AQ_ERR_VALUE
    assert lib.aq_attention(P(t), P(t), P(t), 4, 4, 64, 16, None, 16, P(t), None) == \
        _lib.AQ_ERR_VALUE


def test_swiglu_and_add():
    rng = np.random.default_rng(9)
    n = 8192 + 17
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    g[:4] = [-100.0, 100.0, 0.0, -0.0]
    u = rng.standard_normal(n).astype(np.float32)
    d = dev()
    gd, ud = torch.from_numpy(g).to(d), torch.from_numpy(u).to(d)
    out = torch.empty_like(gd)
    lib = _lib.load()
    _lib.check(lib.aq_swiglu(P(gd), P(ud), n, P(out), None))
    with np.errstate(over="ignore"):
        ref = g / (np.float32(1.0) + np.exp(-g)) * u
    got = out.cpu().numpy()
    assert np.all(np.abs(got - ref) <= 4 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-30)
    # the interleaved form: (gate, up) pairs of one product, the same bits
    gu = torch.from_numpy(np.stack([g, u], axis=1).reshape(-1).copy()).to(d)
    pairs = torch.empty_like(gd)
    _lib.check(lib.aq_swiglu_pairs(P(gu), n, P(pairs), None))
    assert torch.equal(pairs, out)
    assert lib.aq_swiglu_pairs(None, 4, P(pairs), None) == _lib.AQ_ERR_VALUE
    x = torch.from_numpy(g.copy()).to(d)
    _lib.check(lib.aq_add(P(x), P(ud), n, None))
    assert np.array_equal(x.cpu().numpy(), g + u)


def test_greedy_argmax_and_prompt_feed():
    d = dev()
    lib = _lib.load()
    rng = np.random.default_rng(11)
    n = 128256
    logits = rng.standard_normal(n).astype(np.float32) - 50
    logits[[7, 90000, 128255]] = -1.0  # tie at the max: the first index wins
    hist = torch.full((4,), -1, dtype=torch.int64, device=d)
    st = state_tensor(token=3, pos=10)
    ld = torch.from_numpy(logits).to(d)
    _lib.check(lib.aq_greedy_advance(P(ld), n, P(st), None, 0, P(hist), 4, 1, None))
    s = read_state(st)
    assert s == {"token": 7, "key": 0, "pos": 11, "fed": 0, "count": 1}
    assert hist.cpu().tolist() == [7, -1, -1, -1]
    neg = -np.abs(logits) - 1
    neg[123456] = -0.5
    _lib.check(lib.aq_greedy_advance(P(torch.from_numpy(neg).to(d)), n, P(st), None, 0,
                                     P(hist), 4, 1, None))
    assert read_state(st)["token"] == 123456 and hist.cpu().tolist()[:2] == [7, 123456]
    _lib.check(lib.aq_greedy_advance(P(ld), n, P(st), None, 0, P(hist), 4, 0, None))
    s = read_state(st)  # no argmax: only the position moves
    assert s["token"] == 123456 and s["pos"] == 13 and s["count"] == 2
    # while prompt tokens are left they are fed, with or without an argmax
    prompt = torch.tensor([5, 6], dtype=torch.int64, device=d)
    _lib.check(lib.aq_greedy_advance(P(ld), n, P(st), P(prompt), 2, P(hist), 4, 0, None))
    assert read_state(st)["token"] == 5
    _lib.check(lib.aq_greedy_advance(P(ld), n, P(st), P(prompt), 2, P(hist), 4, 1, None))
    s = read_state(st)
    assert s["token"] == 6 and s["fed"] == 2 and s["count"] == 2 and s["pos"] == 15
    _lib.check(lib.aq_greedy_advance(P(ld), n, P(st), P(prompt), 2, P(hist), 4, 1, None))
    s = read_state(st)  # prompt consumed: argmax again
    assert s["token"] == 7 and s["count"] == 3 and s["key"] == 0
    assert lib.aq_greedy_advance(P(ld), 0, P(st), None, 0, None, 0, 1, None) == _lib.AQ_ERR_VALUE


def _window(tokens, last_n, seen=None):
    """Device window of aq_greedy_advance_penalized: [count, ring...]."""
    w = np.zeros(1 + last_n, np.int64)
    for i, t in enumerate(tokens):
        w[1 + i % last_n] = t
    w[0] = len(tokens) if seen is None else seen
    return torch.from_numpy(w).to(dev())


def _penalized(logits, window, penalty, take=1, prompt=None, st=None):
    lib, d = _lib.load(), dev()
    st = state_tensor(token=3, pos=10) if st is None else st
    hist = torch.full((2,), -1, dtype=torch.int64, device=d)
    ld = torch.from_numpy(logits).to(d)
    _lib.check(lib.aq_greedy_advance_penalized(
        P(ld), len(logits), P(st), P(prompt) if prompt is not None else None,
        0 if prompt is None else prompt.numel(), P(hist), 2, P(window), window.numel() - 1,
        ctypes.c_double(penalty), take, None))
    return read_state(st), hist.cpu().tolist(), window.cpu().tolist()


@pytest.mark.parametrize("n", [100, 5000, 128256])
def test_greedy_advance_penalized_matches_oracle(n):
    """The device selection equals sample.py:36-45 (the oracle) on random
    logits and windows: the plain winner in the window, duplicates, several
    tokens in one 2048-logit slice, wrapped rings, negative logits, penalties
    below and above 1, and exact ties (penalty 2)."""
    from oracle.sample_ref import penalized_argmax
    print(f"penalized argmax n={n}", flush=True)
    rng = np.random.default_rng(n)
    for trial in range(24):
        logits = rng.standard_normal(n).astype(np.float32)
        if trial % 4 == 1:
            logits = -np.abs(logits) - 0.5          # every value negative
        if trial % 4 == 2:
            logits = np.round(logits * 4).astype(np.float32) / 4   # many ties
        last_n = int(rng.choice([1, 7, 64, 300]))
        k = int(rng.integers(0, 2 * last_n + 1))
        toks = [int(t) for t in rng.integers(0, n, k)]
        top = np.argsort(-logits.astype(np.float64), kind="stable")[:3]
        toks += [int(top[0])] * int(rng.integers(1, 3)) + [int(top[1])]
        toks += [int(top[0]) + 1] if top[0] + 1 < n else []   # same slice as the winner
        penalty = float(rng.choice([1.1, 2.0, 0.9, 1.5]))
        recent = toks[-last_n:]
        want = penalized_argmax(logits, recent, penalty)
        s, hist, w = _penalized(logits, _window(toks, last_n), penalty)
        assert s["token"] == want and hist[0] == want, (trial, last_n, penalty)
        assert s["count"] == 1 and s["pos"] == 11 and s["key"] == 0
        assert w[0] == len(toks) + 1 and w[1 + len(toks) % last_n] == want  # accepted


def test_greedy_advance_penalized_window_rules():
    d = dev()
    logits = np.zeros(3000, np.float32)
    logits[[10, 2500]] = 4.0
    logits[20] = 2.0
    # penalty 2 is exact: 10 -> 2.0 ties with 20, the lower index wins
    assert _penalized(logits, _window([10, 2500], 4), 2.0)[0]["token"] == 10
    assert _penalized(logits, _window([2500], 4), 2.0)[0]["token"] == 10
    assert _penalized(logits, _window([10], 4), 2.0)[0]["token"] == 2500
    # penalty 1 or 0: plain argmax, the window still accepts the token
    for p in (1.0, 0.0):
        s, _, w = _penalized(logits, _window([10, 2500], 4), p)
        assert s["token"] == 10 and w[:4] == [3, 10, 2500, 10]
    # only the last min(count, last_n) ring entries count; a count beyond
    # last_n means a full ring
    s, _, w = _penalized(logits, _window([10, 11, 12], 3, seen=1), 2.0)
    assert s["token"] == 2500 and w[0] == 2 and w[2] == 2500
    s, _, w = _penalized(logits, _window([2500, 11, 10], 3, seen=1000), 4.0)
    assert s["token"] == 20 and w[0] == 1001 and w[1 + 1000 % 3] == 20  # 4/4 < 2
    # entries outside [0, n) are skipped
    assert _penalized(logits, _window([-5, 3000, 10], 4), 2.0)[0]["token"] == 2500
    # every logit in the window
    small = np.array([-1.0, 3.0], np.float32)
    assert _penalized(small, _window([1, 0], 2), 1.1)[0]["token"] == 1
    assert _penalized(small, _window([1, 0], 2), 0.1)[0]["token"] == 1  # -0.1 < 30
    # prompt tokens fed by the call are accepted too; no argmax while fed
    prompt = torch.tensor([7, 8], dtype=torch.int64, device=d)
    st = state_tensor(token=3, pos=0)
    w = _window([3], 4)
    for want in (7, 8):
        s, _, wl = _penalized(logits, w, 2.0, take=1, prompt=prompt, st=st)
        assert s["token"] == want
    assert wl[:4] == [3, 3, 7, 8] and s["count"] == 0 and s["fed"] == 2
    lib = _lib.load()
    ld = torch.from_numpy(logits).to(d)
    for last_n, pen in ((0, 1.1), (4, float("nan")), (4, float("inf"))):
        assert lib.aq_greedy_advance_penalized(
            P(ld), 3000, P(st), None, 0, None, 0, P(w), last_n, ctypes.c_double(pen), 1,
            None) == _lib.AQ_ERR_VALUE
    assert lib.aq_greedy_advance_penalized(P(ld), 3000, P(st), None, 0, None, 0, None, 4,
                                           ctypes.c_double(1.1), 1, None) == _lib.AQ_ERR_VALUE


@pytest.mark.parametrize("style,n_head,n_kv,hd,n_rot",
                         [("norm", 32, 8, 64, 64), ("neox", 16, 2, 128, 128),
                          ("norm", 8, 8, 64, 40), ("neox", 8, 4, 64, 48)])
@pytest.mark.parametrize("pos", [0, 63, 64, 1500, 2303])
def test_attention_rope_fused_equals_separate(style, n_head, n_kv, hd, n_rot, pos):
    """aq_attention_rope == aq_rope_kv + aq_attention, bit for bit (output and
    cache), and against the oracle."""
    print(f"attention_rope {style} {n_head}/{n_kv} hd={hd} n_rot={n_rot} pos={pos}", flush=True)
    hp = _hp(style, n_head, n_kv, hd, n_rot)
    n_ctx = 2304
    cos, sin = MR.rope_tables(hp, n_ctx)
    rng = np.random.default_rng(pos + hd + n_rot)
    K = rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float32)
    V = rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float32)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    d = dev()
    cd, sd = torch.from_numpy(cos).to(d), torch.from_numpy(sin).to(d)
    lib = _lib.load()
    neox = 1 if style == "neox" else 0
    outs, caches = [], []
    for fused in (True, False):
        kc, vc = torch.from_numpy(K).to(d), torch.from_numpy(V).to(d)
        qd, kd, vd = (torch.from_numpy(a.copy()).to(d) for a in (q, k, v))
        out = torch.empty(n_head * hd, device=d)
        st = state_tensor(pos=pos)
        if fused:
            _lib.check(lib.aq_attention_rope(P(qd), P(kd), P(vd), n_head, n_kv, hd, n_rot,
                                             neox, P(cd), P(sd), P(st), 0, n_ctx, P(kc), P(vc),
                                             P(out), None))
            assert torch.equal(qd, torch.from_numpy(q).to(d))  # q is not modified
        else:
            _lib.check(lib.aq_rope_kv(P(qd), P(kd), P(vd), 1, n_head, n_kv, hd, n_rot, neox,
                                      P(cd), P(sd), P(st), 0, n_ctx, P(kc), P(vc), None))
            _lib.check(lib.aq_attention(P(qd), P(kc), P(vc), n_head, n_kv, hd, n_ctx, P(st),
                                        0, P(out), None))
        outs.append(out.cpu().numpy())
        caches.append((kc.cpu().numpy(), vc.cpu().numpy()))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])
    kr = MR.rope_np(k, n_kv, pos, hp, cos, sin).reshape(n_kv, hd)
    assert np.array_equal(caches[0][0][:, pos], kr) and np.array_equal(caches[0][1][:, pos],
                                                                       v.reshape(n_kv, hd))
    Kr = caches[0][0].transpose(1, 0, 2)[:pos + 1]
    Vr = caches[0][1].transpose(1, 0, 2)[:pos + 1]
    qr = MR.rope_np(q, n_head, pos, hp, cos, sin)
    ref = MR.attention_np(qr, Kr, Vr, hp, n_head // n_kv, 1.0 / math.sqrt(hd))
    assert np.abs(outs[0].reshape(n_head, hd) - ref).max() < 2e-6 * np.abs(Vr).max()
    # repeated calls (the same position stored again, the workspace partials
    # reused) give the same bits
    kc, vc = torch.from_numpy(K).to(d), torch.from_numpy(V).to(d)
    qd, kd, vd = (torch.from_numpy(a.copy()).to(d) for a in (q, k, v))
    out = torch.empty(n_head * hd, device=d)
    for _ in range(3):
        _lib.check(lib.aq_attention_rope(P(qd), P(kd), P(vd), n_head, n_kv, hd, n_rot, neox,
                                         P(cd), P(sd), None, pos, n_ctx, P(kc), P(vc), P(out),
                                         None))
        assert np.array_equal(out.cpu().numpy(), outs[0])


@pytest.fixture(scope="module")
def tiny():
    hp, tensors = synthetic_llama_1b(seed=7, n_layer=2, n_embd=256, n_head=4, n_kv=2,
                                     n_ff=512, n_vocab=1000, n_ctx_train=512)
    return hp, tensors


def test_tiny_model_forward_logits(tiny):
    print("tiny model forward", flush=True)
    hp, tensors = tiny
    gm, rm = Model(hp, tensors), MR.RefModel(hp, tensors)
    for t in (3, 999, 0, 512, 77, 77):
        a, b = gm.forward(t), rm.forward(t)
        assert np.abs(a - b).max() < 1e-4 * np.abs(b).max(), t
    # prefill with prefix reuse, then continue
    toks = [3, 999, 0, 512, 77, 77, 5, 6, 7]
    a, b = gm.prefill(toks), None
    rm.reset()
    b = rm.prefill(toks)
    assert gm.n_past == 9 and np.abs(a - b).max() < 1e-4 * np.abs(b).max()


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("batch_prefill", [True, False])
def test_tiny_model_greedy_tokens(tiny, graph, batch_prefill):
    print(f"tiny model greedy graph={graph} batch_prefill={batch_prefill}", flush=True)
    hp, tensors = tiny
    prompt = list(np.random.default_rng(1).integers(0, hp.n_vocab, 100))
    ref, margins = MR.RefModel(hp, tensors).greedy(prompt, 40)
    gm = Model(hp, tensors)
    gm.prefill_chunk = 48  # several chunks, the last one ragged
    got = gm.generate_greedy(prompt, 40, graph=graph, batch_prefill=batch_prefill)
    assert got == ref, (got, ref, margins)
    # the graph replays leave the model where forward() can continue
    assert gm.n_past == 139
    got2 = gm.generate_greedy(prompt[:50], 8, graph=graph, batch_prefill=batch_prefill)
    assert got2 == MR.RefModel(hp, tensors).greedy(prompt[:50], 8)[0]


@pytest.mark.parametrize("per_graph", [1, 5, 39, 40])
def test_tiny_model_greedy_steps_per_graph(tiny, per_graph):
    """Replays of a graph of several decode steps give the tokens of one step
    per replay: 39 steps after the first token run as 7 x 5 + 4, 1 x 39, and
    39 single replays where the multi-step graph would be longer than the
    run (40)."""
    print(f"tiny model greedy steps_per_graph={per_graph}", flush=True)
    hp, tensors = tiny
    prompt = list(np.random.default_rng(2).integers(0, hp.n_vocab, 60))
    ref, margins = MR.RefModel(hp, tensors).greedy(prompt, 40)
    gm = Model(hp, tensors)
    timing = {}
    got = gm.generate_greedy(prompt, 40, steps_per_graph=per_graph, timing=timing)
    assert got == ref, (got, ref, margins)
    assert gm.n_past == 99
    # and the model continues from there like after single-step replays
    got2 = gm.generate_greedy(prompt[:30], 12, steps_per_graph=per_graph)
    assert got2 == MR.RefModel(hp, tensors).greedy(prompt[:30], 12)[0]


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("penalty,last_n", [(1.1, 64), (1.1, 8)])
def test_tiny_model_greedy_repeat_penalty(tiny, graph, penalty, last_n):
    """The decode loop of tests/bench.py:78-90 (temperature-0 Sampler with
    the repetition penalty) on the device equals the oracle's; the penalty
    changes the tokens of this model."""
    print(f"tiny model penalized greedy graph={graph} {penalty}/{last_n}", flush=True)
    hp, tensors = tiny
    prompt = list(np.random.default_rng(1).integers(0, hp.n_vocab, 100))
    ref, margins = MR.RefModel(hp, tensors).greedy(prompt, 40, repeat_penalty=penalty,
                                                   repeat_last_n=last_n)
    assert ref != MR.RefModel(hp, tensors).greedy(prompt, 40)[0]
    gm = Model(hp, tensors)
    got = gm.generate_greedy(prompt, 40, graph=graph, repeat_penalty=penalty,
                             repeat_last_n=last_n)
    assert got == ref, (got, ref, margins)
    assert gm.generate_greedy(prompt, 40, graph=graph) == MR.RefModel(hp, tensors).greedy(
        prompt, 40)[0]


def test_prefill_chunk_size_does_not_change_results(tiny):
    """Logits and KV cache of the batched step are bit-identical for any
    chunk size (ragged last chunks included), so the device default (2048)
    computes exactly what the reference's 256 would."""
    hp, tensors = tiny
    toks = list(np.random.default_rng(4).integers(0, hp.n_vocab, 150))
    out = []
    for chunk in (150, 64, 37, 7):
        gm = Model(hp, tensors)
        gm.prefill_chunk = chunk
        out.append((gm.prefill(toks), gm.kv[:, :, :, :150].cpu().numpy()))
    for lg, kv in out[1:]:
        assert np.array_equal(lg, out[0][0]) and np.array_equal(kv, out[0][1])


@pytest.fixture(scope="module")
def tiny_qwen2():
    """A qwen2-style model: neox RoPE and q/k/v biases (model.py:22-29,
    :308-310)."""
    import dataclasses

    from alpacca_amd.model import Tensor
    hp, tensors = synthetic_llama_1b(seed=11, n_layer=2, n_embd=256, n_head=4, n_kv=2,
                                     n_ff=512, n_vocab=1000, n_ctx_train=512, std=0.05)
    hp = dataclasses.replace(hp, arch="qwen2", rope_style="neox", rope_base=1000000.0)
    rng = np.random.default_rng(12)
    q_dim, kv_dim = hp.n_head * hp.head_dim, hp.n_kv * hp.head_dim
    for i in range(hp.n_layer):
        for role, n in (("attn_q", q_dim), ("attn_k", kv_dim), ("attn_v", kv_dim)):
            tensors[f"blk.{i}.{role}.bias"] = Tensor(
                "F32", (n,), (rng.standard_normal(n) * 0.5).astype(np.float32))
    return hp, tensors


@pytest.mark.parametrize("fused", [True, False])
def test_qwen2_style_model(tiny_qwen2, fused):
    """q/k/v biases and neox RoPE through the device Model (model.py:308-310,
    :491-496, :532-537): greedy tokens equal the oracle's, and the batched
    prefill (one bias launch per projection) and the decode step stay within
    1e-4 of the oracle's logits."""
    print(f"qwen2-style model fused={fused}", flush=True)
    hp, tensors = tiny_qwen2
    prompt = list(np.random.default_rng(2).integers(0, hp.n_vocab, 100))
    ref, margins = MR.RefModel(hp, tensors).greedy(prompt, 30)
    gm = Model(hp, tensors, fused=fused)
    gm.prefill_chunk = 48
    got = gm.generate_greedy(prompt, 30)
    assert got == ref, (got, ref, margins)
    toks = list(np.random.default_rng(3).integers(0, hp.n_vocab, 130))
    want = MR.RefModel(hp, tensors).prefill(toks)
    scale = np.abs(want).max()
    a = Model(hp, tensors, fused=fused).prefill(toks)
    assert np.abs(a - want).max() < 1e-4 * scale
    c = Model(hp, tensors, fused=fused).prefill(toks, batch=False)
    assert np.abs(c - want).max() < 1e-4 * scale


class _DropIn:
    """The seam of the reference model (tensor.py:82-113) with its matrices
    swapped for QuantMatrix, as the integration notes swap them: the oracle's
    model code then calls matvec / matmul_t / row / rows_at of the device
    matrices with its own host arrays and default arguments."""

    def __init__(self, t):
        from alpacca_amd.qmatrix import QuantMatrix
        self.rows, self.cols = t.shape
        self.q = QuantMatrix(t.data, t.dtype, self.rows, self.cols)

    def matvec(self, x):
        return self.q.matvec(x)

    def matmul_t(self, X):
        return self.q.matmul_t(X)

    def row(self, i):
        return self.q.row(i)

    def rows_at(self, idx):
        return self.q.rows_at(idx)


def _drop_in_model(hp, tensors):
    m = MR.RefModel(hp, tensors, fast=False)
    m.tok_embd = _DropIn(tensors["token_embd.weight"])
    for i, ly in enumerate(m.layers):
        for role in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                     "ffn_down"):
            ly[role] = _DropIn(tensors[f"blk.{i}.{role}.weight"])
    m.output = _DropIn(tensors["output.weight"]) if "output.weight" in tensors else m.tok_embd
    return m


def test_drop_in_reference_prefill_keeps_fp32_bar(tiny):
    """The reference's prefill (forward_batch in chunks of 256,
    model.py:610-641) over 130 tokens with QuantMatrix behind the seam: the
    default matmul_t keeps float32 products, so the logits stay within the
    reference's own batched-vs-sequential bar (1e-4, tests/smoke.py:950-972)
    of the oracle's and of the same model run token by token."""
    hp, tensors = tiny
    toks = list(np.random.default_rng(13).integers(0, hp.n_vocab, 130))
    want = MR.RefModel(hp, tensors).prefill(toks)
    dm = _drop_in_model(hp, tensors)
    got = dm.prefill(toks)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() < 1e-4 * scale
    dm.reset()
    seq = None
    for t in toks:
        seq = dm.forward(int(t))
    assert np.abs(got - seq).max() < 1e-4 * scale


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_tiny_model_batched_prefill(tiny, precision):
    """The batched step (forward_batch) against the oracle's, and against the
    decode step run token by token (the reference's own bar, 1e-4,
    tests/smoke.py:950-972, for the fp32 products; bf16 MFMA within 1e-2)."""
    hp, tensors = tiny
    toks = list(np.random.default_rng(3).integers(0, hp.n_vocab, 130))
    gm = Model(hp, tensors)
    gm.prefill_chunk = 64
    gm.prefill_precision = precision
    a = gm.prefill(toks)
    rm = MR.RefModel(hp, tensors)
    b = rm.prefill(toks, chunk=64)
    tol = 1e-4 if precision == "fp32" else 1e-2
    assert np.abs(a - b).max() < tol * np.abs(b).max()
    gs = Model(hp, tensors)
    c = gs.prefill(toks, batch=False)
    assert np.abs(a - c).max() < tol * np.abs(c).max()
    # the KV caches agree too
    kv_a, kv_c = gm.kv[:, :, :, :130].cpu().numpy(), gs.kv[:, :, :, :130].cpu().numpy()
    assert np.abs(kv_a - kv_c).max() < tol * np.abs(kv_c).max()
    # prefix reuse: the same prompt plus 5 tokens runs only the 5
    more = toks + [1, 2, 3, 4, 5]
    d = gm.prefill(more)
    assert gm.n_past == 135
    rm.reset()
    e = rm.prefill(more, chunk=64)
    assert np.abs(d - e).max() < tol * np.abs(e).max()


@pytest.mark.parametrize("n_head,n_kv,hd", [(32, 8, 64), (8, 2, 128), (4, 4, 64),
                                            (16, 2, 64), (4, 2, 128)])
@pytest.mark.parametrize("pos0,T", [(0, 1), (0, 70), (100, 256), (2000, 17), (0, 2304)])
@pytest.mark.parametrize("path", ["prefill", "prefill_valu", "chunked"])
def test_attention_batch_causal(n_head, n_kv, hd, pos0, T, path, monkeypatch):
    """T > 1 runs the one-launch prefill kernel (online softmax over the
    chunks; on fp32 matrix cores, or on the VALU with AQ_ATTN_PREFILL_VALU)
    unless AQ_ATTN_CHUNKED selects the decode kernels (partials per 64-position
    chunk, then the combine); all against the oracle."""
    if path == "chunked":
        monkeypatch.setenv("AQ_ATTN_CHUNKED", "1")
    if path == "prefill_valu":
        monkeypatch.setenv("AQ_ATTN_PREFILL_VALU", "1")
    print(f"attention batch {n_head}/{n_kv} hd={hd} pos0={pos0} T={T} {path}", flush=True)
    hp = _hp("norm", n_head, n_kv, hd, hd)
    n_ctx = 2304
    rng = np.random.default_rng(pos0 + T + hd)
    q = rng.standard_normal((T, n_head * hd)).astype(np.float32)
    K = rng.standard_normal((n_ctx, n_kv, hd)).astype(np.float32)
    V = rng.standard_normal((n_ctx, n_kv, hd)).astype(np.float32)
    d = dev()
    kc = torch.from_numpy(np.ascontiguousarray(K.transpose(1, 0, 2))).to(d)
    vc = torch.from_numpy(np.ascontiguousarray(V.transpose(1, 0, 2))).to(d)
    qd = torch.from_numpy(q).to(d)
    out = torch.empty((T, n_head * hd), device=d)
    lib = _lib.load()
    _lib.check(lib.aq_attention_batch(P(qd), P(kc), P(vc), T, n_head, n_kv, hd, n_ctx, None,
                                      pos0, P(out), None))
    pos = np.arange(pos0, pos0 + T, dtype=np.int32)
    ref = MR.attention_batch_np(q, K[:pos0 + T], V[:pos0 + T], pos, hp, n_head // n_kv,
                                1.0 / math.sqrt(hd))
    assert np.abs(out.cpu().numpy() - ref).max() < 2e-6 * np.abs(V).max()
    assert lib.aq_attention_batch(P(qd), P(kc), P(vc), T, n_head, n_kv, hd, n_ctx, None,
                                  n_ctx - T + 1, P(out), None) == _lib.AQ_ERR_VALUE


@pytest.mark.parametrize("n_head,n_kv,hd", [(32, 8, 64), (8, 2, 128)])
def test_attention_combine_forms_agree(n_head, n_kv, hd, monkeypatch):
    """The combine merges the per-chunk partials from registers when a call
    has at most 32 partial slots and through LDS tiles above that; the two
    forms run the same operations in the same order, so a cache whose chunk
    count selects either gives the same bits for positions both hold."""
    monkeypatch.setenv("AQ_ATTN_CHUNKED", "1")
    ch = 64 if hd == 64 else 32  # positions per chunk
    small, large = 32 * ch, 64 * ch  # 32 slots (registers), 64 (LDS tiles)
    T, pos0 = 7, small - 40
    print(f"combine forms {n_head}/{n_kv} hd={hd} caches {small}/{large}", flush=True)
    rng = np.random.default_rng(hd + n_head)
    q = rng.standard_normal((T, n_head * hd)).astype(np.float32)
    K = rng.standard_normal((n_kv, large, hd)).astype(np.float32)
    V = rng.standard_normal((n_kv, large, hd)).astype(np.float32)
    d = dev()
    lib = _lib.load()
    qd = torch.from_numpy(q).to(d)
    outs = []
    for n_ctx in (small, large):
        kc = torch.from_numpy(np.ascontiguousarray(K[:, :n_ctx])).to(d)
        vc = torch.from_numpy(np.ascontiguousarray(V[:, :n_ctx])).to(d)
        out = torch.empty((T, n_head * hd), device=d)
        _lib.check(lib.aq_attention_batch(P(qd), P(kc), P(vc), T, n_head, n_kv, hd, n_ctx,
                                          None, pos0, P(out), None))
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])


# ---------------------------------------------------------- fused matvecs ---

FUSED_CASES = [("Q4_K", 2048, 512), ("Q4_K", 4096, 1024), ("Q6_K", 8192, 300),
               ("Q8_0", 14336, 257), ("Q5_K", 2048, 64), ("Q4_0", 1024, 100)]


@pytest.mark.parametrize("dtype,cols,rows", FUSED_CASES)
@pytest.mark.parametrize("mode", ["rmsnorm", "swiglu"])
def test_matvec_fused(dtype, cols, rows, mode):
    """aq_matvec_fused against the oracle's composition: x_eff from the
    reference's NumPy expressions, float64 product over the exact decode,
    2e-5 of ||W_r|| * ||x_eff||; the residual is added on top."""
    from alpacca_amd import synth
    from alpacca_amd.qmatrix import QuantMatrix, matvec_fused_device
    from oracle.qmatrix_ref import RefMatrix, normalized_error
    print(f"fused {mode} {dtype} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(cols + rows)
    datas = [synth.random_matrix_bytes(dtype, rows + 7 * i, cols, seed=i) for i in range(2)]
    qms = [QuantMatrix(dd, dtype, rows + 7 * i, cols) for i, dd in enumerate(datas)]
    refs = [RefMatrix(dd, dtype, rows + 7 * i, cols) for i, dd in enumerate(datas)]
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    x2 = rng.standard_normal(cols).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    if mode == "rmsnorm":
        xe = MR.rmsnorm(x, nw, 1e-5)
    else:
        with np.errstate(over="ignore"):
            xe = x / (np.float32(1.0) + np.exp(-x)) * x2
    d = dev()
    xd, x2d, nwd = (torch.from_numpy(a).to(d) for a in (x, x2, nw))
    y0 = [rng.standard_normal(q.rows).astype(np.float32) for q in qms]
    for accumulate in (False, True):
        ys = [torch.from_numpy(a.copy()).to(d) for a in y0]
        matvec_fused_device(qms, xd.data_ptr(), [y.data_ptr() for y in ys], 0,
                            x2_ptr=x2d.data_ptr(), norm_w_ptr=nwd.data_ptr(), eps=1e-5,
                            rmsnorm=mode == "rmsnorm", swiglu=mode == "swiglu",
                            accumulate=accumulate)
        torch.cuda.synchronize()
        for y, ref, base in zip(ys, refs, y0):
            want = ref.matvec_f64(xe) + (base.astype(np.float64) if accumulate else 0.0)
            got = y.cpu().numpy().astype(np.float64)
            assert normalized_error(got, want, ref.row_norms(), xe) < 2e-5


def test_matvec_fused_rejects_bad_flags():
    from alpacca_amd import synth
    from alpacca_amd.qmatrix import QuantMatrix
    qm = QuantMatrix(synth.random_matrix_bytes("Q4_K", 8, 256, 1), "Q4_K", 8, 256)
    lib = _lib.load()
    x = torch.zeros(256, device=dev())
    y = torch.zeros(8, device=dev())
    hs = (ctypes.c_void_p * 1)(qm.handle)
    yp = (ctypes.c_void_p * 1)(y.data_ptr())
    io = _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE
    both = io | _lib.AQ_X_RMSNORM | _lib.AQ_X_SWIGLU
    assert lib.aq_matvec_fused(hs, 1, P(x), P(x), P(x), ctypes.c_float(0), yp, both,
                               None) == _lib.AQ_ERR_VALUE
    assert lib.aq_matvec_fused(hs, 1, P(x), None, None, ctypes.c_float(0), yp,
                               io | _lib.AQ_X_RMSNORM, None) == _lib.AQ_ERR_VALUE
    assert lib.aq_matvec_fused(hs, 1, P(x), None, None, ctypes.c_float(0), yp,
                               _lib.AQ_X_SWIGLU, None) == _lib.AQ_ERR_VALUE


@pytest.mark.parametrize("dtype,cols", [("Q4_K", 2048), ("Q6_K", 512), ("Q8_0", 1024),
                                        ("Q4_0", 96)])
def test_matvec_swiglu_pairs(dtype, cols):
    """Interleaved gate/up rows with AQ_Y_SWIGLU_PAIRS: each output is
    silu(gate) * up of the same launch's two rows, bit-identical to the
    separate gate/up outputs combined by aq_swiglu (the same fp32 ops), with
    and without RMSNorm staging and accumulation."""
    from alpacca_amd import synth
    from alpacca_amd.qmatrix import (QuantMatrix, interleave_rows, matvec_fused_device,
                                     pair_rows_supported)
    n = 300
    assert pair_rows_supported(dtype, cols)
    g = synth.random_matrix_bytes(dtype, n, cols, seed=1)
    u = synth.random_matrix_bytes(dtype, n, cols, seed=2)
    G, U = QuantMatrix(g, dtype, n, cols), QuantMatrix(u, dtype, n, cols)
    GU = QuantMatrix(interleave_rows(g, u, n, cols, dtype), dtype, 2 * n, cols)
    d = dev()
    rng = np.random.default_rng(cols)
    x = torch.from_numpy((rng.standard_normal(cols) * 2).astype(np.float32)).to(d)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, cols).astype(np.float32)).to(d)
    base = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(d)
    lib = _lib.load()
    for rmsnorm in (False, True):
        yg, yu, ref = (torch.empty(n, device=d) for _ in range(3))
        matvec_fused_device([G, U], x.data_ptr(), [yg.data_ptr(), yu.data_ptr()], 0,
                            norm_w_ptr=nw.data_ptr(), eps=1e-5, rmsnorm=rmsnorm)
        _lib.check(lib.aq_swiglu(P(yg), P(yu), n, P(ref), None))
        for acc in (False, True):
            y = base.clone()
            matvec_fused_device([GU], x.data_ptr(), [y.data_ptr()], 0, norm_w_ptr=nw.data_ptr(),
                                eps=1e-5, rmsnorm=rmsnorm, swiglu_pairs=True, accumulate=acc)
            torch.cuda.synchronize()
            want = (base + ref) if acc else ref
            assert torch.equal(y, want), (rmsnorm, acc)
    # refused: odd rows, rows too wide for pairs, two dtypes
    odd = QuantMatrix(synth.random_matrix_bytes(dtype, 3, cols, seed=3), dtype, 3, cols)
    y = torch.empty(2, device=d)
    with pytest.raises(ValueError, match="even row count"):
        matvec_fused_device([odd], x.data_ptr(), [y.data_ptr()], 0, swiglu_pairs=True)
    wide = QuantMatrix(synth.random_matrix_bytes("Q4_K", 2, 4096, seed=4), "Q4_K", 2, 4096)
    xw = torch.zeros(4096, device=d)
    assert not pair_rows_supported("Q4_K", 4096)
    with pytest.raises(ValueError, match="32 lane units"):
        matvec_fused_device([wide], xw.data_ptr(), [y.data_ptr()], 0, swiglu_pairs=True)


def test_tiny_model_unfused_matches_fused(tiny):
    hp, tensors = tiny
    prompt = list(np.random.default_rng(2).integers(0, hp.n_vocab, 30))
    a = Model(hp, tensors, fused=True).generate_greedy(prompt, 12)
    b = Model(hp, tensors, fused=False).generate_greedy(prompt, 12)
    assert a == b == MR.RefModel(hp, tensors).greedy(prompt, 12)[0]
