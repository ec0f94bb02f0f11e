"""GPU test of aq_attention_rope_noalloc: the decode attention (RoPE, KV store,
partials, combine) with its partials in the library's static device scratch
instead of allocated memory.  Its output and cache writes must be the same
bits as aq_attention_rope's (the same kernels) on two calls in a row, the
second with a smaller cache and position, with the position given on the
host and in a device-resident decode state, eagerly and replayed from a HIP
graph; sizes past the scratch are refused before anything is launched."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from alpacca_amd import _lib
from alpacca_amd.model import Hyperparams, rope_tables

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _noalloc(lib):
    return lib.aq_attention_rope_noalloc


def P(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _state(pos):
    st = np.zeros(8, np.int32)
    st[4] = pos
    return torch.from_numpy(st).cuda()


@pytest.mark.parametrize("n_head,n_kv,hd,neox", [(32, 8, 64, 0), (8, 2, 128, 1)])
def test_noalloc_attention_equals_allocating_entry(n_head, n_kv, hd, neox):
    lib = _lib.ensure_device()
    noalloc = _noalloc(lib)
    # two calls in a row: the second with a smaller cache and an earlier position
    for n_ctx, pos, use_state in ((2304, 1500, False), (640, 100, True)):
        print(f"noalloc attention n_head={n_head} n_kv={n_kv} hd={hd} n_ctx={n_ctx} "
              f"pos={pos} state={use_state}", flush=True)
        hp = Hyperparams(arch="llama", n_layer=1, n_embd=n_head * hd, n_head=n_head,
                         n_kv=n_kv, n_ff=64, n_vocab=64, n_ctx_train=n_ctx, head_dim=hd,
                         n_rot=hd, rms_eps=1e-5, rope_base=500000.0,
                         rope_style="neox" if neox else "norm")
        cos, sin = (torch.from_numpy(np.ascontiguousarray(t)).cuda() for t in rope_tables(hp, n_ctx))
        rng = np.random.default_rng(n_ctx + pos)
        q = torch.from_numpy(rng.standard_normal(n_head * hd).astype(np.float32)).cuda()
        k = torch.from_numpy(rng.standard_normal(n_kv * hd).astype(np.float32)).cuda()
        v = torch.from_numpy(rng.standard_normal(n_kv * hd).astype(np.float32)).cuda()
        kc = torch.from_numpy(rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float32)).cuda()
        vc = torch.from_numpy(rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float32)).cuda()
        st = _state(pos) if use_state else None
        p0 = 0 if use_state else pos
        outs = []
        for fn in (lib.aq_attention_rope, noalloc):
            kcc, vcc = kc.clone(), vc.clone()
            out = torch.full((n_head * hd,), float("nan"), device="cuda")
            _lib.check(fn(P(q), P(k), P(v), n_head, n_kv, hd, hd, neox, P(cos), P(sin), P(st),
                          p0, n_ctx, P(kcc), P(vcc), P(out), None))
            torch.cuda.synchronize()
            outs.append((out.cpu().numpy(), kcc.cpu().numpy(), vcc.cpu().numpy()))
        for a, b in zip(*outs):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.isfinite(outs[1][0]).all()


def test_noalloc_attention_graph_replays():
    """Captured in a HIP graph and replayed, with eager work on the same
    scratch between the replays, every replay gives the eager result."""
    lib = _lib.ensure_device()
    noalloc = _noalloc(lib)
    n_head, n_kv, hd, n_ctx, pos = 32, 8, 64, 1024, 700
    hp = Hyperparams(arch="llama", n_layer=1, n_embd=n_head * hd, n_head=n_head, n_kv=n_kv,
                     n_ff=64, n_vocab=64, n_ctx_train=n_ctx, head_dim=hd, n_rot=hd,
                     rms_eps=1e-5, rope_base=500000.0, rope_style="norm")
    cos, sin = (torch.from_numpy(np.ascontiguousarray(t)).cuda() for t in rope_tables(hp, n_ctx))
    rng = np.random.default_rng(9)
    q, k, v = (torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
               for n in (n_head * hd, n_kv * hd, n_kv * hd))
    kc = torch.from_numpy(rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float32)).cuda()
    vc = torch.from_numpy(rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float32)).cuda()
    kc2, vc2 = kc.clone(), vc.clone()  # caches of the eager calls between replays
    st = _state(pos)
    out = torch.empty(n_head * hd, device="cuda")
    other = torch.empty(n_head * hd, device="cuda")
    s = torch.cuda.Stream()

    def call(o, p=0, state=st, caches=(kc, vc)):
        _lib.check(noalloc(P(q), P(k), P(v), n_head, n_kv, hd, hd, 0, P(cos), P(sin),
                           P(state), p, n_ctx, P(caches[0]), P(caches[1]), P(o),
                           ctypes.c_void_p(s.cuda_stream)))

    with torch.cuda.stream(s):
        call(out)
    torch.cuda.synchronize()
    want = out.cpu().numpy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(out)
    for i in range(4):
        with torch.cuda.stream(s):
            out.fill_(float("nan"))
            call(other, p=900 + i, state=None, caches=(kc2, vc2))  # the same scratch
            g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), i


def test_noalloc_attention_refuses_sizes_past_the_scratch():
    lib = _lib.ensure_device()
    noalloc = _noalloc(lib)
    dummy = torch.zeros(16, device="cuda")
    # 512 query heads x 32 splits x 132 floats = 8.25 MiB of partials: past the
    # scratch (the cache length does not matter past 32 chunks)
    n_ctx = 1 << 20
    rc = noalloc(P(dummy), P(dummy), P(dummy), 512, 64, 128, 128, 0, P(dummy), P(dummy), None,
                 0, n_ctx, P(dummy), P(dummy), P(dummy), None)
    assert rc == _lib.AQ_ERR_VALUE
    assert b"static scratch" in lib.aq_last_error()
