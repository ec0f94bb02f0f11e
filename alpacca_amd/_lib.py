"""ctypes binding of libalpacca_amd.so (declared in include/alpacca_amd.h).

The library is the only compute path: if it is not built, or no HIP device is
visible, the calls below raise instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_native" / "libalpacca_amd.so"

AQ_OK, AQ_ERR_VALUE, AQ_ERR_INDEX, AQ_ERR_RUNTIME = 0, 1, 2, 3
AQ_IN_DEVICE, AQ_OUT_DEVICE, AQ_MATVEC_FP32 = 1, 2, 4
AQ_X_RMSNORM, AQ_X_SWIGLU, AQ_Y_ACCUMULATE, AQ_Y_SWIGLU_PAIRS = 8, 16, 32, 64
AQ_PREC_AUTO, AQ_PREC_FP32, AQ_PREC_BF16, AQ_PREC_INT8 = 0, 1, 2, 3
AQ_LAYOUT_AUTO, AQ_LAYOUT_RAW, AQ_LAYOUT_SPLIT = 0, 1, 2

# ggml tensor type ids (GGUF), as used by the C ABI
DTYPE_IDS = {"Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8,
             "Q4_K": 12, "Q5_K": 13, "Q6_K": 14,
             "F32": 0, "F16": 1, "BF16": 30}  # the last three: dense matrices
LAYOUT_IDS = {"auto": AQ_LAYOUT_AUTO, "raw": AQ_LAYOUT_RAW, "split": AQ_LAYOUT_SPLIT}
PREC_IDS = {"auto": AQ_PREC_AUTO, "fp32": AQ_PREC_FP32, "bf16": AQ_PREC_BF16,
            "int8": AQ_PREC_INT8}

# every symbol include/alpacca_amd.h declares, with (restype, argtypes)
_c = ctypes
_vp, _i32, _i64, _sz = _c.c_void_p, _c.c_int, _c.c_int64, _c.c_size_t
SIGNATURES = {
    "aq_version": (_c.c_char_p, []),
    "aq_last_error": (_c.c_char_p, []),
    "aq_init": (_i32, [_i32]),
    "aq_device_count": (_i32, [_c.POINTER(_i32)]),
    "aq_geometry": (_i32, [_i32, _c.POINTER(_i32), _c.POINTER(_i32),
                           _c.POINTER(_i32), _c.POINTER(_i32)]),
    "aq_matrix_create": (_i32, [_vp, _sz, _i32, _i64, _i64, _i32, _c.POINTER(_vp)]),
    "aq_matrix_destroy": (_i32, [_vp]),
    "aq_matrix_info": (_i32, [_vp, _c.POINTER(_i64), _c.POINTER(_i64),
                              _c.POINTER(_i32), _c.POINTER(_i32), _c.POINTER(_sz)]),
    "aq_matvec": (_i32, [_vp, _vp, _vp, _i32, _vp]),
    "aq_matvec_multi": (_i32, [_c.POINTER(_vp), _i32, _vp, _c.POINTER(_vp), _i32, _vp]),
    "aq_matvec_fused": (_i32, [_c.POINTER(_vp), _i32, _vp, _vp, _vp, _c.c_float,
                               _c.POINTER(_vp), _i32, _vp]),
    "aq_matmul_t": (_i32, [_vp, _vp, _i64, _vp, _i32, _i32, _vp]),
    "aq_matmul_t_swiglu": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _i32, _vp]),
    "aq_dequant_rows": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp]),
    "aq_synchronize": (_i32, [_vp]),
    "aq_release_workspace": (_i32, [_vp]),
    "aq_rmsnorm": (_i32, [_vp, _vp, _i64, _i64, _c.c_float, _vp, _vp]),
    "aq_add_rmsnorm": (_i32, [_vp, _vp, _vp, _i64, _i64, _c.c_float, _vp, _vp]),
    "aq_rope_kv": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                          _vp, _i64, _i64, _vp, _vp, _vp]),
    "aq_attention": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i64, _vp, _i64, _vp, _vp]),
    "aq_attention_batch": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _vp, _i64, _vp,
                                  _vp]),
    "aq_attention_rope": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                                 _vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "aq_attention_rope_noalloc": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp,
                                         _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "aq_attention_scratch_info": (_i32, [_i32, _i32, _i32, _i64, _i64, _c.POINTER(_sz),
                                         _c.POINTER(_sz)]),
    "aq_swiglu": (_i32, [_vp, _vp, _i64, _vp, _vp]),
    "aq_swiglu_pairs": (_i32, [_vp, _i64, _vp, _vp]),
    "aq_add": (_i32, [_vp, _vp, _i64, _vp]),
    "aq_add_rows": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "aq_greedy_advance": (_i32, [_vp, _i64, _vp, _vp, _i64, _vp, _i64, _i32, _vp]),
    "aq_greedy_advance_penalized": (_i32, [_vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _i64,
                                           ctypes.c_double, _i32, _vp]),
    "aq_stream_read": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp]),
}

# sizeof(aq_decode_state): int64 token, uint64 key, int32 pos/fed/count/done
DECODE_STATE_BYTES = 32

_lib = None
_lock = threading.Lock()
_device_ready = False


def _share_torch_runtime() -> None:
    """PyTorch-ROCm ships its own libamdhip64.so.7.  If the library loaded
    first, /opt/rocm's copy would be mapped as well and the process would run
    two HIP runtimes that cannot share the GPU.  Importing torch first (when
    it is installed) makes our DT_NEEDED resolve to torch's already-loaded
    runtime, so device buffers and streams are interchangeable."""
    if os.environ.get("ALPACCA_AMD_NO_TORCH"):
        return
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load() -> ctypes.CDLL:
    """Load the shared library (no device is touched)."""
    global _lib
    if _lib is not None:
        return _lib
    _share_torch_runtime()
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m alpacca_amd.build` "
                    "(the HIP library is the only implementation of this path)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc == AQ_OK:
        return
    msg = (load().aq_last_error() or b"").decode(errors="replace")
    if rc == AQ_ERR_VALUE:
        raise ValueError(msg)
    if rc == AQ_ERR_INDEX:
        raise IndexError(msg)
    raise RuntimeError(msg or f"alpacca_amd error {rc}")


def device_count() -> int:
    n = ctypes.c_int(0)
    check(load().aq_device_count(ctypes.byref(n)))
    return n.value


def ensure_device() -> ctypes.CDLL:
    """Load the library and bind the HIP device (ALPACCA_AMD_DEVICE, default 0)."""
    global _device_ready
    lib = load()
    if not _device_ready:
        with _lock:
            if not _device_ready:
                if device_count() == 0:
                    raise RuntimeError(
                        "no HIP device is visible: the alpacca_amd quantized path "
                        "runs only on an AMD GPU (gfx950)")
                check(lib.aq_init(int(os.environ.get("ALPACCA_AMD_DEVICE", "0"))))
                _device_ready = True
    return lib
