"""ctypes binding of the C ABI in include/swvr.h (libswvr_hip.so).

The library is found next to this file.  Loading fails loudly when it is
missing: there is no other implementation to fall back to.
"""
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libswvr_hip.so")
ABI_VERSION = 1

BF16, F16, F32 = 0, 1, 2
DTYPE_TAG = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}

OK, EINVAL, EDTYPE, EHIP, EWORKSPACE = 0, -1, -2, -3, -4

# Every symbol include/swvr.h declares, with (restype, argtypes).
_i, _i64, _p, _f, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "swvr_abi_version": (_i, []),
    "swvr_last_error": (ctypes.c_char_p, []),
    "swvr_max_d": (_i64, [_i]),
    "swvr_fwd_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64]),
    "swvr_fwd": (_i, [_i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f,
                      _p, _p, _p, _sz, _p]),
    "swvr_fwd_mixed": (_i, [_i, _i, _i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f,
                            _p, _p, _p, _sz, _p]),
    "swvr_fwd_active_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64]),
    "swvr_fwd_active": (_i, [_i, _i, _i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f,
                             _p, _p, _p, _p, _sz, _p]),
    "swvr_bwd_workspace_size_mixed": (_sz, [_i, _i, _i64, _i64, _i64, _i64, _i64, _i]),
    "swvr_bwd_mixed": (_i, [_i, _i, _i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f,
                            _p, _p, _p, _p, _i64, _p, _i, _p, _i, _p, _i, _p, _p, _sz, _p]),
    "swvr_fwd_partial": (_i, [_i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f,
                              _p, _p, _p, _p, _sz, _p]),
    "swvr_combine": (_i, [_i64, _i64, _i64, _p, _p, _p, _p, _p, _p]),
    "swvr_bwd_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64, _i64, _i]),
    "swvr_bwd": (_i, [_i, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f,
                      _p, _p, _p, _p, _i64, _p, _i, _p, _i, _p, _i, _p, _p, _sz, _p]),
    "swvr_fwd_f64_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "swvr_fwd_f64": (_i, [_i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, ctypes.c_double, _i64,
                          _p, _p, _p, _sz, _p]),
    "swvr_bwd_f64_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "swvr_bwd_f64": (_i, [_i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, ctypes.c_double, _p, _p, _p, _p,
                          _i64, _p, _p, _p, _p, _p, _sz, _p]),
    "swvr_bwd_tiling": (_i, [_i, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_int64), _i]),
    "swvr_fwd_fp8_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "swvr_fwd_fp8": (_i, [_i64, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _f,
                          _p, _p, _p, _sz, _p]),
    "swvr_bwd_fp8_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i]),
    "swvr_bwd_fp8": (_i, [_i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _f, _p, _i64, _i64, _p, _p,
                          _i64, _p, _p, _p, _p, _p, _i64, _p, _i, _p, _i, _p, _i, _p, _p, _sz, _p]),
    "swvr_quantize_e4m3_workspace_size": (_sz, [_i64, _i]),
    "swvr_quantize_e4m3": (_i, [_i64, _i64, _i64, _p, _i64, _i, _i, _p, _i64, _p, _p, _sz, _p]),
    "swvr_mse_loss_workspace_size": (_sz, [_i64]),
    "swvr_mse_loss": (_i, [_i64, _i64, _p, _p, _p, _i, _i64, _p, _f, _i, _p, _p, _p, _p, _p, _sz, _p]),
    "swvr_mse_loss_noalloc": (_i, [_i64, _i64, _p, _p, _p, _i, _i64, _p, _f, _i, _p, _p, _p, _p, _p]),
    "swvr_probe_mfma": (_i, [_i64, _i64, _i, _p, _p]),
    "swvr_timing_enable": (_i, [_i]),
    "swvr_timing_collect": (_i, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), _i]),
    "swvr_kernel_name": (ctypes.c_char_p, [_i]),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load libswvr_hip.so once and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"swvr_amd: {LIB_PATH} is missing. Build it first "
                    "(python -m swvr_amd.build, or __graft_entry__.build()).")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            if lib.swvr_abi_version() != ABI_VERSION:
                raise RuntimeError(f"swvr_amd: ABI version {lib.swvr_abi_version()} != {ABI_VERSION}")
            _lib = lib
    return _lib


def check(rc):
    """Raise the Python exception that matches a C-ABI status code."""
    if rc == OK:
        return
    msg = load().swvr_last_error().decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(f"swvr_amd: {msg}")
    if rc == EDTYPE:
        raise NotImplementedError(f"swvr_amd: {msg}")
    raise RuntimeError(f"swvr_amd (status {rc}): {msg}")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def bwd_tiling(dtype, N, K, V, D, chunk):
    """The backward's tiling for this shape (swvr_bwd_tiling): dict with BM, BV, G, C,
    n_chunks, DP and kernel (0 general, 1 narrow ring, 2 wide)."""
    lib = load()
    out = (ctypes.c_int64 * 7)()
    rc = lib.swvr_bwd_tiling(DTYPE_TAG[dtype], N, K, V, D, chunk, out, 7)
    if rc < 0:
        check(rc)
    return dict(zip(("BM", "BV", "G", "C", "n_chunks", "DP", "kernel"), list(out)))


def kernel_timing(enable=None):
    """Turn launch timing on/off, or (enable=None) collect {kernel: (ms, launches)}."""
    lib = load()
    if enable is not None:
        lib.swvr_timing_enable(1 if enable else 0)
        return None
    n = 32
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int64 * n)()
    k = lib.swvr_timing_collect(ms, cnt, n)
    if k < 0:
        check(k)
    return {lib.swvr_kernel_name(i).decode(): (ms[i], cnt[i]) for i in range(k) if cnt[i] > 0}
