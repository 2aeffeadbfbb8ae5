"""ctypes binding of libmacai_gdr.so (the C ABI declared in include/macai_gdr.h).

The library is built in-tree by mac-ai-engineering_amd/build.py (hipcc, gfx950) next to this file.  There is no
fallback: if it is missing or fails to load, every call raises.
"""
import ctypes
import os

import torch

LIB_NAME = "libmacai_gdr.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

F32, BF16, F16 = 0, 1, 2
BF16_F32 = 3                          # MACAI_GDR_BF16_F32: bf16 tensors, float32 arithmetic (prep, state_fwd, chunk_bwd)
OK, EINVAL, EUNSUP, ELAUNCH = 0, 1, 2, 3
STORE_STATES, NO_OUTPUT = 1, 8
NOALLOC_SCRATCH_BYTES = 128 << 20     # MACAI_GDR_NOALLOC_SCRATCH_BYTES
ABI_VERSION = 13

_p, _i64, _i32, _f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
# name -> argument types (the order of include/macai_gdr.h)
SIGNATURES = {
    "macai_gdr_prep": [_p] * 12 + [_i64] * 6 + [_i32, _i32, _f, _p, _i64, _p],
    "macai_gdr_state_fwd": [_p] * 11 + [_i64] * 5 + [_i32, _i32, _i32, _p, _i64, _p],
    "macai_gdr_state_bwd": [_p] * 10 + [_i64] * 5 + [_i32, _i32, _p, _i64, _p],
    "macai_gdr_state_pair": [_p] * 14 + [_i64] * 5 + [_i32, _i32, _p, _i64, _p],
    "macai_gdr_state_map": [_p] * 5 + [_i64] * 5 + [_i32, _i32, _p, _i64, _p],
    "macai_gdr_state_scan": [_p] * 3 + [_i64] * 5 + [_p],
    "macai_gdr_chunk_bwd": [_p] * 16 + [_i64] * 6 + [_i32, _i32, _f, _p, _i64, _p],
    "macai_gdr_decode": [_p] * 8 + [_i64] * 5 + [_i32, _i32, _f, _p],
    "macai_gdr_group_sum": [_p] * 2 + [_i64] * 5 + [_i32, _p],
    "macai_gdr_conv_fwd": [_p] * 5 + [_i64] * 7 + [_i32, _i32, _p],
    "macai_gdr_conv_bwd": [_p] * 8 + [_i64] * 7 + [_i32, _i32, _p],
    "macai_gdr_conv_partials": [_i64] * 3,
    "macai_gdr_gates_fwd": [_p] * 6 + [_i64] * 2 + [_i32, _p],
    "macai_gdr_gates_bwd": [_p] * 10 + [_i64] * 2 + [_i32, _p],
    "macai_gdr_forward": [_p] * 9 + [_i64] * 7 + [_i32, _i32, _f, _i32, _p, _i64, _p],
    "macai_gdr_forward_workspace": [_i64] * 5 + [_i32, _i64],
    "macai_gdr_forward_noalloc": [_p] * 8 + [_i64] * 6 + [_i32, _i32, _f, _i32, _p, _i64, _p],
    "macai_gdr_probe_stream": [_i32, _p, _p, _i64, _i32, _p],
    "macai_gdr_probe_mfma": [_i32, _i32, _p, _i32, _p],
    "macai_gdr_probe_mfma_flops": [_i32, _i32, _i32],
}
# the rest return an int status
RESTYPES = {"macai_gdr_conv_partials": _i64, "macai_gdr_forward_workspace": _i64, "macai_gdr_probe_mfma_flops": _i64}

_lib = None
_fns = {}        # name -> the library's function object (a lookup per call costs host time on every launch)


class NativeError(RuntimeError):
    """A HIP launch failure reported by the library."""


def lib():
    """The loaded library (loaded once); raises RuntimeError when it is not built or does not load."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                               "(or mac-ai-engineering_amd/build.py) first")
        L = ctypes.CDLL(LIB_PATH)
        L.macai_gdr_last_error.restype = ctypes.c_char_p
        L.macai_gdr_last_error.argtypes = []
        L.macai_gdr_abi_version.restype = ctypes.c_int
        L.macai_gdr_abi_version.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = RESTYPES.get(name, ctypes.c_int)
            fn.argtypes = args
        if L.macai_gdr_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {L.macai_gdr_abi_version()}, expected {ABI_VERSION}")
        _lib = L
    return _lib


def ptr(t):
    return None if t is None else t.data_ptr()


def dtype_code(dt, f16=False):
    """The dtype code of a torch dtype: float32 or bfloat16 (and float16 where the entry point takes it)."""
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if f16 and dt == torch.float16:
        return F16
    raise NotImplementedError(f"the HIP kernels take float32 or bfloat16{' or float16' if f16 else ''}, got {dt}")


def stream_of(t):
    """hipStream_t of torch's current stream on t's device (the raw handle, without building a Stream object)."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def call(name, *args):
    """Call entry point `name`; raise on a non-zero return (ValueError for bad arguments, NotImplementedError for an
    unsupported shape or dtype, NativeError for a launch failure)."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != OK:
        msg = lib().macai_gdr_last_error().decode()
        if rc == EINVAL:
            raise ValueError(msg)
        if rc == EUNSUP:
            raise NotImplementedError(msg)
        raise NativeError(msg)
