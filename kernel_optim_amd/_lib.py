"""ctypes binding of libkoptim.so, the C-ABI boundary of the HIP kernels.

Every entry point returns an int status: 0 on success, a positive hipError_t
from the launch, or a negative code for an argument error caught on the host
before anything was launched. ``call`` raises RuntimeError on any nonzero
status. There is no fallback: if the library is missing, using an op raises.
"""

import ctypes
import os

from .build import LIB_PATH

_c_void_p = ctypes.c_void_p
_int = ctypes.c_int
_ll = ctypes.c_longlong
_f = ctypes.c_float

# name -> argument types (all return c_int). Mirrors include/koptim.h.
SIGNATURES = {
    "ko_decode_attn_partial": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _ll, _ll,
                               _int, _int, _int, _int, _int, _int, _int, _f, _c_void_p,
                               _c_void_p, _c_void_p],
    "ko_decode_attn_combine": [_c_void_p, _c_void_p, _c_void_p, _int, _int, _int, _int, _int,
                               _int, _int, _int, _c_void_p, _c_void_p],
    "ko_decode_attn": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _ll, _ll, _int,
                       _int, _int, _int, _int, _int, _int, _f, _c_void_p, _c_void_p, _c_void_p,
                       _c_void_p, _c_void_p],
    "ko_decode_attn_qkv": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int,
                           _c_void_p, _c_void_p, _c_void_p, _int, _ll, _ll, _int, _int, _int,
                           _int, _int, _int, _f, _f, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                           _c_void_p, _int, _c_void_p],
    "ko_rope_rows": [_c_void_p, _c_void_p, _c_void_p, _int, _int, _int, _c_void_p, _c_void_p],
    "ko_add_rms_norm": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _f, _c_void_p],
    "ko_qk_norm_rope": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                        _c_void_p, _c_void_p, _c_void_p, _int, _int, _ll, _ll, _f, _int, _int,
                        _int, _int, _c_void_p],
    "ko_qk_norm_rope_acc": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _ll, _ll,
                            _f, _int, _int, _int, _int, _c_void_p],
    "ko_silu_mul": [_c_void_p, _c_void_p, _int, _int, _c_void_p],
    "ko_embed_ss": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _int, _c_void_p],
    "ko_gemv": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _ll, _int, _int, _int, _int,
                _int, _int, _int, _int, _int, _f, _c_void_p],
    "ko_lm_head_argmax": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                          _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int,
                          _c_void_p, _c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _ll, _int,
                          _int, _int, _int, _int, _int, _f, _c_void_p],
    "ko_gemv_argmax_scratch": [_int, _int, _int, _int],
    "ko_gemv_tile": [_c_void_p, _c_void_p, _int, _int, _c_void_p],
    "ko_argmax_rows": [_c_void_p, _ll, _int, _int, _c_void_p, _c_void_p],
    "ko_decode_attn_qkv_oproj": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int,
                                 _c_void_p, _c_void_p, _c_void_p, _int, _ll, _ll, _int, _int,
                                 _int, _int, _int, _int, _f, _f, _c_void_p, _c_void_p,
                                 _c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _c_void_p,
                                 _c_void_p, _int, _int, _c_void_p, _c_void_p],
    "ko_decode_attn_qkv_oproj_sync_ints": [],
    "ko_decode_attn_noalloc": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _int, _ll, _ll,
                               _int, _int, _int, _int, _int, _int, _int, _f, _c_void_p,
                               _c_void_p],
    "ko_decode_attn_token_rows": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _ll, _ll,
                                  _int, _int, _int, _int, _int, _int, _int, _f, _c_void_p,
                                  _c_void_p, _c_void_p, _c_void_p, _c_void_p],
}

# Entry points whose return value is a size, not a status.
RESTYPES = {"ko_gemv_argmax_scratch": _ll, "ko_decode_attn_qkv_oproj_sync_ints": _ll}

_ERRORS = {-22: "invalid argument", -34: "size out of range", -95: "unsupported shape"}

_lib = None


def lib():
    """Load the in-tree library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python -m kernel_optim_amd.build)")
        h = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(h, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, _int)
        _lib = h
    return _lib


def status_message(code):
    if code < 0:
        return _ERRORS.get(code, f"argument error {code}")
    return f"HIP error {code}"


def call(name, *args):
    st = getattr(lib(), name)(*args)
    if st != 0:
        raise RuntimeError(f"{name} failed: {status_message(st)} (status {st})")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


_hip = None


def host_device_ptr(t):
    """The device address of a pinned host tensor (hipHostGetDevicePointer), for
    kernels that store into host memory. Raises if the memory is not mapped
    pinned memory (a kernel store through it would fault)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(_c_void_p), _c_void_p,
                                                 ctypes.c_uint]
        _hip.hipHostGetDevicePointer.restype = _int
    if t.is_cuda or not t.is_pinned():
        raise ValueError("host_device_ptr needs a pinned CPU tensor")
    dev = _c_void_p()
    st = _hip.hipHostGetDevicePointer(ctypes.byref(dev), _c_void_p(t.data_ptr()), 0)
    if st != 0 or not dev.value:
        raise RuntimeError(f"hipHostGetDevicePointer failed (status {st})")
    return dev.value


def stream_ptr(device=None):
    import torch
    return torch.cuda.current_stream(device).cuda_stream
