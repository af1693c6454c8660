"""ctypes binding of libdryft_decode.so (the C ABI declared in include/dryft_decode.h).

torch is imported before the library is opened: torch ships its own libamdhip64 with the same
soname as the system one, so loading torch first makes the library bind to torch's HIP runtime
and torch's stream handles and device pointers are valid in every call.

There is no fallback: if the library is missing or fails to load, ``lib()`` raises.
"""
import ctypes
import os

import torch  # noqa: F401  (load order: see module docstring)

LIB_NAME = "libdryft_decode.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 15

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGS = {
    "dd_abi_version": (_I, []),
    "dd_rmsnorm": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "dd_add_rmsnorm": (_I, [_P, _P, _P, _P, _P, _I, _I, _F, _P]),
    "dd_gemv": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "dd_gemv_counters": (_I, [_I]),
    "dd_gemv_splitk": (_I, [_I, _I, _I]),
    "dd_gemv_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "dd_gemv_add_rmsnorm": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _I, _P, _P, _P]),
    "dd_gemv_add_rmsnorm_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "dd_gate_up_silu": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "dd_silu_mul": (_I, [_P, _P, _I, _I, _P]),
    "dd_qkv_post_decode": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _P, _P, _P,
                                _I, _I, _I, _I, _I, _I, _F, _P, _P]),
    "dd_attn_decode": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "dd_attn_chunk": (_I, [_I, _I, _I]),
    "dd_attn_ws_bytes": (_Z, [_I, _I, _I, _I, _I, _I, _I]),
    "dd_attn_decode_noalloc": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P]),
    "dd_qkv_post_prefill": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P, _P, _P, _I, _I, _I,
                                 _I, _F, _P, _P]),
    "dd_attn_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _I, _P]),
    "dd_spec_seed": (_I, [_P, _I, _P, _P, _I, _P, _P, _P]),
    "dd_spec_draft": (_I, [_P, _I, _P, _P, _I, _I, _P, _P, _P, _P]),
    "dd_spec_accept": (_I, [_P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "dd_gemm_bf16": (_I, [_P, _P, _P, _I, _I, _I, _P, _Z, _I, _P]),
    "dd_gemm_ws_bytes": (_Z, []),
    "dd_gemm_bf16_solutions": (_I, [_I, _I, _I, _Z, _P, _I]),
    "dd_gemm_bf16_supported": (_I, [_I, _I, _I, _Z, _I]),
    "dd_fp8_quant": (_I, [_P, _Z, _P, _P, _P, _P]),
    "dd_fp8_quant_ws_bytes": (_Z, [_Z]),
    "dd_embed_rmsnorm": (_I, [_P, _P, _I, _P, _P, _P, _I, _I, _F, _P, _P]),
    "dd_argmax": (_I, [_P, _I, _I, _P, _P, _I, _P, _P, _P]),
    "dd_argmax_ws_bytes": (_Z, [_I, _I]),
    "dd_step_grid": (_I, []),
    "dd_step_supported": (_I, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "dd_step_counters": (_I, []),
    "dd_step_counters_alloc": (_I, [ctypes.POINTER(_P)]),
    "dd_step_counters_read": (_I, [_P, _P]),
    "dd_step_counters_write": (_I, [_P, _P]),
    "dd_step_counters_clear": (_I, [_P]),
    "dd_step_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "dd_tiled_bytes": (_Z, [_I, _I]),
    "dd_tile_weight": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "dd_decode_step": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                            _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P]),
    "dd_stream_read": (_I, [_P, _Z, _I, _I, _P, _P]),
    "dd_kv_read": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P]),
}

_LIB = None


def exported_symbols():
    """Names of every C-ABI entry point this binding declares."""
    return sorted(_SIGS)


def lib():
    """Load (once) and return the library with argument types declared."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_NAME} is not built ({LIB_PATH}); run `python -c 'import __graft_entry__ as g; "
            "g.build()'` from the repository root")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    v = handle.dd_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"{LIB_NAME} ABI version {v}, binding expects {ABI_VERSION}")
    _LIB = handle
    return _LIB


def check(status, name):
    """Raise on a nonzero status from a C-ABI call."""
    if status != 0:
        what = {1: "invalid argument",
                2: "out of memory (for a no-allocation entry point: the shape needs more than "
                   "its static scratch)"}.get(status, f"hipError {status}")
        raise RuntimeError(f"{name} failed: {what}")
