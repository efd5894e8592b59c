"""ctypes binding of the gfx950 C-ABI library (``include/kp.h``).

This is the only place that touches ``libkp_hip.so``.  torch is imported
first so that the library's ``libamdhip64.so.7`` dependency resolves to the
HIP runtime torch already loaded (one runtime per process, shared streams).

There is no fallback: if the library is missing or was built for another
target, every entry point raises.  Build it with
``python -m kernelproblems_amd.build``.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent / "libkp_hip.so"

KP_OK = 0
KP_EINVAL = 1
KP_EUNSUPPORTED = 2
KP_EHIP = 3
KP_EWORKSPACE = 4
KP_EBUSY = 5
KP_DTYPE_F32 = 0
KP_DTYPE_BF16 = 1
KP_ROPE_HALF = 0
KP_ROPE_INTERLEAVED = 1
KP_STORE_NONTEMPORAL = 0
KP_STORE_WRITE_THROUGH = 1

_STATUS = {
    KP_EINVAL: "invalid argument",
    KP_EUNSUPPORTED: "unsupported",
    KP_EHIP: "HIP error",
    KP_EWORKSPACE: "workspace too small",
    KP_EBUSY: "scratch busy on another stream",
}


class KPError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        self.fn = fn
        self.status = status
        super().__init__(f"{fn}: {_STATUS.get(status, status)}: {message}")


vp = C.c_void_p
i64 = C.c_int64
i32 = C.c_int
f32 = C.c_float
f64 = C.c_double
sz = C.c_size_t
pvp = C.POINTER(C.c_void_p)
pi64 = C.POINTER(C.c_int64)
pi32 = C.POINTER(C.c_int32)
pf32 = C.POINTER(C.c_float)

# name -> (restype, argtypes); mirrors include/kp.h one for one.
SIGNATURES = {
    "kp_version": (C.c_char_p, []),
    "kp_last_hip_error": (i32, []),
    "kp_last_error_message": (C.c_char_p, []),
    "kp_profile_dominant_kernel": (None, [vp, vp]),
    "kp_debug_block_trace": (None, [vp, sz]),
    "kp_rmsnorm_fwd_bf16": (
        i32,
        [pvp, pi64, i32, vp, i64, i64, vp, i64, vp, i64, vp, i64, i64, f32, vp],
    ),
    "kp_rmsnorm_bwd_workspace_size": (sz, [i64, i64]),
    "kp_rmsnorm_bwd_bf16": (
        i32,
        [pvp, pi64, i32, pvp, pi64, i32, vp, vp, i64, i64, vp, i64, vp, i64, vp, vp, i32,
         i64, i64, f32, vp, sz, vp],
    ),
    "kp_rmsnorm_bwd_noalloc_max_bytes": (sz, []),
    "kp_rmsnorm_bwd_bf16_noalloc": (
        i32,
        [pvp, pi64, i32, pvp, pi64, i32, vp, vp, i64, i64, vp, i64, vp, i64, vp, vp, i32,
         i64, i64, f32, vp],
    ),
    "kp_rmsnorm_fwd_bwd_workspace_size": (sz, [i64, i64]),
    "kp_rmsnorm_fwd_bwd_bf16": (
        i32,
        [pvp, pi64, i32, pvp, pi64, i32, vp, i64, i64, vp, i64, vp, i64, vp, vp, i64, vp, i64, vp, vp, i32,
         i64, i64, f32, vp, sz, vp],
    ),
    "kp_embedding_fwd_bf16": (i32, [vp, i64, i64, i64, vp, i32, i64, vp, i64, vp, vp]),
    "kp_embedding_bwd_workspace_size": (sz, [i64, i64, i64]),
    "kp_embedding_bwd_bf16": (
        i32,
        [vp, i64, vp, i32, i64, i64, i64, i64, i32, vp, i32, i32, vp, sz, vp, vp],
    ),
    "kp_rmsnorm_embedding_bwd_workspace_size": (sz, [i64, i64, i64]),
    "kp_rmsnorm_embedding_bwd_bf16": (
        i32,
        [pvp, pi64, i32, vp, i64, vp, vp, i64, i64, vp, i64, vp, i64, vp, vp, vp, i32, i64, i64, f32,
         vp, i32, i64, i64, vp, i32, i32, vp, sz, vp, vp],
    ),
    "kp_rope_bf16": (
        i32,
        [vp, vp, i64, pi64, pi64, vp, vp, i64, pi64, pi64, i64, i64, i64, vp, i32, i64, i64,
         i32, f64, vp, i64, i64, i32, i32, vp, vp],
    ),
    "kp_rope_bf16_twice": (
        i32,
        [vp, vp, i64, pi64, pi64, vp, vp, i64, pi64, pi64, i64, i64, i64, vp, i32, i64, i64,
         i32, f64, vp, i64, i64, i32, i32, vp, vp, vp, vp],
    ),
    "kp_rope_c64": (i32, [vp, vp, i64, pi64, pi64, vp, vp, i64, pi64, pi64, i64, i64, i64, vp, i32, i64, i64, vp, i64, i64,
                          i32, vp, vp]),
    "kp_unshard_bf16": (i32, [vp, i64, i64, pi64, pi64, pvp, i32, vp]),
    "kp_stream_probe": (i32, [pvp, i32, i64, pvp, i32, i64, i32, i32, vp]),
    "kp_embedding_rmsnorm_fwd_bf16": (i32, [vp, i64, i64, vp, i32, i64, vp, i64, i64, vp, i64, vp, i64, vp, i64, f32,
                                            vp, vp]),
    "kp_swiglu_fwd_bf16": (i32, [vp, i64, vp, i64, vp, i64, i64, i64, vp]),
    "kp_swiglu_bwd_bf16": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i64, i64, vp]),
    "kp_silu_bf16": (i32, [vp, i64, vp, i64, i64, i64, vp]),
    "kp_swiglu_fwd_bwd_bf16": (i32, [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i64, i64, vp]),
    "kp_swiglu_math_selftest": (i32, [vp, vp, vp, vp, vp]),
    "kp_cross_entropy_fwd_workspace_size": (sz, [i64]),
    "kp_cross_entropy_fwd_bf16": (i32, [vp, i64, i64, i64, vp, i32, i64, f32, vp, vp, vp, vp, vp, sz, vp]),
    "kp_cross_entropy_bwd_bf16": (i32, [vp, i64, vp, i32, i64, f32, vp, i64, i64, i64, vp, vp]),
    "kp_cross_entropy_fwd_bwd_bf16": (i32, [vp, i64, i64, i64, vp, i32, i64, f32, vp, i64, f32, vp, vp, vp, vp, sz, vp]),
}

_lib = None


def lib() -> C.CDLL:
    """Loads libkp_hip.so once and declares every signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m kernelproblems_amd.build` "
                "(there is no CPU fallback)"
            )
        handle = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


_fns = {}


def call(name: str, *args) -> None:
    """Calls an entry point and raises KPError on a non-zero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    st = fn(*args)
    if st != KP_OK:
        msg = lib().kp_last_error_message().decode(errors="replace")
        raise KPError(name, st, msg)


def ptr_array(ptrs):
    return (C.c_void_p * len(ptrs))(*ptrs)


def i64_array(vals):
    return (C.c_int64 * len(vals))(*vals)


def version() -> str:
    return lib().kp_version().decode()
