"""MI355X (gfx950) kernels for the memory-bound fused graph fragments of
SherlockNoMad/KernelProblems: RMSNorm forward/backward (with residual-add and
gradient epilogues), embedding gather and its dense deterministic backward,
rotary position embedding on q/k, the SwiGLU gate forward/backward and the
vocabulary cross-entropy loss forward/backward.

Layers:
  * ``include/kp.h`` + ``csrc/*.hip``  -- the C ABI and the HIP kernels;
  * ``_lib``      -- ctypes binding of ``libkp_hip.so`` (no fallback path);
  * ``_kp_torch`` -- native torch extension (``csrc/kp_torch.cpp``): the
    bodies of the tensor-level operations, calling the C ABI;
  * ``fused``     -- tensor-level fused operations over the C ABI;
  * ``aten``      -- drop-ins for the aten operators used by the fragments;
  * ``fragments`` -- ``kernel_function`` drop-ins for individual reference
    fragments, keyed by their reference id.
"""
from . import aten, fused
from ._lib import KPError, LIB_PATH, version
from .fused import (
    check_indices,
    cross_entropy_backward,
    cross_entropy_forward_backward,
    cross_entropy_loss,
    embedding,
    embedding_dense_backward,
    embedding_rms_norm,
    index_checking,
    rms_norm,
    rms_norm_backward,
    rms_norm_forward_backward,
    rope,
    rope_complex,
    set_index_checking,
    silu,
    swiglu,
    swiglu_backward,
    swiglu_forward_backward,
    unshard,
)

__all__ = [
    "KPError",
    "LIB_PATH",
    "aten",
    "check_indices",
    "cross_entropy_backward",
    "cross_entropy_forward_backward",
    "cross_entropy_loss",
    "embedding",
    "embedding_dense_backward",
    "embedding_rms_norm",
    "fused",
    "index_checking",
    "rms_norm",
    "rms_norm_backward",
    "rms_norm_forward_backward",
    "rope",
    "rope_complex",
    "set_index_checking",
    "silu",
    "swiglu",
    "swiglu_backward",
    "swiglu_forward_backward",
    "unshard",
    "version",
]
