"""Tensor-level entry points over the C ABI: the fused hot-path operations.

Each function validates its tensors (device, dtype, shapes), allocates the
outputs and any workspace with torch's caching allocator, and enqueues the
HIP kernels on the current stream of the input's device -- all of it in one
call into the native module _kp_torch (csrc/kp_torch.cpp), which calls the C
ABI of libkp_hip.so: a call costs the kernel launches plus a few allocations
of host time (about half of what the same work took through ctypes).  This
module keeps the per-device out-of-range flag and the index-checking mode.
Nothing here computes on the CPU and nothing falls back to torch ops: a CPU
tensor, an unsupported dtype or a missing library raises.

The aten-compatible drop-ins (``kernelproblems_amd.aten``) and the
per-fragment ``kernel_function``s (``kernelproblems_amd.fragments``) are
thin compositions of these.
"""
from __future__ import annotations

import os
from typing import Optional, Sequence

import torch

from . import _lib as L

_native_mod = None


def _native():
    """The native wrapper module (_kp_torch.so, built beside libkp_hip.so)."""
    global _native_mod
    if _native_mod is None:
        try:
            from . import _kp_torch
        except ImportError as e:
            raise RuntimeError(
                f"kernelproblems_amd/_kp_torch.so is missing or does not load ({e}): build it with "
                "`python -m kernelproblems_amd.build` (there is no CPU fallback)") from e
        _native_mod = _kp_torch
    return _native_mod


_index_checking = os.environ.get("KP_CHECK_INDICES", "0") not in ("", "0")


def set_index_checking(enabled: bool) -> None:
    """When enabled, index-taking ops synchronise after the launch and raise
    IndexError if an id / position / target was out of range.  When disabled
    (the default: no host synchronisation per call) the kernels still never
    read out of bounds -- such rows come out as zeros (targets count as
    ignored) -- and still record the event in a per-device flag that
    check_indices() reports."""
    global _index_checking
    _index_checking = bool(enabled)
    # (switching modes keeps what unchecked calls recorded for check_indices;
    # each checked call clears the record before it runs)


def index_checking() -> bool:
    return _index_checking


_flags = {}


def check_indices() -> None:
    """Raises IndexError if any index-taking call on any device met an
    out-of-range id, position or target since the last check (or since it
    raised), then clears the record.  Synchronises the devices that have
    made such calls; call it where a synchronisation is paid anyway (e.g.
    once per step)."""
    bad = [i for i, f in _flags.items() if int(f.item()) != 0]
    for i in bad:
        _flags[i].zero_()
    if bad:
        raise IndexError(f"index out of range in a kernel call on device(s) {bad} since the last check")


# ---------------------------------------------------------------- helpers
def _flag(device: torch.device):
    """The device's persistent int32 out-of-range flag (allocated on first
    use; kernels only ever set it, check_indices() clears it).  In checking
    mode it is cleared before the call, so that the check after the call
    reports that call alone."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    f = _flags.get(idx)
    if f is None:
        f = _flags[idx] = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", idx))
    elif _index_checking:
        f.zero_()
    return f


def _raise_if_flagged(flag, what: str) -> None:
    """With index checking on: synchronise and raise if the flag is set."""
    if _index_checking and flag is not None and int(flag.item()) != 0:
        flag.zero_()
        raise IndexError(f"{what}: index out of range")


# ---------------------------------------------------------------- RMSNorm
def rms_norm(
    x_terms: Sequence[torch.Tensor],
    weight: Optional[torch.Tensor],
    eps: float,
    n: int,
    *,
    return_h: bool = False,
    return_rstd: bool = True,
):
    """Fused (residual add +) RMSNorm forward.

    h = bf16 running sum of x_terms (eager bf16 add.Tensor rounding), y =
    bf16(h * rstd * w), rstd = 1/sqrt(mean(h^2) + eps) over the trailing n
    elements.  Returns (h or None, y, rstd[M] or None); y has x_terms[0]'s shape.
    """
    return _native().rms_norm(x_terms, weight, float(eps), int(n), bool(return_h), bool(return_rstd))


def rms_norm_backward(
    dy_terms: Sequence[torch.Tensor],
    x_terms: Sequence[torch.Tensor],
    rstd: Optional[torch.Tensor],
    weight: Optional[torch.Tensor],
    eps: float,
    n: int,
    *,
    dx_residual: Optional[torch.Tensor] = None,
    want_dx: bool = True,
    dw: Optional[str] = "f32",
):
    """Fused RMSNorm backward.

    dy / x are bf16 running sums of their terms; rstd (fp32, M values) is
    recomputed from x with eps when None.  dx = bf16(dx_residual + bf16(dx))
    when dx_residual is given.  ``dw`` selects the weight gradient: "f32"
    (fp32 sum), "f32_bf16" (the reference's bf16 rounding widened to fp32),
    "bf16", or None.  Returns (dx, dw).
    """
    return _native().rms_norm_backward(dy_terms, x_terms, rstd, weight, float(eps), int(n), dx_residual,
                                       bool(want_dx), dw)


def rms_norm_forward_backward(
    dy_terms: Sequence[torch.Tensor],
    x_terms: Sequence[torch.Tensor],
    weight: Optional[torch.Tensor],
    eps: float,
    n: int,
    *,
    dx_residual: Optional[torch.Tensor] = None,
    dw: Optional[str] = "f32",
    return_h: bool = False,
    return_rstd: bool = False,
):
    """RMSNorm forward and backward of the same rows in one row pass: the
    _fused_rms_norm -> _fused_rms_norm_backward regions whose forward rstd
    only feeds the backward (v6/0b493aad68f0/problem.py:16-47,
    v6/822931829090/problem.py:10-66).  x = bf16 running sum of x_terms,
    dy = that of dy_terms; rstd is computed once from x and eps and used for
    both y = bf16(x * rstd * w) and the backward (as rms_norm_backward with
    rstd=None).  Returns (y, dx, dw, h or None, rstd or None); y and dx have
    x_terms[0]'s shape, h is only produced for several x terms."""
    return _native().rms_norm_forward_backward(dy_terms, x_terms, weight, float(eps), int(n), dx_residual, dw,
                                               bool(return_h), bool(return_rstd))


# ---------------------------------------------------------------- embedding
def embedding(table: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """out[..., :] = table[indices[...], :] (bit copy), shape indices.shape + [D]."""
    flag = _flag(table.device) if table.is_cuda else None
    out = _native().embedding(table, indices, flag)
    _raise_if_flagged(flag, "embedding")
    return out


def embedding_rms_norm(
    table: torch.Tensor,
    indices: torch.Tensor,
    weight: Optional[torch.Tensor],
    eps: float,
    *,
    return_h: bool = False,
    return_rstd: bool = True,
):
    """RMSNorm of embedding rows: h = table[indices] (bit copy), y =
    bf16(h * rstd * w), in one launch that reads each gathered row straight
    into the norm (the embedding.default -> _fused_rms_norm region of
    v8/12545c1e9b06/problem.py:24-42).  The weight may be a segmented FSDP
    view as in rms_norm.  Returns (h or None, y, rstd or None), shaped
    indices.shape + [D].  Row shapes without a fused kernel run the gather
    and the norm as two launches (same results)."""
    flag = _flag(table.device) if table.is_cuda else None
    out = _native().embedding_rms_norm(table, indices, weight, float(eps), bool(return_h), bool(return_rstd), flag)
    _raise_if_flagged(flag, "embedding_rms_norm")
    return out


def embedding_dense_backward(
    grad_output: torch.Tensor,
    indices: torch.Tensor,
    num_weights: int,
    padding_idx: int = -1,
    scale_grad_by_freq: bool = False,
    *,
    out_dtype: torch.dtype = torch.float32,
    round_to_bf16: bool = False,
) -> torch.Tensor:
    """Dense [num_weights, D] gradient of an embedding, fp32 accumulation,
    deterministic sort-and-segment.  Every row is written; the rows at the top
    of the vocabulary that the early launches zero unconditionally are written
    a second time when an id touches them."""
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"embedding_dense_backward: unsupported out_dtype {out_dtype}")
    flag = _flag(grad_output.device) if grad_output.is_cuda else None
    out = _native().embedding_dense_backward(grad_output, indices, int(num_weights),
                                             -1 if padding_idx is None else int(padding_idx), bool(scale_grad_by_freq),
                                             out_dtype == torch.float32, bool(round_to_bf16), flag)
    _raise_if_flagged(flag, "embedding_dense_backward")
    return out


def rms_norm_embedding_backward(
    dy_terms: Sequence[torch.Tensor],
    x: torch.Tensor,
    rstd: Optional[torch.Tensor],
    weight: Optional[torch.Tensor],
    eps: float,
    n: int,
    dx_residual: torch.Tensor,
    indices: torch.Tensor,
    num_weights: int,
    padding_idx: int = -1,
    *,
    want_y: bool = False,
    dw: Optional[str] = "f32",
    out_dtype: torch.dtype = torch.float32,
    round_to_bf16: bool = False,
):
    """The RMSNorm backward whose residual output g = bf16(dx_residual + dx)
    feeds embedding_dense_backward of the same tokens, as one row pass that
    sums g into the table without storing it (the _fused_rms_norm_backward ->
    add -> embedding_dense_backward chains of v6/0b493aad68f0/problem.py:45-71,
    v5/118d525f44e0/problem.py:50-80, v8/f6251e84e3fa/problem.py:37-57).

    rstd=None recomputes rstd from x (and with want_y the same pass writes the
    forward's y = bf16(x * rstd * w)); otherwise rstd is the saved forward's.
    The table is what embedding_dense_backward(g, indices, num_weights,
    padding_idx) returns (no scale_grad_by_freq); the weight gradient is that
    of rms_norm_backward, summed in a different (fixed) grouping of rows.
    Returns (y or None, dw or None, table)."""
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"rms_norm_embedding_backward: unsupported out_dtype {out_dtype}")
    flag = _flag(x.device) if x.is_cuda else None
    out = _native().rms_norm_embedding_backward(dy_terms, x, rstd, weight, float(eps), int(n), dx_residual,
                                                bool(want_y), dw, indices, int(num_weights),
                                                -1 if padding_idx is None else int(padding_idx),
                                                out_dtype == torch.float32, bool(round_to_bf16), flag)
    _raise_if_flagged(flag, "rms_norm_embedding_backward")
    return out


# ---------------------------------------------------------------- RoPE
_PAIRING = {"half": L.KP_ROPE_HALF, "interleaved": L.KP_ROPE_INTERLEAVED}


def rope(
    q: torch.Tensor,
    k: Optional[torch.Tensor] = None,
    *,
    positions: Optional[torch.Tensor] = None,
    theta: Optional[float] = None,
    freqs_cis: Optional[torch.Tensor] = None,
    pairing: str = "half",
    conj: bool = False,
    q_dtype: torch.dtype = torch.bfloat16,
    k_dtype: torch.dtype = torch.bfloat16,
    copies: bool = False,
):
    """Rotary embedding of q (and k) laid out [B, S, H, D] (unit stride on D).

    Angles come from ``theta`` (inv_freq_i = theta^(-2i/D), angle =
    fp32(pos * inv_freq_i), cos/sin evaluated in fp32 in-kernel) or from the
    complex64 table ``freqs_cis`` whose last dim is D/2 (row p used for
    position p).  positions: [B, S] or [S] integer tensor, default s.
    pairing "half" = (i, i + D/2), "interleaved" = (2i, 2i+1).  conj=True
    rotates by the conjugate (backward).  q_dtype / k_dtype pick each
    output's type, bf16 or fp32 (the fp32 rotation result without the final
    rounding).  Returns contiguous (q_out, k_out); with copies=True, returns
    (q_out, k_out, q_copy, k_copy), the copies separate tensors holding the
    same values, written by the same pass over q and k (kp_rope_bf16_twice).
    """
    for dt in (q_dtype, k_dtype):
        if dt not in (torch.bfloat16, torch.float32):
            raise RuntimeError(f"rope: output dtype must be bfloat16 or float32, got {dt}")
    mode = _PAIRING.get(pairing)
    if mode is None:
        raise ValueError(f"rope: pairing must be 'half' or 'interleaved', got {pairing!r}")
    flag = _flag(q.device) if (freqs_cis is not None and q.is_cuda) else None
    out = _native().rope(q, k, positions, None if theta is None else float(theta), freqs_cis, mode, bool(conj),
                         q_dtype == torch.float32, k_dtype == torch.float32, bool(copies), flag)
    _raise_if_flagged(flag, "rope")
    return out


def rope_complex(q: torch.Tensor, k: Optional[torch.Tensor] = None, *, freqs_cis: torch.Tensor,
                 positions: Optional[torch.Tensor] = None, conj: bool = False):
    """q (and k) already viewed as complex64 [B, S, H, P] times the complex64
    table ``freqs_cis`` (last dim P, row p for position p; a [1, S, 1, P] or
    [S, P] table), in fp32 -- the index -> mul regions of
    v1/075cb40f3d5d/problem.py:8-27.  positions: [B, S], [1, S] or [S]
    integers, default s.  conj=True multiplies by the conjugate table.
    Returns contiguous complex64 (q_out, k_out)."""
    flag = _flag(q.device) if q.is_cuda else None
    out = _native().rope_complex(q, k, freqs_cis, positions, bool(conj), flag)
    _raise_if_flagged(flag, "rope_complex")
    return out


# ---------------------------------------------------------------- FSDP unshard
def unshard(flat: torch.Tensor, shards: int, split_sizes: Sequence[int], keep: Sequence[int]):
    """Contiguous copies of column segments of a sharded flat parameter buffer.

    ``flat`` holds ``shards`` rows of equal length (a 1-D all-gather output or
    a [shards, L] row-strided view); the row is split into ``split_sizes``.
    Returns, for each index in ``keep``, a fresh contiguous [shards, size]
    tensor -- the view -> split_with_sizes -> clone chain of an FSDP unshard,
    done for all kept segments in one launch.
    """
    return _native().unshard(flat, int(shards), [int(v) for v in split_sizes], [int(i) for i in keep])


# ---------------------------------------------------------------- SwiGLU gate
def swiglu(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """bf16(bf16(silu(a)) * b): the silu -> mul region between the w1/w3 and
    w2 projections of a feed-forward block (v8/c68dae22972b/problem.py:15-28),
    fp32 arithmetic (silu = a / (1 + exp(-a))).  Returns a contiguous tensor
    of a's shape."""
    return _native().swiglu(a, b)


def swiglu_backward(g: torch.Tensor, s: torch.Tensor, b: torch.Tensor, a: torch.Tensor):
    """Gradients of the SwiGLU gate out = s * b, s = silu(a), given g = dout
    (v8/385e1beb9bb9/problem.py:17-33): db = bf16(g * s) and
    da = silu_backward(bf16(g * b), a) = t * sig * (1 + a * (1 - sig)).
    s is the recomputed silu(a) the graph keeps.  Returns contiguous
    (db, da) of g's shape."""
    return _native().swiglu_backward(g, s, b, a)


def silu(a: torch.Tensor) -> torch.Tensor:
    """bf16(silu(a)) alone (v7/58e7a4d6cde3/problem.py:10-19), the same bits as
    eager's bf16 silu.  Returns a contiguous tensor of a's shape."""
    return _native().silu(a)


def swiglu_forward_backward(a: torch.Tensor, b: torch.Tensor, g: torch.Tensor):
    """The SwiGLU gate forward recomputed with its backward in one pass
    (v6/182d2dcd0652/problem.py:10-46): with s = bf16(silu(a)) kept in
    registers, h = bf16(s * b), db = bf16(g * s) and
    da = silu_backward(bf16(g * b), a).  Returns contiguous (h, db, da)."""
    return _native().swiglu_forward_backward(a, b, g)


# ---------------------------------------------------------------- cross-entropy
def cross_entropy_loss(logits: torch.Tensor, targets: torch.Tensor, *, ignore_index: int = -100, scale: float = 1.0,
                       return_lse: bool = False):
    """Summed token cross-entropy of bf16 logits [..., V] against integer
    targets [...]: loss = scale * sum over rows with target != ignore_index of
    (logsumexp(fp32 logits) - logit[target]), the fp32 _log_softmax ->
    nll_loss_forward(reduction sum) -> div region of v8/71f1d2c9f38b/problem.py:15-40
    without materialising the log-softmax.  Returns 0-dim fp32 tensors
    (loss, total_weight) and, with return_lse, the fp32 per-row logsumexp."""
    flag = _flag(logits.device) if logits.is_cuda else None
    out = _native().cross_entropy_loss(logits, targets, int(ignore_index), float(scale), bool(return_lse), flag)
    _raise_if_flagged(flag, "cross_entropy")
    return out


def cross_entropy_forward_backward(logits: torch.Tensor, targets: torch.Tensor, grad_loss: float, *,
                                   ignore_index: int = -100, scale: float = 1.0, return_loss: bool = False,
                                   in_place: bool = False):
    """The bf16 logits gradient of the summed cross-entropy straight from the
    bf16 logits [..., V]: out = grad - exp(x - lse) * sum(grad), grad =
    -grad_loss at each counted row's target (v5/fb5b36393cbd/problem.py:16-59:
    _log_softmax -> nll_loss_forward -> nll_loss_backward ->
    _log_softmax_backward_data -> _to_copy(bf16), the fp32 log-softmax never
    stored).  With return_loss also (loss, total_weight) as
    cross_entropy_loss(..., scale=scale) computes them.  in_place=True writes
    the gradient over the logits (which must then be contiguous) and
    returns them."""
    flag = _flag(logits.device) if logits.is_cuda else None
    out = _native().cross_entropy_forward_backward(logits, targets, float(grad_loss), int(ignore_index), float(scale),
                                                   bool(return_loss), bool(in_place), flag)
    _raise_if_flagged(flag, "cross_entropy_forward_backward")
    return out


def cross_entropy_backward(log_softmax: torch.Tensor, targets: torch.Tensor, grad_loss: float, *,
                           ignore_index: int = -100) -> torch.Tensor:
    """Gradient of the summed cross-entropy w.r.t. the logits, in bf16, from
    the saved fp32 log-softmax L [..., V]: out = grad - exp(L) * sum(grad) with
    grad = -grad_loss at each non-ignored row's target
    (v8/622c35f5d1c6/problem.py:16-33: nll_loss_backward(sum) ->
    _log_softmax_backward_data -> _to_copy(bf16)).  grad_loss is the
    upstream gradient of the loss as a Python float (a constant in the
    fragment: 1 / 8192).  Returns a contiguous bf16 tensor of L's shape."""
    flag = _flag(log_softmax.device) if log_softmax.is_cuda else None
    out = _native().cross_entropy_backward(log_softmax, targets, float(grad_loss), int(ignore_index), flag)
    _raise_if_flagged(flag, "cross_entropy_backward")
    return out
