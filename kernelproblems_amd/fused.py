"""Tensor-level entry points over the C ABI: the fused hot-path operations.

Each function validates its tensors (device, dtype, shapes), allocates the
outputs and any workspace with torch's caching allocator, and enqueues the
HIP kernels on the current stream of the input's device.  rms_norm,
rms_norm_backward, embedding, rope and rope_complex -- the entry points most
fragments call -- do all of that in the native module _kp_torch
(csrc/kp_torch.cpp), which halves their host time per call.  Nothing here
computes on the CPU and nothing falls back to torch ops: a CPU tensor, an
unsupported dtype or a missing library raises.

The aten-compatible drop-ins (``kernelproblems_amd.aten``) and the
per-fragment ``kernel_function``s (``kernelproblems_amd.fragments``) are
thin compositions of these.
"""
from __future__ import annotations

import math
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
def _stream(device: torch.device) -> int:
    """The raw hipStream_t of the device's current torch stream (read without
    building a Stream object: this runs on every call)."""
    idx = device.index
    return torch._C._cuda_getCurrentRawStream(idx if idx is not None else torch.cuda.current_device())


def _need_gpu(name: str, t: torch.Tensor, dtype: Optional[torch.dtype] = torch.bfloat16) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name}: expected a GPU tensor, got device {t.device} (no CPU path exists)")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name}: expected dtype {dtype}, got {t.dtype}")


def _as_rows(t: torch.Tensor, n: int):
    """Returns (tensor, row_stride, rows) for t viewed as [rows, n] with unit
    inner stride; copies to contiguous only if no such view exists."""
    numel = t.numel()
    if numel % n != 0:
        raise RuntimeError(f"tensor of {numel} elements is not a whole number of rows of {n}")
    m = numel // n
    if m == 0:
        return t, n, 0
    if t.is_contiguous():
        return t, n, m
    try:
        v = t.view(m, n)
        if n == 1 or v.stride(1) == 1:
            return t, v.stride(0), m
    except RuntimeError:
        pass
    t = t.contiguous()
    return t, n, m


def _weight_segments(w: torch.Tensor, n: int):
    """(tensor, seg_len, seg_stride): element i of the flattened weight sits at
    (i // seg_len) * seg_stride + i % seg_len.  Covers contiguous vectors and
    2-D row-strided views such as an [8, 512] slice of an FSDP flat buffer."""
    if w.numel() != n:
        raise RuntimeError(f"weight has {w.numel()} elements, expected {n}")
    if w.dim() == 1 and (w.stride(0) == 1 or n == 1):
        return w, n, n
    if w.dim() == 2 and (w.stride(1) == 1 or w.shape[1] == 1):
        return w, w.shape[1], w.stride(0)
    if w.is_contiguous():
        return w, n, n
    w = w.contiguous()
    return w, n, n


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


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


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


def _bwd_operands(who, dy_terms, x_terms, weight, n, dx_residual):
    """Row views of the backward's operands: (dev, x shape, M, dy rows,
    dy strides, x rows, x strides, weight segments, residual rows, stride)."""
    dy0 = dy_terms[0]
    _need_gpu(f"{who} grad_out", dy0)
    dev, shape = dy0.device, x_terms[0].shape
    dyr, dys = [], []
    m = None
    for i, t in enumerate(dy_terms):
        _need_gpu(f"{who} grad term {i}", t)
        if t.numel() != dy0.numel():
            raise RuntimeError(f"{who}: grad terms must have the same number of elements")
        tt, rs, m = _as_rows(t, n)
        dyr.append(tt)
        dys.append(rs)
    xr, xs = [], []
    for i, t in enumerate(x_terms):
        _need_gpu(f"{who} input term {i}", t)
        if t.numel() != dy0.numel():
            raise RuntimeError(f"{who}: input and grad must have the same number of elements")
        tt, rs, _ = _as_rows(t, n)
        xr.append(tt)
        xs.append(rs)
    w_seg = (None, n, n)
    if weight is not None:
        _need_gpu(f"{who} weight", weight)
        w_seg = _weight_segments(weight, n)
    res_t, res_s = None, n
    if dx_residual is not None:
        _need_gpu(f"{who} residual", dx_residual)
        res_t, res_s, _ = _as_rows(dx_residual, n)
    return dev, shape, m, dyr, dys, xr, xs, w_seg, res_t, res_s


def _dw_outputs(who, dw, weight, n, dev):
    dw_f32 = dw_bf16 = None
    if dw is not None:
        if weight is None:
            raise RuntimeError(f"{who}: no weight, no weight gradient")
        if dw in ("f32", "f32_bf16"):
            dw_f32 = torch.empty(n, dtype=torch.float32, device=dev)
        elif dw == "bf16":
            dw_bf16 = torch.empty(n, dtype=torch.bfloat16, device=dev)
        else:
            raise ValueError(f"{who}: unknown dw mode {dw!r}")
    return dw_f32, dw_bf16


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
    who = "rms_norm_forward_backward"
    dev, shape, m, dyr, dys, xr, xs, (w_t, seg_len, seg_stride), res_t, res_s = _bwd_operands(
        who, dy_terms, x_terms, weight, n, dx_residual)
    y = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    dx = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    h = torch.empty(shape, dtype=torch.bfloat16, device=dev) if (return_h and len(x_terms) > 1) else None
    rstd = torch.empty(m, dtype=torch.float32, device=dev) if return_rstd else None
    dw_f32, dw_bf16 = _dw_outputs(who, dw, weight, n, dev)
    ws_bytes = int(L.lib().kp_rmsnorm_fwd_bwd_workspace_size(m, n))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    L.call(
        "kp_rmsnorm_fwd_bwd_bf16",
        L.ptr_array([t.data_ptr() for t in dyr]), L.i64_array(dys), len(dyr),
        L.ptr_array([t.data_ptr() for t in xr]), L.i64_array(xs), len(xr),
        _ptr(w_t), seg_len, seg_stride,
        _ptr(h), n, y.data_ptr(), n, _ptr(rstd),
        _ptr(res_t), res_s, dx.data_ptr(), n,
        _ptr(dw_f32), _ptr(dw_bf16), 1 if dw == "f32_bf16" else 0,
        m, n, float(eps), ws.data_ptr(), ws_bytes, _stream(dev),
    )
    out_dw = dw_f32 if dw_f32 is not None else dw_bf16
    if weight is not None and out_dw is not None:
        out_dw = out_dw.view(weight.shape)
    if return_h and h is None:
        h = x_terms[0]
    return y, dx, out_dw, h, rstd


# ---------------------------------------------------------------- embedding
def _index_info(indices: torch.Tensor):
    if indices.device.type != "cuda":
        raise RuntimeError(f"indices must be a GPU tensor, got {indices.device}")
    if indices.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"indices must be int64 or int32, got {indices.dtype}")
    idx = indices.contiguous()
    return idx, idx.element_size()


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
    _need_gpu("embedding_rms_norm table", table)
    if table.dim() != 2:
        raise RuntimeError("embedding_rms_norm: table must be 2-D")
    idx, ib = _index_info(indices)
    V, D = table.shape
    dev = table.device
    tt, trs, _ = _as_rows(table, D)
    T = idx.numel()
    y = torch.empty((*indices.shape, D), dtype=torch.bfloat16, device=dev)
    h = torch.empty_like(y) if return_h else None
    rstd = torch.empty(indices.shape, dtype=torch.float32, device=dev) if return_rstd else None
    w_t, seg_len, seg_stride = (None, D, D)
    if weight is not None:
        _need_gpu("embedding_rms_norm weight", weight)
        w_t, seg_len, seg_stride = _weight_segments(weight, D)
    flag = _flag(dev)
    st = L.lib().kp_embedding_rmsnorm_fwd_bf16(
        tt.data_ptr(), V, trs, idx.data_ptr(), ib, T, _ptr(w_t), seg_len, seg_stride, _ptr(h), D, y.data_ptr(), D,
        _ptr(rstd), D, float(eps), _ptr(flag), _stream(dev))
    if st == L.KP_EUNSUPPORTED:
        emb = embedding(table, indices)
        _, y, r = rms_norm([emb], weight, eps, D, return_rstd=return_rstd)
        return (emb if return_h else None), y, (r.view(indices.shape) if return_rstd else None)
    if st != L.KP_OK:
        raise L.KPError("kp_embedding_rmsnorm_fwd_bf16", st, L.lib().kp_last_error_message().decode())
    _raise_if_flagged(flag, "embedding_rms_norm")
    return h, y, rstd


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
    deterministic sort-and-segment, every row written once."""
    _need_gpu("embedding_dense_backward grad_output", grad_output)
    idx, ib = _index_info(indices)
    T = idx.numel()
    D = grad_output.shape[-1]
    if grad_output.numel() != T * D:
        raise RuntimeError(
            f"embedding_dense_backward: grad_output {tuple(grad_output.shape)} does not match {T} indices")
    g, grs, _ = _as_rows(grad_output, D)
    if out_dtype == torch.float32:
        code = L.KP_DTYPE_F32
    elif out_dtype == torch.bfloat16:
        code = L.KP_DTYPE_BF16
    else:
        raise RuntimeError(f"embedding_dense_backward: unsupported out_dtype {out_dtype}")
    dev = grad_output.device
    out = torch.empty((num_weights, D), dtype=out_dtype, device=dev)
    ws_bytes = int(L.lib().kp_embedding_bwd_workspace_size(T, num_weights, D))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    flag = _flag(dev)
    L.call(
        "kp_embedding_bwd_bf16",
        g.data_ptr(), grs, idx.data_ptr(), ib, T, num_weights, D,
        -1 if padding_idx is None else int(padding_idx), 1 if scale_grad_by_freq else 0,
        out.data_ptr(), code, 1 if round_to_bf16 else 0, ws.data_ptr(), ws_bytes,
        _ptr(flag), _stream(dev),
    )
    _raise_if_flagged(flag, "embedding_dense_backward")
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
    _need_gpu("unshard buffer", flat)
    if flat.dim() == 1:
        if flat.numel() % shards != 0:
            raise RuntimeError(f"unshard: {flat.numel()} elements do not split into {shards} shards")
        row_len = flat.numel() // shards
        if flat.stride(0) != 1 and flat.numel() > 1:
            flat = flat.contiguous()
        stride = row_len
    elif flat.dim() == 2 and flat.shape[0] == shards and (flat.stride(1) == 1 or flat.shape[1] == 1):
        row_len, stride = flat.shape[1], flat.stride(0)
    else:
        raise RuntimeError(f"unshard: expected a 1-D buffer or a [{shards}, L] view, got {tuple(flat.shape)}")
    if sum(split_sizes) != row_len:
        raise RuntimeError(f"unshard: split sizes sum to {sum(split_sizes)}, shard row has {row_len}")
    offs = [0]
    for s in split_sizes:
        offs.append(offs[-1] + s)
    outs = [torch.empty((shards, split_sizes[i]), dtype=torch.bfloat16, device=flat.device) for i in keep]
    for start in range(0, len(outs), 16):
        sel = list(range(start, min(start + 16, len(outs))))
        L.call(
            "kp_unshard_bf16",
            flat.data_ptr(), shards, stride,
            L.i64_array([offs[keep[i]] for i in sel]), L.i64_array([split_sizes[keep[i]] for i in sel]),
            L.ptr_array([outs[i].data_ptr() for i in sel]), len(sel), _stream(flat.device),
        )
    return outs


# ---------------------------------------------------------------- SwiGLU gate
def _same_rows(name: str, ts: Sequence[torch.Tensor]):
    """Views of same-shape bf16 GPU tensors as [rows, N] (unit inner stride)."""
    shape = ts[0].shape
    for i, t in enumerate(ts):
        _need_gpu(f"{name} operand {i}", t)
        if t.numel() != ts[0].numel() or (t.dim() and t.shape[-1] != shape[-1]):
            raise RuntimeError(f"{name}: operand {i} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        if t.device != ts[0].device:
            raise RuntimeError(f"{name}: operands on different devices")
    n = shape[-1] if len(shape) else 1
    if n == 0 or ts[0].numel() == 0:
        return [(t, max(n, 1), 0) for t in ts], n
    return [_as_rows(t, n) for t in ts], n


def swiglu(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """bf16(bf16(silu(a)) * b): the silu -> mul region between the w1/w3 and
    w2 projections of a feed-forward block (v8/c68dae22972b/problem.py:15-28),
    fp32 arithmetic (silu = a / (1 + exp(-a))).  Returns a contiguous tensor
    of a's shape."""
    (ra, rb), n = _same_rows("swiglu", [a, b])
    out = torch.empty(a.shape, dtype=torch.bfloat16, device=a.device)
    m = ra[2]
    if m:
        L.call("kp_swiglu_fwd_bf16", ra[0].data_ptr(), ra[1], rb[0].data_ptr(), rb[1], out.data_ptr(), n, m, n,
               _stream(a.device))
    return out


def swiglu_backward(g: torch.Tensor, s: torch.Tensor, b: torch.Tensor, a: torch.Tensor):
    """Gradients of the SwiGLU gate out = s * b, s = silu(a), given g = dout
    (v8/385e1beb9bb9/problem.py:17-33): db = bf16(g * s) and
    da = silu_backward(bf16(g * b), a) = t * sig * (1 + a * (1 - sig)).
    s is the recomputed silu(a) the graph keeps.  Returns contiguous
    (db, da) of g's shape."""
    (rg, rs, rb, ra), n = _same_rows("swiglu_backward", [g, s, b, a])
    db = torch.empty(g.shape, dtype=torch.bfloat16, device=g.device)
    da = torch.empty(g.shape, dtype=torch.bfloat16, device=g.device)
    m = rg[2]
    if m:
        L.call("kp_swiglu_bwd_bf16", rg[0].data_ptr(), rg[1], rs[0].data_ptr(), rs[1], rb[0].data_ptr(), rb[1],
               ra[0].data_ptr(), ra[1], db.data_ptr(), n, da.data_ptr(), n, m, n, _stream(g.device))
    return db, da


def silu(a: torch.Tensor) -> torch.Tensor:
    """bf16(silu(a)) alone (v7/58e7a4d6cde3/problem.py:10-19), the same bits as
    eager's bf16 silu.  Returns a contiguous tensor of a's shape."""
    (ra,), n = _same_rows("silu", [a])
    out = torch.empty(a.shape, dtype=torch.bfloat16, device=a.device)
    m = ra[2]
    if m:
        L.call("kp_silu_bf16", ra[0].data_ptr(), ra[1], out.data_ptr(), n, m, n, _stream(a.device))
    return out


def swiglu_forward_backward(a: torch.Tensor, b: torch.Tensor, g: torch.Tensor):
    """The SwiGLU gate forward recomputed with its backward in one pass
    (v6/182d2dcd0652/problem.py:10-46): with s = bf16(silu(a)) kept in
    registers, h = bf16(s * b), db = bf16(g * s) and
    da = silu_backward(bf16(g * b), a).  Returns contiguous (h, db, da)."""
    (ra, rb, rg), n = _same_rows("swiglu_forward_backward", [a, b, g])
    h, db, da = (torch.empty(a.shape, dtype=torch.bfloat16, device=a.device) for _ in range(3))
    m = ra[2]
    if m:
        L.call("kp_swiglu_fwd_bwd_bf16", ra[0].data_ptr(), ra[1], rb[0].data_ptr(), rb[1], rg[0].data_ptr(), rg[1],
               h.data_ptr(), n, db.data_ptr(), n, da.data_ptr(), n, m, n, _stream(a.device))
    return h, db, da


# ---------------------------------------------------------------- cross-entropy
def _targets(targets: torch.Tensor, M: int, device: torch.device):
    if not isinstance(targets, torch.Tensor) or targets.device != device:
        raise RuntimeError("cross_entropy: targets must be a tensor on the logits' device")
    if targets.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"cross_entropy: targets must be int64 or int32, got {targets.dtype}")
    if targets.numel() != M:
        raise RuntimeError(f"cross_entropy: {targets.numel()} targets for {M} rows")
    t = targets.reshape(-1)
    if M > 1 and t.stride(0) != 1:
        t = t.contiguous()
    return t, t.element_size()


def cross_entropy_loss(logits: torch.Tensor, targets: torch.Tensor, *, ignore_index: int = -100, scale: float = 1.0,
                       return_lse: bool = False):
    """Summed token cross-entropy of bf16 logits [..., V] against integer
    targets [...]: loss = scale * sum over rows with target != ignore_index of
    (logsumexp(fp32 logits) - logit[target]), the fp32 _log_softmax ->
    nll_loss_forward(reduction sum) -> div region of v8/71f1d2c9f38b/problem.py:15-40
    without materialising the log-softmax.  Returns 0-dim fp32 tensors
    (loss, total_weight) and, with return_lse, the fp32 per-row logsumexp."""
    _need_gpu("cross_entropy logits", logits)
    dev = logits.device
    V = logits.shape[-1] if logits.dim() else 1
    lt, rs, M = _as_rows(logits, V)
    t, tb = _targets(targets, M, dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    tw = torch.empty((), dtype=torch.float32, device=dev)
    lse = torch.empty(logits.shape[:-1], dtype=torch.float32, device=dev) if return_lse else None
    ws_bytes = int(L.lib().kp_cross_entropy_fwd_workspace_size(M))
    ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
    flag = _flag(dev)
    L.call("kp_cross_entropy_fwd_bf16", lt.data_ptr(), rs, M, V, t.data_ptr(), tb, int(ignore_index), float(scale),
           loss.data_ptr(), tw.data_ptr(), _ptr(lse), _ptr(flag), ws.data_ptr(), ws_bytes, _stream(dev))
    _raise_if_flagged(flag, "cross_entropy")
    return (loss, tw, lse) if return_lse else (loss, tw)


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
    _need_gpu("cross_entropy logits", logits)
    dev = logits.device
    V = logits.shape[-1] if logits.dim() else 1
    lt, rs, M = _as_rows(logits, V)
    t, tb = _targets(targets, M, dev)
    if in_place:
        if not logits.is_contiguous():
            raise RuntimeError("cross_entropy_forward_backward: in_place needs contiguous logits")
        out = logits
    else:
        out = torch.empty(logits.shape, dtype=torch.bfloat16, device=dev)
    loss = tw = None
    ws, ws_bytes = None, 0
    if return_loss:
        loss = torch.empty((), dtype=torch.float32, device=dev)
        tw = torch.empty((), dtype=torch.float32, device=dev)
        ws_bytes = int(L.lib().kp_cross_entropy_fwd_workspace_size(M))
        ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
    flag = _flag(dev)
    L.call("kp_cross_entropy_fwd_bwd_bf16", lt.data_ptr(), rs, M, V, t.data_ptr(), tb, int(ignore_index),
           float(grad_loss), out.data_ptr(), V, float(scale), _ptr(loss), _ptr(tw), _ptr(flag), _ptr(ws), ws_bytes,
           _stream(dev))
    _raise_if_flagged(flag, "cross_entropy_forward_backward")
    return (out, loss, tw) if return_loss else out


def cross_entropy_backward(log_softmax: torch.Tensor, targets: torch.Tensor, grad_loss: float, *,
                           ignore_index: int = -100) -> torch.Tensor:
    """Gradient of the summed cross-entropy w.r.t. the logits, in bf16, from
    the saved fp32 log-softmax L [..., V]: out = grad - exp(L) * sum(grad) with
    grad = -grad_loss at each non-ignored row's target
    (v8/622c35f5d1c6/problem.py:16-33: nll_loss_backward(sum) ->
    _log_softmax_backward_data -> _to_copy(bf16)).  grad_loss is the
    upstream gradient of the loss as a Python float (a constant in the
    fragment: 1 / 8192).  Returns a contiguous bf16 tensor of L's shape."""
    _need_gpu("cross_entropy log_softmax", log_softmax, torch.float32)
    dev = log_softmax.device
    V = log_softmax.shape[-1] if log_softmax.dim() else 1
    lt, rs, M = _as_rows(log_softmax, V)
    t, tb = _targets(targets, M, dev)
    out = torch.empty(log_softmax.shape, dtype=torch.bfloat16, device=dev)
    flag = _flag(dev)
    if M:
        L.call("kp_cross_entropy_bwd_bf16", lt.data_ptr(), rs, t.data_ptr(), tb, int(ignore_index), float(grad_loss),
               out.data_ptr(), V, M, V, _ptr(flag), _stream(dev))
    _raise_if_flagged(flag, "cross_entropy_backward")
    return out
