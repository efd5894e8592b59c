"""Torch eager restatement of the hot-path fragments -- TEST INFRASTRUCTURE ONLY.

Each function restates, with torch eager ops, the aten op sequence of the
reference fragment(s) it cites, for inputs on any device.  On a GPU this is
the "reference torch eager fragment" (torch-ROCm kernels); on the CPU it is
the reference CPU eager path that bench.py times as the cpu_baseline.

``_fused_rms_norm_backward`` has no CPU kernel
(torchgen/packaged/ATen/native/native_functions.yaml:3347-3349), so on the
CPU the backward runs torch's own Python decomposition of that operator
(torch/_decomp/decompositions.py:1815-1887).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch._decomp import decompositions as _dec

aten = torch.ops.aten


def _rms_bwd(dy, x, n, rstd, w):
    if x.device.type == "cuda":
        return aten._fused_rms_norm_backward.default(dy, x, [n], rstd, w, [True, True])
    return _dec._fused_rms_norm_backward(dy, x, [n], rstd, w, [True, True])


def rms_norm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float):
    """C1 / v7/59f786beb25f/problem.py:16-21: _fused_rms_norm -> (y, rstd)."""
    return aten._fused_rms_norm.default(x, [x.shape[-1]], w, eps)


def rms_norm_bwd(x: torch.Tensor, dy: torch.Tensor, w: torch.Tensor, eps: float):
    """C2 / v7/45990c83cfd6/problem.py:17-28: rstd recomputed by the forward,
    _fused_rms_norm_backward, weight gradient widened with _to_copy(f32)
    (v8/d8f596b3df34/problem.py:41-44)."""
    n = x.shape[-1]
    _, rstd = aten._fused_rms_norm.default(x, [n], w, eps)
    dx, dw = _rms_bwd(dy, x, n, rstd, w)
    return dx, dw.to(torch.float32)


def add_rms_norm_fwd(x: torch.Tensor, res: torch.Tensor, w: torch.Tensor, eps: float):
    """C5 forward / v8/7884328a5557/problem.py:20-33: h = add.Tensor(res, x), y = rms(h)."""
    h = aten.add.Tensor(res, x)
    y, _ = aten._fused_rms_norm.default(h, [h.shape[-1]], w, eps)
    return h, y


def add_rms_norm_bwd(x: torch.Tensor, res: torch.Tensor, dy: torch.Tensor, w: torch.Tensor, eps: float):
    """C5 backward / v8/3c6c589cdf81/problem.py:22-53: h recomputed from the
    adds, rstd recomputed, backward, weight gradient to f32."""
    h = aten.add.Tensor(res, x)
    n = h.shape[-1]
    _, rstd = aten._fused_rms_norm.default(h, [n], w, eps)
    dx, dw = _rms_bwd(dy, h, n, rstd, w)
    return dx, dw.to(torch.float32)


def embedding_fwd(table: torch.Tensor, ids: torch.Tensor):
    """C3 forward / v7/1e49beb8a123/problem.py:23."""
    return aten.embedding.default(table, ids)


def embedding_bwd(grad: torch.Tensor, ids: torch.Tensor, num_weights: int, padding_idx: int = -1):
    """C3 backward / v7/a12a160cb11b/problem.py:16-20: embedding_dense_backward then _to_copy(f32)."""
    g = aten.embedding_dense_backward.default(grad, ids, num_weights, padding_idx, False)
    return aten._to_copy.default(g, dtype=torch.float32)


def rope_half(q: torch.Tensor, k: torch.Tensor, positions: Optional[torch.Tensor], theta: float):
    """C4: rotate-half RoPE, inv_freq = theta^(-2i/D) in fp32, angle = pos * inv_freq
    in fp32, cos/sin in fp32, rotation in fp32, output cast to bf16."""
    B, S, _, D = q.shape
    dev = q.device
    inv = (theta ** (-torch.arange(0, D, 2, dtype=torch.float64, device=dev) / D)).to(torch.float32)
    pos = torch.arange(S, device=dev).expand(B, S) if positions is None else positions
    ang = pos.to(torch.float32)[..., None] * inv  # [B, S, D/2]
    cos = torch.cos(ang)[:, :, None, :]
    sin = torch.sin(ang)[:, :, None, :]

    def rot(x):
        xf = x.to(torch.float32)
        x1, x2 = xf[..., : D // 2], xf[..., D // 2:]
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(torch.bfloat16)

    return rot(q), rot(k)


def rope_complex(x: torch.Tensor, freqs_cis: torch.Tensor):
    """Interleaved complex RoPE as in v7/e29b92927600/problem.py:16-37:
    _to_copy f32 -> view_as_complex -> mul(freqs_cis) -> view_as_real -> _to_copy bf16.
    x: [B, S, H, D]; freqs_cis broadcastable to [B, S, 1, D/2]."""
    B, S, H, D = x.shape
    xc = torch.view_as_complex(x.to(torch.float32).reshape(B, S, H, D // 2, 2))
    return torch.view_as_real(xc * freqs_cis).reshape(B, S, H, D).to(torch.bfloat16)


def swiglu_fwd(a: torch.Tensor, b: torch.Tensor):
    """v8/c68dae22972b/problem.py:15-28: silu.default -> mul.Tensor."""
    return aten.mul.Tensor(aten.silu.default(a), b)


def swiglu_bwd(g: torch.Tensor, s: torch.Tensor, b: torch.Tensor, a: torch.Tensor):
    """v8/385e1beb9bb9/problem.py:17-33: mul.Tensor(g, s); silu_backward(mul.Tensor(g, b), a)."""
    return aten.mul.Tensor(g, s), aten.silu_backward.default(aten.mul.Tensor(g, b), a)


def silu(a: torch.Tensor):
    """v7/58e7a4d6cde3/problem.py:10-19: silu.default."""
    return aten.silu.default(a)


def swiglu_fwd_bwd(a: torch.Tensor, b: torch.Tensor, g: torch.Tensor):
    """v6/182d2dcd0652/problem.py:10-46: s = silu(a); (mul(s, b), mul(g, s),
    silu_backward(mul(g, b), a))."""
    s = aten.silu.default(a)
    return aten.mul.Tensor(s, b), aten.mul.Tensor(g, s), aten.silu_backward.default(aten.mul.Tensor(g, b), a)


def cross_entropy_fwd(logits: torch.Tensor, targets: torch.Tensor, scale: float):
    """v8/71f1d2c9f38b/problem.py:15-40: _to_copy(f32) -> _log_softmax ->
    nll_loss_forward(sum, ignore_index=-100) -> div."""
    lsm = aten._log_softmax.default(aten._to_copy.default(logits, dtype=torch.float32), 1, False)
    loss, tw = aten.nll_loss_forward.default(lsm, targets, None, 2, -100)
    return aten.mul.Tensor(loss, scale), tw


def cross_entropy_bwd(lsm: torch.Tensor, targets: torch.Tensor, grad_loss: float):
    """v8/622c35f5d1c6/problem.py:16-33: nll_loss_backward(sum) ->
    _log_softmax_backward_data -> _to_copy(bf16)."""
    g = torch.tensor(grad_loss, dtype=torch.float32, device=lsm.device)
    tw = (targets != -100).sum().to(torch.float32)
    gi = aten.nll_loss_backward.default(g, lsm, targets, None, 2, -100, tw)
    d = aten._log_softmax_backward_data.default(gi, lsm, 1, torch.float32)
    return aten._to_copy.default(d, dtype=torch.bfloat16)


def cross_entropy_fwd_bwd(logits: torch.Tensor, targets: torch.Tensor, grad_loss: float):
    """v5/fb5b36393cbd/problem.py:16-59: _to_copy(f32) -> _log_softmax ->
    nll_loss_forward(sum) -> nll_loss_backward -> _log_softmax_backward_data
    -> _to_copy(bf16)."""
    lsm = aten._log_softmax.default(aten._to_copy.default(logits, dtype=torch.float32), 1, False)
    _, tw = aten.nll_loss_forward.default(lsm, targets, None, 2, -100)
    g = torch.tensor(grad_loss, dtype=torch.float32, device=logits.device)
    gi = aten.nll_loss_backward.default(g, lsm, targets, None, 2, -100, tw)
    d = aten._log_softmax_backward_data.default(gi, lsm, 1, torch.float32)
    return aten._to_copy.default(d, dtype=torch.bfloat16)


def embedding_rms_norm_fwd(table: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, eps: float):
    """v8/12545c1e9b06/problem.py:24-42: embedding.default -> _fused_rms_norm."""
    x = aten.embedding.default(table, ids)
    return aten._fused_rms_norm.default(x, [x.shape[-1]], w, eps)[0]
