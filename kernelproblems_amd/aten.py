"""Drop-ins for the aten operators the reference fragments are built from.

Same names, argument meaning, output shapes and dtypes as the torch
operators called in the reference's ``problem.py`` files (see each
docstring), computed by the gfx950 kernels.  Only bfloat16 data is
implemented (every reference fragment on this path is bf16); other dtypes
raise.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import fused


def _norm_numel(x: torch.Tensor, normalized_shape: Sequence[int]) -> int:
    k = len(normalized_shape)
    if k == 0 or list(x.shape[x.dim() - k:]) != list(normalized_shape):
        raise RuntimeError(
            f"normalized_shape {list(normalized_shape)} does not match the trailing dims of {list(x.shape)}")
    return math.prod(normalized_shape)


def _rstd_shape(x: torch.Tensor, normalized_shape: Sequence[int]) -> List[int]:
    k = len(normalized_shape)
    return list(x.shape[: x.dim() - k]) + [1] * k


def _fused_rms_norm(
    input: torch.Tensor,
    normalized_shape: Sequence[int],
    weight: Optional[torch.Tensor],
    eps: Optional[float],
) -> Tuple[torch.Tensor, torch.Tensor]:
    """aten._fused_rms_norm(input, normalized_shape, weight, eps) -> (out, rstd).

    As called at v7/59f786beb25f/problem.py:16; semantics of
    torch/_decomp/decompositions.py:1760-1812 (fp32 compute, one rounding of
    x * rstd * w to bf16, rstd fp32 with trailing dims kept as 1).
    """
    n = _norm_numel(input, normalized_shape)
    if eps is None:
        eps = torch.finfo(torch.float32).eps
    _, y, rstd = fused.rms_norm([input], weight, eps, n, return_rstd=True)
    return y, rstd.view(_rstd_shape(input, normalized_shape))


def _fused_rms_norm_backward(
    grad_out: torch.Tensor,
    input: torch.Tensor,
    normalized_shape: Sequence[int],
    rstd: torch.Tensor,
    weight: Optional[torch.Tensor],
    output_mask: Sequence[bool],
) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """aten._fused_rms_norm_backward(grad_out, input, normalized_shape, rstd,
    weight, output_mask) -> (grad_input, grad_weight), both in input's dtype.

    As called at v7/45990c83cfd6/problem.py:23; semantics of
    torch/_decomp/decompositions.py:1815-1887.
    """
    n = _norm_numel(input, normalized_shape)
    want_dx = bool(output_mask[0])
    want_dw = bool(output_mask[1]) and weight is not None
    if input.numel() == 0:
        dx = torch.zeros_like(input) if want_dx else None
        dw = torch.zeros(input.shape[input.dim() - len(normalized_shape):], dtype=input.dtype,
                         device=input.device) if want_dw else None
        return dx, dw
    dx, dw = fused.rms_norm_backward(
        [grad_out], [input], rstd, weight, 0.0, n, want_dx=want_dx, dw="bf16" if want_dw else None)
    return dx, dw


def embedding(
    weight: torch.Tensor,
    indices: torch.Tensor,
    padding_idx: int = -1,
    scale_grad_by_freq: bool = False,
    sparse: bool = False,
) -> torch.Tensor:
    """aten.embedding(weight, indices, ...) -> weight[indices] (v7/1e49beb8a123/problem.py:23)."""
    return fused.embedding(weight, indices)


def embedding_dense_backward(
    grad_output: torch.Tensor,
    indices: torch.Tensor,
    num_weights: int,
    padding_idx: int,
    scale_grad_by_freq: bool,
) -> torch.Tensor:
    """aten.embedding_dense_backward(...) -> [num_weights, D] in grad_output's
    dtype (bf16), accumulated in fp32 (v7/a12a160cb11b/problem.py:16;
    torch/_decomp/decompositions.py:1245-1275).  Any token count below 2^31
    and any vocabulary (2^21 ids or more run one sort pass per slab of the
    vocabulary)."""
    return fused.embedding_dense_backward(
        grad_output, indices, num_weights, padding_idx, scale_grad_by_freq, out_dtype=torch.bfloat16)
