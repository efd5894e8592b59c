"""Helpers of the RoPE drop-ins: interleaved complex pairs (2i, 2i+1)
multiplied by a complex64 table, as the reference's
_to_copy -> view_as_complex -> mul -> view_as_real -> _to_copy chains
(e.g. v8/c8c60d8f7015/problem.py:18-71)."""
from __future__ import annotations

import torch

from .. import fused as F


def heads(t: torch.Tensor, head_dim: int = 128) -> torch.Tensor:
    """[S, H*D] or [1, S, H*D] -> [1, S, H, D] view (aten.view(.., [1, S, -1, 128]))."""
    return t.view(1, t.shape[-2], -1, head_dim)


def table_rows(freqs: torch.Tensor) -> torch.Tensor:
    """A complex table broadcast as [1, S, 1, D/2] (one row per position),
    viewed as [S, D/2]."""
    if freqs.dim() == 4 and (freqs.shape[0] != 1 or freqs.shape[2] != 1):
        raise RuntimeError(f"rope: table must broadcast as [1, S, 1, D/2], got {tuple(freqs.shape)}")
    return freqs.reshape(-1, freqs.shape[-1])


def rotate(x, k=None, *, freqs, positions=None, q_dtype=torch.bfloat16, k_dtype=torch.bfloat16, copies=False):
    return F.rope(x, k, positions=positions, freqs_cis=freqs, pairing="interleaved",
                  q_dtype=q_dtype, k_dtype=k_dtype, copies=copies)
