"""Shared pieces of the per-fragment drop-ins.

Every RMSNorm fragment of the reference normalizes the last dim (4096) with
eps=1e-05 (e.g. v7/59f786beb25f/problem.py:16), and every per-layer FSDP flat
parameter buffer is 8 shards of 27264000 bf16 split as LAYER_SPLITS
(v8/94985bdb7630/problem.py:18): attention_norm.weight, wq, wk, wv, wo,
ffn_norm.weight, w1, w2, w3 of one Llama-3-8B layer.
"""
from __future__ import annotations

import torch

EPS = 1e-05
SHARDS = 8
LAYER_SPLITS = (512, 2097152, 524288, 524288, 2097152, 512, 7340032, 7340032, 7340032)
LAYER_SHAPES = ((4096,), (4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (4096,),
                (14336, 4096), (14336, 4096), (14336, 4096))


def randn(shape, dtype=torch.bfloat16, device="cuda", generator=None) -> torch.Tensor:
    return torch.randn(shape, dtype=dtype, device=device, generator=generator)


def randint(high, shape, dtype=torch.int64, device="cuda", generator=None) -> torch.Tensor:
    return torch.randint(0, high, shape, dtype=dtype, device=device, generator=generator)


def strided_randn(numel, shape, stride, device="cuda", generator=None) -> torch.Tensor:
    return randn((numel,), device=device, generator=generator).as_strided(shape, stride)


def rows2d(t: torch.Tensor) -> torch.Tensor:
    """[..., N] -> [M, N] view (the fragments' aten.view(t, [8192, 4096]))."""
    return t.view(-1, t.shape[-1])


def rstd_view(rstd: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """rstd as _fused_rms_norm returns it: x.shape[:-1] + [1], fp32."""
    return rstd.view(*x.shape[:-1], 1)


def layer_norm_weight(flat: torch.Tensor, index: int = 0) -> torch.Tensor:
    """The [8, 512] row-strided view of norm weight ``index`` (0 or 5) inside a
    per-layer flat buffer; the kernels read it in place, no clone."""
    rows = flat.view(SHARDS, -1)
    off = sum(LAYER_SPLITS[:index])
    return rows[:, off:off + LAYER_SPLITS[index]]


def norm_saved(x: torch.Tensor, w: torch.Tensor, eps: float = EPS):
    """The (y, rstd) tuple _fused_rms_norm returns for x, w, eps -- the saved
    forward a backward-only fragment receives as its first input (e.g.
    v8/43f0c930291e/problem.py:12,21: only element [1], rstd [..., 1] fp32, is
    read).  Input synthesis only: plain torch fp32 ops, not this package's
    kernels."""
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * rstd * w.float()).to(torch.bfloat16), rstd
