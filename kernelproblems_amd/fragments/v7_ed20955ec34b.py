"""RMSNorm backward of the first layer's attention norm with a three-term
gradient: v7/ed20955ec34b/problem.py:10-44 (inputs :47-55).
dy = bf16(bf16(view_1794 + mm_672) + mm_674), out = bf16(add_220 + dx),
dw = fp32(bf16 weight gradient)."""
import torch

from .. import fused as F
from ._common import EPS, randn


def get_inputs(device="cuda", generator=None):
    return [randn([8192, 4096], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator),
            randn([8192, 4096], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator),
            randn([1, 8192, 1], dtype=torch.float32, device=device, generator=generator),
            randn([4096], device=device, generator=generator),
            randn([1, 8192, 4096], device=device, generator=generator)]


def kernel_function(mm_672, view_1794, mm_674, embedding, getitem_1_recomputed, _unsafe_view_432, add_220):
    n = embedding.shape[-1]
    out, dw = F.rms_norm_backward([view_1794, mm_672, mm_674], [embedding], getitem_1_recomputed, _unsafe_view_432,
                                  EPS, n, dx_residual=add_220, dw="f32_bf16")
    return out, dw
