"""RoPE of q and k with position-gathered table: v7/0f38bc55457c/problem.py:10-66
(inputs :69-74).  This fragment returns the q rotation in fp32 (the
view_as_real result, never cast: :64-66) and k in bf16."""
import torch

from ._common import randint, randn
from ._rope import heads, rotate


def get_inputs(device="cuda", generator=None):
    return [randn([8192, 4096], device=device, generator=generator),
            randn([8192, 1024], device=device, generator=generator),
            randint(100, [1, 8192], dtype=torch.int32, device=device, generator=generator),
            randn([8192, 64], dtype=torch.complex64, device=device, generator=generator)]


def kernel_function(mm, mm_1, arg586_1, arg582_1):
    return rotate(heads(mm), heads(mm_1), freqs=arg582_1, positions=arg586_1.view(1, -1),
                  q_dtype=torch.float32)
