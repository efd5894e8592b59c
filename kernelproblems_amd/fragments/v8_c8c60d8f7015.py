"""RoPE forward of q and k with the table gathered by position ids:
v8/c8c60d8f7015/problem.py:10-71 (inputs :74-79).  index(freqs_cis, pos) is
done inside the kernel (one table row read per position, shared by all 40
heads); an out-of-range position yields zeros, and raises when index
checking is enabled."""
import torch

from ._common import randint, randn
from ._rope import heads, rotate


def get_inputs(device="cuda", generator=None):
    return [randint(100, [1, 8192], dtype=torch.int32, device=device, generator=generator),
            randn([8192, 64], dtype=torch.complex64, device=device, generator=generator),
            randn([8192, 4096], device=device, generator=generator),
            randn([8192, 1024], device=device, generator=generator)]


def kernel_function(arg586_1, arg582_1, mm, mm_1):
    return rotate(heads(mm), heads(mm_1), freqs=arg582_1, positions=arg586_1.view(1, -1))
