"""RoPE forward of q and k with the table gathered by position ids, returned
twice (the graph rotates q and k once for attention and once more for the
recompute) as [1, H, S, D] transposed views: v5/ca76bd89ec38/problem.py:10-132
(inputs :135-140).  The two pairs are separate tensors, as in the fragment;
one launch reads q and k once and writes both pairs."""
import torch

from ._common import randint, randn
from ._rope import heads, rotate


def get_inputs(device="cuda", generator=None):
    return [randint(100, [1, 8192], dtype=torch.int32, device=device, generator=generator),
            randn([8192, 64], dtype=torch.complex64, device=device, generator=generator),
            randn([8192, 4096], device=device, generator=generator),
            randn([8192, 1024], device=device, generator=generator)]


def rotate_twice(pos, freqs, mm_q, mm_k):
    q, k, q2, k2 = rotate(heads(mm_q), heads(mm_k), freqs=freqs, positions=pos.view(1, -1), copies=True)
    return q.transpose(1, 2), k.transpose(1, 2), q2.transpose(1, 2), k2.transpose(1, 2)


def kernel_function(arg586_1, arg582_1, mm_217, mm_218):
    return rotate_twice(arg586_1, arg582_1, mm_217, mm_218)
