"""RoPE backward of q: v7/bfe872e373e4/problem.py:10-40 (inputs :43-46).
As v7/5c65f62b0422 with 32 heads; output [8192, 4096]."""
import torch

from ._common import randn, strided_randn
from ._rope import rotate, table_rows


def get_inputs(device="cuda", generator=None):
    return [strided_randn(33554432, [1, 32, 8192, 128], [33554432, 128, 4096, 1], device=device, generator=generator),
            randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator)]


def kernel_function(getitem_641, clone_63):
    out, _ = rotate(getitem_641.transpose(1, 2), freqs=table_rows(clone_63))
    return out.view(out.shape[1], -1)
