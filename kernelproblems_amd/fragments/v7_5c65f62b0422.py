"""RoPE backward of k: v7/5c65f62b0422/problem.py:10-40 (inputs :43-46).
The gradient arrives as a [1, 8, 8192, 128] view with [S, H, D] memory
order; transpose(1, 2) makes it [1, 8192, 8, 128] and the kernel reads it
through those strides.  clone_62 is already the conjugated table, so the
rotation is a plain multiply; the output is an [8192, 1024] view."""
import torch

from ._common import randn, strided_randn
from ._rope import rotate, table_rows


def get_inputs(device="cuda", generator=None):
    return [strided_randn(8388608, [1, 8, 8192, 128], [8388608, 128, 1024, 1], device=device, generator=generator),
            randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator)]


def kernel_function(getitem_642, clone_62):
    out, _ = rotate(getitem_642.transpose(1, 2), freqs=table_rows(clone_62))
    return out.view(out.shape[1], -1)
