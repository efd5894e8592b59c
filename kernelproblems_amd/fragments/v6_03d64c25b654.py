"""RoPE backward of k: v6/03d64c25b654/problem.py:10-43 (inputs :46-49).
As v7/5c65f62b0422 with the table first; the fragment's clone of the
(already conjugated) table is read in place."""
import torch

from ._common import randn, strided_randn
from ._rope import rotate, table_rows


def get_inputs(device="cuda", generator=None):
    return [randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator),
            strided_randn(8388608, [1, 8, 8192, 128], [8388608, 128, 1024, 1], device=device, generator=generator)]


def kernel_function(_conj_62, getitem_642):
    out, _ = rotate(getitem_642.transpose(1, 2), freqs=table_rows(_conj_62))
    return out.view(out.shape[1], -1)
