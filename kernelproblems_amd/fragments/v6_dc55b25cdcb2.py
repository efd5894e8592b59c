"""RoPE backward of q: v6/dc55b25cdcb2/problem.py:10-43 (inputs :46-49).
As v6/03d64c25b654 with 32 heads; output [8192, 4096]."""
import torch

from ._common import randn, strided_randn
from ._rope import rotate, table_rows


def get_inputs(device="cuda", generator=None):
    return [randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator),
            strided_randn(33554432, [1, 32, 8192, 128], [33554432, 128, 4096, 1], device=device, generator=generator)]


def kernel_function(_conj_63, getitem_641):
    out, _ = rotate(getitem_641.transpose(1, 2), freqs=table_rows(_conj_63))
    return out.view(out.shape[1], -1)
