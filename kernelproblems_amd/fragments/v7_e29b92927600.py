"""RoPE forward of k (8 heads): v7/e29b92927600/problem.py:10-37 (inputs
:40-43).  Row s of the [1, 8192, 1, 64] complex table rotates position s."""
import torch

from ._common import randn
from ._rope import heads, rotate, table_rows


def get_inputs(device="cuda", generator=None):
    return [randn([8192, 1024], device=device, generator=generator),
            randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator)]


def kernel_function(mm_218, view_788):
    out, _ = rotate(heads(mm_218), freqs=table_rows(view_788))
    return out
