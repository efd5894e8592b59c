"""RoPE forward of q (32 heads): v8/493cad38cac9/problem.py:10-37 (inputs
:40-43)."""
import torch

from ._common import randn
from ._rope import heads, rotate, table_rows


def get_inputs(device="cuda", generator=None):
    return [randn([8192, 4096], device=device, generator=generator),
            randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator)]


def kernel_function(mm_217, view_788):
    out, _ = rotate(heads(mm_217), freqs=table_rows(view_788))
    return out
