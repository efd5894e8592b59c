"""Complex RoPE of q and k with the table rows gathered by position ids:
v1/075cb40f3d5d/problem.py:8-27 (inputs :30-35).  q [1, 8192, 32, 64] and
k [1, 8192, 8, 64] arrive as complex64; one launch rotates both (the
index(freqs_cis, pos) gather fused), complex64 out."""
import torch

from .. import fused as F
from ._common import randint, randn


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randint(100, [1, 8192], dtype=torch.int32, **kw), randn([8192, 64], dtype=torch.complex64, **kw),
            randn([1, 8192, 32, 64], dtype=torch.complex64, **kw), randn([1, 8192, 8, 64], dtype=torch.complex64, **kw)]


def kernel_function(arg586_1, arg582_1, view_as_complex_60, view_as_complex_61):
    return F.rope_complex(view_as_complex_60, view_as_complex_61, freqs_cis=arg582_1, positions=arg586_1.view(1, -1))
