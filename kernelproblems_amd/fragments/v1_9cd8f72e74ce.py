"""Complex RoPE backward of q: the gradient viewed as complex64 times the
(already conjugated) table, row s for position s:
v1/9cd8f72e74ce/problem.py:8-16 (inputs :19-22).  The fragment's clone of
the table is read in place."""
import torch

from .. import fused as F
from ._common import randn


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randn([1, 8192, 1, 64], dtype=torch.complex64, **kw), randn([1, 8192, 32, 64], dtype=torch.complex64, **kw)]


def kernel_function(_conj_63, view_as_complex_127):
    out, _ = F.rope_complex(view_as_complex_127, freqs_cis=_conj_63)
    return out
