"""Complex RoPE backward of k (8 heads): v1/f23f9bb4567a/problem.py:8-16
(inputs :19-22).  As v1/9cd8f72e74ce."""
import torch

from .. import fused as F
from ._common import randn


def get_inputs(device="cuda", generator=None):
    kw = dict(device=device, generator=generator)
    return [randn([1, 8192, 1, 64], dtype=torch.complex64, **kw), randn([1, 8192, 8, 64], dtype=torch.complex64, **kw)]


def kernel_function(_conj_62, view_as_complex_126):
    out, _ = F.rope_complex(view_as_complex_126, freqs_cis=_conj_62)
    return out
