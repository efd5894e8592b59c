"""Token cross-entropy backward, nll_loss_backward -> _log_softmax_backward_data
-> _to_copy(bf16): v8/622c35f5d1c6/problem.py:10-33 (inputs :36-41).

The upstream gradient is ones_like(div) / 8192 -- a constant, so div's value
and total_weight (getitem_419, unused by the sum reduction) are not read.
Returns the bf16 [8192, 128256] logits gradient from one streaming launch
over the saved fp32 log-softmax."""
import torch

from .. import fused as F
from ._common import randint, randn

M, V = 8192, 128256


def get_inputs(device="cuda", generator=None):
    return [randn([], dtype=torch.float32, device=device, generator=generator),
            randn([M, V], dtype=torch.float32, device=device, generator=generator),
            randint(100, [M], device=device, generator=generator),
            randn([], dtype=torch.float32, device=device, generator=generator)]


def kernel_function(div, _log_softmax, view_805, getitem_419):
    return F.cross_entropy_backward(_log_softmax, view_805, 1.0 / 8192.0, ignore_index=-100)
