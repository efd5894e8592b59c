"""Token cross-entropy forward, _to_copy -> _log_softmax -> nll_loss_forward
(sum, ignore_index -100) -> div: v8/71f1d2c9f38b/problem.py:10-40 (inputs
:43-46).

Returns (loss / 8192, total_weight) as 0-dim fp32 tensors.  The fp32
log-softmax of the [8192, 128256] logits is never materialised: one pass
reads the bf16 logits once."""
from .. import fused as F
from ._common import randint, randn

M, V = 8192, 128256


def get_inputs(device="cuda", generator=None):
    return [randint(100, [1, M], device=device, generator=generator),
            randn([M, V], device=device, generator=generator)]


def kernel_function(arg584_1, mm_224):
    return F.cross_entropy_loss(mm_224, arg584_1.view(-1), ignore_index=-100, scale=1.0 / 8192.0)
