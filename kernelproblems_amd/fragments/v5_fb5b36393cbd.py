"""Token cross-entropy forward and backward in one region, from the bf16
logits to their bf16 gradient: v5/fb5b36393cbd/problem.py:10-59 (inputs
:62-65).  The fragment's only output is the gradient, as the transposed
[128256, 8192] view the lm_head weight-gradient matmul reads.  One launch
holds each logits row in registers (lse, then every gradient entry): the
logits are read once and the gradient written once, the fp32 log-softmax is
never stored."""
from .. import fused as F
from ._common import randint, randn

M, V = 8192, 128256


def get_inputs(device="cuda", generator=None):
    return [randint(100, [1, M], device=device, generator=generator),
            randn([M, V], device=device, generator=generator)]


def loss_gradient_t(arg584_1, mm_224):
    return F.cross_entropy_forward_backward(mm_224, arg584_1.view(-1), 1.0 / 8192.0, ignore_index=-100).t()


def kernel_function(arg584_1, mm_224):
    return loss_gradient_t(arg584_1, mm_224)
