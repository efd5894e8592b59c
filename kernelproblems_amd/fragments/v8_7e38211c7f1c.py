"""RoPE backward of k with the attention backward's gradients passed as a
tuple: v8/7e38211c7f1c/problem.py:10-43 (64 instances per step).

getitem = _scaled_dot_product_flash_attention_backward_31[1], the k gradient
[1, 8, 8192, 128] with [S, H, D] memory order (strides [8388608, 128, 1024,
1]); transpose(1, 2) -> complex multiply by clone_62 (already the conjugated
per-position table, [1, 8192, 1, 64] complex64) -> bf16 -> [8192, 1024] view:
the rotation of v7/5c65f62b0422 in one launch reading the gradient through its
strides.  The reference's own get_inputs hands a 0-dim tensor where the graph
passes the tuple; get_inputs here builds (grad_q, grad_k, grad_v) with the
attention backward's layouts."""
import torch

from ._common import randn, strided_randn
from .v7_5c65f62b0422 import kernel_function as _rope_k_backward


def get_inputs(device="cuda", generator=None):
    gq = strided_randn(33554432, [1, 32, 8192, 128], [33554432, 128, 4096, 1], device=device, generator=generator)
    gk = strided_randn(8388608, [1, 8, 8192, 128], [8388608, 128, 1024, 1], device=device, generator=generator)
    gv = strided_randn(8388608, [1, 8, 8192, 128], [8388608, 128, 1024, 1], device=device, generator=generator)
    return [(gq, gk, gv), randn([1, 8192, 1, 64], dtype=torch.complex64, device=device, generator=generator)]


def kernel_function(_scaled_dot_product_flash_attention_backward_31, clone_62):
    return _rope_k_backward(_scaled_dot_product_flash_attention_backward_31[1], clone_62)
