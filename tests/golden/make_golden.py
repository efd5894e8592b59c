"""Writes tests/golden/golden.npz: small seeded inputs and their expected
outputs, computed here with torch library ops in float64 (F.rms_norm and
its autograd, torch's decomposition of _fused_rms_norm_backward, index_add_,
torch.polar / complex multiply with torchtitan's frequency formula, silu and
the autograd of x * sigmoid(x), log_softmax / nll_loss and their backward
ops) and one correctly rounded bf16 conversion
per rounding point of the reference op sequence.  None of it calls the oracle or the HIP
kernels, which tests/test_golden.py checks against these vectors.

Run from the repository root:  python -m tests.golden.make_golden
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
from torch._decomp import decompositions as dec

from tests._util import bf16_round_exact, to_u16

OUT = Path(__file__).resolve().parent / "golden.npz"


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _bf(shape, g, mean=0.0, std=1.0):
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def rms_cases(d):
    g = _g(100)
    M, N, eps = 16, 256, 1e-5
    x, res, dy = _bf((M, N), g), _bf((M, N), g), _bf((M, N), g)
    w = _bf((N,), g, mean=1.0, std=0.1)
    h = res + x                                              # eager bf16 add
    for tag, inp in (("rms", x), ("addrms", h)):
        r64 = torch.rsqrt(inp.double().pow(2).mean(-1) + eps)
        r32 = r64.float()
        y64 = inp.double() * r32.double()[:, None] * w.double()
        d[f"{tag}_rstd"] = r32.numpy()
        d[f"{tag}_y"] = bf16_round_exact(y64.numpy()).reshape(M, N)
    d.update(rms_x=to_u16(x), rms_res=to_u16(res), rms_w=to_u16(w), rms_dy=to_u16(dy), rms_h=to_u16(h),
             rms_eps=np.float64(eps))
    # backward, rstd recomputed: fp64 autograd of F.rms_norm
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    torch.nn.functional.rms_norm(xd, [N], wd, eps).backward(dy.double())
    d["rmsbwd_dx"] = xd.grad.numpy()
    d["rmsbwd_dw"] = wd.grad.numpy()
    # backward with a given (arbitrary) rstd: torch's decomposition in fp64
    rstd = torch.randn(M, generator=g)
    dx, dw = dec._fused_rms_norm_backward(dy.double(), x.double(), [N], rstd.double()[:, None], w.double(),
                                          [True, True])
    d.update(rmsbwd_given_rstd=rstd.numpy(), rmsbwd_given_dx=dx.numpy(), rmsbwd_given_dw=dw.numpy())


def embedding_cases(d):
    g = _g(200)
    V, D, T, pad = 64, 48, 300, 3
    table, grad = _bf((V, D), g, std=0.02), _bf((T, D), g)
    ids = torch.cat([torch.randint(0, 8, (T // 2,), generator=g), torch.randint(0, V, (T - T // 2,), generator=g)])
    ids[::17] = pad
    keep = ids != pad
    dense = torch.zeros(V, D, dtype=torch.float64).index_add_(0, ids[keep], grad[keep].double())
    absd = torch.zeros(V, D, dtype=torch.float64).index_add_(0, ids[keep], grad[keep].double().abs())
    d.update(emb_table=to_u16(table), emb_ids=ids.numpy(), emb_grad=to_u16(grad), emb_pad=np.int64(pad),
             emb_fwd=to_u16(table[ids]), emb_bwd=dense.numpy(), emb_bwd_abs=absd.numpy())


def rope_cases(d):
    g = _g(300)
    B, S, H, D, theta = 1, 16, 4, 64, 500000.0
    x = _bf((B, S, H, D), g)
    pos = (torch.arange(S) * 37 % 4096).view(1, S)
    freqs = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = pos[0].float()[:, None] * freqs.float()[None, :]  # fp32 angles
    cs = torch.polar(torch.ones_like(ang, dtype=torch.float64), ang.double())
    c, s = cs.real[None, :, None, :], cs.imag[None, :, None, :]
    x1, x2 = x.double()[..., : D // 2], x.double()[..., D // 2:]
    half = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    P = 32
    table = torch.polar(torch.ones(P, D // 2), torch.rand(P, D // 2, generator=g) * 6.283) * (
        1 + 0.1 * torch.randn(P, D // 2, generator=g))
    tpos = torch.randint(0, P, (1, S), generator=g)
    xc = torch.view_as_complex(x.double().reshape(B, S, H, D // 2, 2).contiguous())
    inter = torch.view_as_real(xc * table.to(torch.complex128)[tpos][:, :, None, :]).reshape(B, S, H, D)
    d.update(rope_x=to_u16(x), rope_pos=pos.numpy(), rope_theta=np.float64(theta), rope_half=half.numpy(),
             rope_table=table.numpy(), rope_tpos=tpos.numpy(), rope_inter=inter.numpy())


def swiglu_cases(d):
    """v8/c68dae22972b (silu -> mul) and v8/385e1beb9bb9 (mul, mul ->
    silu_backward) on a ragged [17, 43] block whose first row holds special
    gate values (zeros, the zero of silu' near -1.2785, saturation, overflow
    of e^-x, infinities)."""
    g = _g(400)
    M, N = 17, 43
    a, b, gr, s = (_bf((M, N), g, std=3.0) for _ in range(4))
    special = torch.tensor([0.0, -0.0, 1.0, -1.0, -1.2785, -1.28, 20.0, -20.0, 88.0, -88.0, 90.0, -90.0, 1e-30,
                            -1e-30, 3e38, -3e38, float("inf"), float("-inf")])
    a[0, : special.numel()] = special.to(torch.bfloat16)
    ad = a.double()
    s16 = bf16_round_exact(torch.nn.functional.silu(ad).numpy()).reshape(M, N)
    sv = torch.from_numpy(s16.view(np.int16)).view(torch.bfloat16).double()
    out = bf16_round_exact((sv * b.double()).numpy())
    t16 = bf16_round_exact((gr.double() * b.double()).numpy()).reshape(M, N)
    t = torch.from_numpy(t16.view(np.int16)).view(torch.bfloat16)
    x = ad.clone().requires_grad_(True)
    (x * torch.sigmoid(x)).backward(t.double())
    d.update(swiglu_a=to_u16(a), swiglu_b=to_u16(b), swiglu_g=to_u16(gr), swiglu_s=to_u16(s),
             swiglu_out=out.reshape(M, N), swiglu_db=bf16_round_exact((gr.double() * s.double()).numpy()).reshape(M, N),
             swiglu_da_exact=x.grad.numpy())


def loss_cases(d):
    """v8/71f1d2c9f38b (log_softmax -> nll_loss sum -> / 8192) and
    v8/622c35f5d1c6 (nll_loss_backward -> _log_softmax_backward_data ->
    bf16) on [6, 333] with an ignored row, through torch's fp64 ops."""
    g = _g(500)
    M, V, scale = 6, 333, 1.0 / 8192
    x = _bf((M, V), g, std=3.0)
    t = torch.randint(0, V, (M,), generator=g)
    t[4] = -100
    lsm64 = torch.log_softmax(x.double(), 1)
    loss = torch.nn.functional.nll_loss(lsm64, t, reduction="sum", ignore_index=-100) * scale
    L = torch.log_softmax(x.float(), 1)                        # the saved fp32 log-softmax
    gi = torch.ops.aten.nll_loss_backward(torch.tensor(scale, dtype=torch.float64), L.double(), t, None, 2, -100,
                                          torch.tensor(float((t != -100).sum()), dtype=torch.float64))
    grad = torch.ops.aten._log_softmax_backward_data(gi, L.double(), 1, torch.float64)
    d.update(xent_x=to_u16(x), xent_t=t.numpy(), xent_scale=np.float64(scale), xent_loss=np.float64(loss.item()),
             xent_tw=np.float64((t != -100).sum().item()), xent_lse=torch.logsumexp(x.double(), 1).numpy(),
             xent_L=L.numpy(), xent_grad=bf16_round_exact(grad.numpy()).reshape(M, V))


def main():
    d = {}
    rms_cases(d)
    embedding_cases(d)
    rope_cases(d)
    swiglu_cases(d)
    loss_cases(d)
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(d)} arrays)")


if __name__ == "__main__":
    main()
