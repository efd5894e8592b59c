"""Every RMSNorm and RoPE BASELINE configuration at its full size, element by
element, on bench.py's own seed-0 inputs (the same draws in the same order as
bench.py's RmsFwd / RmsBwd / Rope workloads).

Each output element is compared against two references on the GPU:
  * an fp64 evaluation of the fragment's formula with torch (the RMSNorm
    closed forms of torch/_decomp/decompositions.py:1760-1887; RoPE with the
    fp32 angle pos * fp32(theta^(-2i/D)) and fp64 cos / sin of it);
  * torch-ROCm eager, the reference fragment's own ops on this GPU
    (aten._fused_rms_norm, aten._fused_rms_norm_backward, the rotate-half
    chain of oracle/torch_ref.py).
Bars, on every element: the north-star tolerance |a - e| <= 1e-2 + 1.6e-2 |e|
against both references; against fp64, faithful rounding (the output is one
of the two bf16 neighbours of the fp64 value) except where the formula
cancels, where the fp32 evaluation's own error bound 2^-20 * (sum of the
magnitudes of the cancelling terms, plus for dx the fp32 row sum's error
bound) applies; against eager, at most one bf16
ulp for the forward outputs.  The weight gradient is compared with the fp64
column sums (2^-20 of the column's magnitude sum) and with eager's bf16
weight gradient (its own bf16 rounding).
  c1  RMSNorm fwd       x [4096, 4096], eps 1e-6
  c2  RMSNorm bwd       x, dy [8192, 4096], eps 1e-6
  c4  RoPE rotate-half  q [4, 4096, 32, 128], k [4, 4096, 8, 128], positions 0..4095, theta 5e5
  c5f add + RMSNorm fwd x, res [16384, 8192], eps 1e-5
  c5b add + RMSNorm bwd x, res, dy [16384, 8192], eps 1e-5
"""
import pytest
import torch

import kernelproblems_amd as kp
from oracle import torch_ref
from tests._util import BF16_ATOL, BF16_RTOL

pytestmark = pytest.mark.gpu

aten = torch.ops.aten


def _gen0():
    return torch.Generator().manual_seed(0)


def _randn(shape, g, mean=0.0, std=1.0):  # bench.py's _randn: fp32 draws on the CPU, cast to bf16
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def _ulp_key(t):
    """bf16 -> int32 key, monotone in the value (the distance of two keys is
    their distance in bf16 ulps)."""
    u = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    return torch.where(u >= 0x8000, 0x8000 - (u & 0x7FFF), 0x8000 + u)


def _ulps(a, b):
    return (_ulp_key(a) - _ulp_key(b)).abs()


def _bf16_ulp(v64):
    """One bf16 ulp at each fp64 value (8 significant bits; subnormal floor)."""
    _, e = torch.frexp(v64)
    return torch.ldexp(torch.ones_like(v64), (e - 8).clamp(min=-133))


def _north_star(a, e, what):
    d = (a.double() - e.double()).abs()
    bad = d > BF16_ATOL + BF16_RTOL * e.double().abs()
    n = int(bad.sum())
    assert n == 0, f"{what}: {n} of {a.numel()} elements outside rtol={BF16_RTOL} atol={BF16_ATOL} (max |diff| {float(d.max()):.4g})"


def _faithful(a, v64, scale, what):
    """a (bf16) within one bf16 ulp of the fp64 value v64, or within the fp32
    evaluation bound 2^-20 * scale where the formula cancels."""
    d = (a.double() - v64).abs()
    ok = (d < _bf16_ulp(v64)) | (d <= 2.0**-20 * scale)
    n = int((~ok).sum())
    assert n == 0, f"{what}: {n} of {a.numel()} elements neither faithfully rounded nor within the fp32 bound"


def _rstd64(h, eps):
    return torch.rsqrt(h.double().pow(2).mean(-1) + eps)


@pytest.mark.parametrize("cfg", ["c1", "c5f"])
def test_rmsnorm_fwd_every_element(gpu, cfg):
    M, N, eps, residual = (4096, 4096, 1e-6, False) if cfg == "c1" else (16384, 8192, 1e-5, True)
    print(f"[config full] {cfg} [{M},{N}] seed 0", flush=True)
    g = _gen0()
    x = _randn((M, N), g).to(gpu)
    res = _randn((M, N), g).to(gpu) if residual else None
    w = _randn(N, g, 1.0, 0.02).to(gpu)
    terms = [x, res] if residual else [x]
    h, y, r = kp.rms_norm(terms, w, eps, N, return_h=residual, return_rstd=True)
    hh = aten.add.Tensor(res, x) if residual else x  # eager's h (v8/7884328a5557/problem.py:20)
    if residual:
        assert torch.equal(h, hh), "h must be eager's bf16 add bit for bit"
    y_e, r_e = aten._fused_rms_norm.default(hh, [N], w, eps)
    r64 = _rstd64(hh, eps)
    y64 = hh.double() * r64[:, None] * w.double()
    assert float(((r.double() - r64).abs() / r64).max()) < 1e-6
    torch.testing.assert_close(r.view(-1), r_e.view(-1), rtol=1e-5, atol=0)
    _north_star(y, y64, f"{cfg} y vs fp64")
    _north_star(y, y_e, f"{cfg} y vs eager")
    _faithful(y, y64, torch.zeros_like(y64), f"{cfg} y vs fp64")
    u = _ulps(y, y_e)
    assert int(u.max()) <= 1, f"{cfg} y: {int((u > 1).sum())} elements more than 1 ulp from eager"
    print(f"[config full] {cfg}: y bit-equal to eager on {float((u == 0).double().mean()):.5f} of elements", flush=True)


@pytest.mark.parametrize("cfg", ["c2", "c5b"])
def test_rmsnorm_bwd_every_element(gpu, cfg):
    M, N, eps, residual = (8192, 4096, 1e-6, False) if cfg == "c2" else (16384, 8192, 1e-5, True)
    print(f"[config full] {cfg} [{M},{N}] seed 0", flush=True)
    g = _gen0()
    x = _randn((M, N), g).to(gpu)
    res = _randn((M, N), g).to(gpu) if residual else None
    w = _randn(N, g, 1.0, 0.02).to(gpu)
    dy = _randn((M, N), g).to(gpu)
    dx, dw = kp.rms_norm_backward([dy], [x, res] if residual else [x], None, w, eps, N, dw="f32")
    h = aten.add.Tensor(res, x) if residual else x  # v8/3c6c589cdf81/problem.py: h recomputed
    # torch-ROCm eager: rstd from the forward, then the fused backward (dw in bf16)
    _, r_e = aten._fused_rms_norm.default(h, [N], w, eps)
    dx_e, dw_e = aten._fused_rms_norm_backward.default(dy, h, [N], r_e, w, [True, True])
    # fp64: dx = (g - xhat * sum(xhat g) / N) * rstd, g = dy w; dw = sum_rows dy xhat
    r64 = _rstd64(h, eps)[:, None]
    xhat = h.double() * r64
    gg = dy.double() * w.double()
    xg = xhat * gg
    c = xg.sum(1, keepdim=True) / N
    cmag = xg.abs().sum(1, keepdim=True) / N  # bounds the fp32 row sum's error: |dc| <= ~48 * 2^-24 * cmag
    del xg
    dx64 = (gg - xhat * c) * r64
    scale = (gg.abs() + (xhat * c).abs() + 64.0 * xhat.abs() * cmag) * r64
    del gg
    _north_star(dx, dx64, f"{cfg} dx vs fp64")
    _north_star(dx, dx_e, f"{cfg} dx vs eager")
    _faithful(dx, dx64, scale, f"{cfg} dx vs fp64")
    del dx64, scale
    u = _ulps(dx, dx_e)
    print(f"[config full] {cfg}: dx bit-equal to eager on {float((u == 0).double().mean()):.5f} of elements, "
          f"max {int(u.max())} ulp", flush=True)
    dyx = dy.double() * xhat
    dw64, mag = dyx.sum(0), dyx.abs().sum(0)
    assert bool(((dw.double() - dw64).abs() <= 2.0**-20 * mag + 1e-6).all()), f"{cfg} dw vs fp64"
    dwd = (dw.double() - dw_e.double()).abs()
    assert bool((dwd <= 2.0**-7 * dw_e.double().abs() + 2.0**-20 * mag + 1e-6).all()), f"{cfg} dw vs eager's bf16 dw"


def test_rope_every_element(gpu):
    B, S, Hq, Hk, D, theta = 4, 4096, 32, 8, 128, 500000.0
    print("[config full] c4 rope seed 0", flush=True)
    g = _gen0()
    q, k = _randn((B, S, Hq, D), g).to(gpu), _randn((B, S, Hk, D), g).to(gpu)
    pos = torch.arange(S, dtype=torch.int64).expand(B, S).contiguous().to(gpu)
    qo, ko = kp.rope(q, k, positions=pos, theta=theta, pairing="half")
    qe, ke = torch_ref.rope_half(q, k, pos, theta)
    inv = (theta ** (-torch.arange(0, D, 2, dtype=torch.float64, device=gpu) / D)).to(torch.float32)
    ang = (pos.to(torch.float32)[..., None] * inv).double()  # the fp32 angle, exactly
    cos, sin = torch.cos(ang)[:, :, None, :], torch.sin(ang)[:, :, None, :]
    for name, x, o, e in (("q", q, qo, qe), ("k", k, ko, ke)):
        xf = x.double()
        x1, x2 = xf[..., : D // 2], xf[..., D // 2:]
        o64 = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
        scale = torch.cat([(x1 * cos).abs() + (x2 * sin).abs(), (x2 * cos).abs() + (x1 * sin).abs()], dim=-1)
        _north_star(o, o64, f"c4 {name} vs fp64")
        _north_star(o, e, f"c4 {name} vs eager")
        _faithful(o, o64, scale, f"c4 {name} vs fp64")
        u = _ulps(o, e)
        far = (u > 1) & ((o.double() - e.double()).abs() > 2.0**-19 * scale)
        assert int(far.sum()) == 0, f"c4 {name}: {int(far.sum())} elements more than 1 ulp from eager"
        print(f"[config full] c4 {name}: bit-equal to eager on {float((u == 0).double().mean()):.5f} of elements",
              flush=True)
        del o64, scale, u, far
