"""Pins the oracle's RMSNorm forward/backward (oracle.rmsnorm_fwd / _bwd)
against torch library ops on the CPU, fp64 autograd, torch's own
decomposition of _fused_rms_norm_backward, closed forms and invariants."""
import numpy as np
import pytest
import torch
from torch._decomp import decompositions as dec

import oracle
from tests._util import bf, from_u16, gen, randn_bf16, to_u16, ulp_bf16

aten = torch.ops.aten


def _inputs(M, N, seed, wstd=0.02):
    g = gen(seed)
    x = randn_bf16((M, N), g)
    w = randn_bf16((N,), g, mean=1.0, std=wstd)
    dy = randn_bf16((M, N), g)
    return x, w, dy


@pytest.mark.parametrize("M,N,eps", [(64, 256, 1e-5), (33, 96, 1e-6), (8, 4096, 1e-5)])
def test_fwd_matches_torch_fused_rms_norm(M, N, eps):
    x, w, _ = _inputs(M, N, M + N)
    y_t, r_t = aten._fused_rms_norm.default(x, [N], w, eps)
    _, y, r = oracle.rmsnorm_fwd([to_u16(x)], to_u16(w), eps, N)
    # rstd: torch accumulates in fp32, the oracle in fp64 -> within a few fp32 ulps
    np.testing.assert_allclose(r, r_t.view(-1).numpy(), rtol=4 * 2.0**-24)
    u = ulp_bf16(y, to_u16(y_t))
    assert u.max() <= 1 and (u == 0).mean() > 0.99


def test_fwd_constant_and_one_hot_rows():
    N, eps = 64, 1e-5
    c = 0.75
    rows = np.zeros((3, N))
    rows[0, :] = c
    rows[1, 5] = -2.5       # one-hot
    rows[2, :] = -c
    x = oracle.f64_to_bf16(rows)
    w = oracle.f64_to_bf16(np.full(N, 1.5))
    _, y, r = oracle.rmsnorm_fwd([x], w, eps, N)
    # constant row: mean(x^2) = c^2; one-hot: a^2 / N
    r_exp = np.array([1 / np.sqrt(c * c + eps), 1 / np.sqrt(2.5**2 / N + eps), 1 / np.sqrt(c * c + eps)])
    np.testing.assert_allclose(r, r_exp, rtol=2.0**-23)
    yv = bf(y)
    np.testing.assert_allclose(yv[0], c * r_exp[0] * 1.5, rtol=2.0**-8)
    np.testing.assert_allclose(yv[2], -c * r_exp[2] * 1.5, rtol=2.0**-8)
    assert yv[1, 5] == pytest.approx(-np.sqrt(N) * 1.5, rel=2.0**-8)
    assert np.count_nonzero(yv[1]) == 1


def test_fwd_unit_weight_norm():
    """w = 1, eps -> 0: every output row has ||y||^2 = N up to bf16 rounding."""
    x, _, _ = _inputs(16, 512, 3)
    _, y, _ = oracle.rmsnorm_fwd([to_u16(x)], None, 1e-12, 512)
    ss = (bf(y) ** 2).sum(axis=1)
    np.testing.assert_allclose(ss, 512, rtol=2 * 2.0**-8)


def test_fwd_residual_terms_and_segmented_weight():
    """h is torch's bf16 add chain bit for bit; a segmented (FSDP view) weight
    gives the same y as its contiguous copy."""
    M, N = 24, 512
    g = gen(4)
    a, b, c = (randn_bf16((M, N), g) for _ in range(3))
    flat = randn_bf16((4, 1000), g, mean=1.0, std=0.02)
    wv = flat[:, 16:16 + 128]          # 4 shards x 128 = 512 weights
    # the segmented weight starts at the view's first element (offset 16)
    h2, y2, r2 = oracle.rmsnorm_fwd([to_u16(a), to_u16(b), to_u16(c)], to_u16(flat.reshape(-1)[16:]), 1e-5, N,
                                    w_seg=(128, 1000))
    hs = (a + b) + c
    assert np.array_equal(h2, to_u16(hs))
    y_t, _ = aten._fused_rms_norm.default(hs, [N], wv.contiguous().view(-1), 1e-5)
    u = ulp_bf16(y2, to_u16(y_t))
    assert u.max() <= 1 and (u == 0).mean() > 0.99
    _, y3, _ = oracle.rmsnorm_fwd([to_u16(hs)], to_u16(wv.contiguous().view(-1)), 1e-5, N)
    assert np.array_equal(y2, y3)


@pytest.mark.parametrize("M,N", [(16, 64), (7, 320)])
def test_bwd_matches_fp64_autograd(M, N):
    x, w, dy = _inputs(M, N, 10 + N, wstd=0.3)
    eps = 1e-5
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    y = torch.nn.functional.rms_norm(xd, [N], wd, eps)
    y.backward(dy.double())
    dx, dw, r = oracle.rmsnorm_bwd([to_u16(dy)], [to_u16(x)], None, to_u16(w), eps, N)
    # the oracle uses the fp32-rounded rstd (relative 2^-24), then one bf16 rounding
    ex = xd.grad.numpy()
    scale = np.abs(ex).max()
    assert np.all(np.abs(bf(dx) - ex) <= 2.0**-8 * np.abs(ex) + 1e-6 * scale)
    # dw = sum_rows dy * x * rstd: the fp32 rstd's relative error bounds the
    # error by 2^-23 sum_rows |dy * x * rstd| (cancellation makes rtol useless)
    mag = (np.abs(dy.double().numpy() * x.double().numpy()) * r[:, None].astype(np.float64)).sum(0)
    assert np.all(np.abs(dw - wd.grad.numpy()) <= 2.0**-23 * mag + 1e-12)


def test_bwd_given_rstd_matches_torch_decomposition():
    """rstd passed in (not recomputed, any sign), as the v8/d8f596b3df34
    fragment does: torch's decomposition of _fused_rms_norm_backward in fp64."""
    M, N = 12, 256
    x, w, dy = _inputs(M, N, 21, wstd=0.5)
    rstd = torch.randn(M, generator=gen(22))
    dx_t, dw_t = dec._fused_rms_norm_backward(dy.double(), x.double(), [N], rstd.double().view(M, 1), w.double(),
                                              [True, True])
    dx, dw, _ = oracle.rmsnorm_bwd([to_u16(dy)], [to_u16(x)], rstd.numpy(), to_u16(w), 1e-5, N)
    ex = dx_t.numpy()
    assert np.all(np.abs(bf(dx) - ex) <= 2.0**-8 * np.abs(ex) + 1e-9 * np.abs(ex).max())
    np.testing.assert_allclose(dw, dw_t.numpy(), rtol=1e-12, atol=1e-12 * np.abs(dw).max())


def test_bwd_unit_weight_orthogonality():
    """w = 1, eps -> 0: sum_j xhat_j dx_j = 0 for every row (dx is orthogonal
    to x); the bf16 rounding of dx bounds the residual."""
    M, N = 8, 1024
    x, _, dy = _inputs(M, N, 30)
    dx, _, r = oracle.rmsnorm_bwd([to_u16(dy)], [to_u16(x)], None, None, 1e-12, N)
    xh = x.double().numpy() * r[:, None]
    prod = xh * bf(dx)
    assert np.all(np.abs(prod.sum(1)) <= 2.0**-8 * np.abs(prod).sum(1))


def test_bwd_gradient_terms_and_residual_epilogue():
    """dy = bf16(a + b + c) in torch's add order and out = bf16(res + bf16(dx)),
    bit for bit against torch's bf16 adds on the oracle's own dx."""
    M, N = 10, 128
    g = gen(40)
    x, a, b, c, res = (randn_bf16((M, N), g) for _ in range(5))
    w = randn_bf16((N,), g, mean=1.0, std=0.1)
    dyt = (a + b) + c
    dx1, dw1, _ = oracle.rmsnorm_bwd([to_u16(a), to_u16(b), to_u16(c)], [to_u16(x)], None, to_u16(w), 1e-5, N)
    dx2, dw2, _ = oracle.rmsnorm_bwd([to_u16(dyt)], [to_u16(x)], None, to_u16(w), 1e-5, N)
    assert np.array_equal(dx1, dx2) and np.array_equal(dw1, dw2)
    out, _, _ = oracle.rmsnorm_bwd([to_u16(dyt)], [to_u16(x)], None, to_u16(w), 1e-5, N, dx_residual=to_u16(res))
    assert np.array_equal(out, to_u16(res + from_u16(dx2)))


def test_bwd_recomputed_rstd_equals_forward_rstd():
    x, w, dy = _inputs(9, 200, 50)
    _, _, r_f = oracle.rmsnorm_fwd([to_u16(x)], to_u16(w), 1e-5, 200)
    _, _, r_b = oracle.rmsnorm_bwd([to_u16(dy)], [to_u16(x)], None, to_u16(w), 1e-5, 200)
    assert np.array_equal(r_f, r_b)
