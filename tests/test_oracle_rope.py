"""Pins the oracle's RoPE: table mode against torch's complex64 multiply
(the reference op chain), theta mode against torchtitan's published
frequency formula evaluated with torch.polar, and the rotation's
invariants (pos 0 is the identity, pair norms preserved, conj inverts,
rotate-half == interleaved up to the fixed pair permutation)."""
import numpy as np
import pytest
import torch

import oracle
from tests._util import bf, gen, randn_bf16, to_u16, ulp_bf16


def _perm_half_to_interleaved(D):
    """Column order that maps rotate-half pairs (i, i + D/2) onto (2i, 2i+1)."""
    h = D // 2
    return np.stack([np.arange(h), np.arange(h) + h], axis=1).reshape(-1)


def test_table_matches_torch_complex_multiply():
    g = gen(1)
    B, S, H, D, P = 1, 40, 4, 128, 64
    x = randn_bf16((B, S, H, D), g)
    freqs = torch.polar(torch.ones(P, D // 2), torch.rand(P, D // 2, generator=g) * 6.28)
    freqs = freqs * (1 + 0.1 * torch.randn(P, D // 2, generator=g))  # not unit modulus, like randn tables
    pos = torch.randint(0, P, (B, S), generator=g)
    out = oracle.rope(to_u16(x), pos.numpy(), pairing="interleaved", freqs=freqs.numpy())
    xc = torch.view_as_complex(x.float().reshape(B, S, H, D // 2, 2))
    ref = torch.view_as_real(xc * freqs[pos][:, :, None, :]).reshape(B, S, H, D).bfloat16()
    u = ulp_bf16(out, to_u16(ref))
    # torch rounds ac - bd in fp32 first; near cancellation that can move a few ulps
    far = (u > 1) & (np.abs(bf(out) - ref.double().numpy()) > 4e-6)
    assert not far.any() and (u == 0).mean() > 0.98


@pytest.mark.parametrize("theta,S", [(10000.0, 64), (500000.0, 4096)])
def test_theta_matches_torchtitan_formula(theta, S):
    """freqs = 1 / theta^(arange(0, D, 2) / D), angles = outer(pos, freqs) in
    fp32, rotate-half pairs (i, i + D/2)."""
    g = gen(2)
    D, H = 128, 2
    x = randn_bf16((1, S, H, D), g)
    freqs = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.outer(torch.arange(S, dtype=torch.float32), freqs.float())
    cs = torch.polar(torch.ones_like(ang, dtype=torch.float64), ang.double())
    x1, x2 = x.double()[..., : D // 2], x.double()[..., D // 2:]
    c, s = cs.real[None, :, None, :], cs.imag[None, :, None, :]
    ref = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1).numpy()
    out = bf(oracle.rope(to_u16(x), None, pairing="half", theta=theta))
    # one bf16 rounding; the angle p * inv_freq agrees to the fp32 rounding
    # of inv_freq (relative 2^-24, i.e. up to p * 2^-24 rad)
    err = np.abs(out - ref)
    tol = 2.0**-8 * np.abs(ref) + (S * 2.0**-23) * np.abs(x.double().numpy()).max() + 1e-30
    assert np.all(err <= tol)


def test_pos_zero_is_identity():
    x = randn_bf16((1, 1, 8, 64), gen(3))
    for pairing in ("half", "interleaved"):
        out = oracle.rope(to_u16(x), np.zeros((1, 1), np.int64), pairing=pairing, theta=10000.0)
        assert np.array_equal(out, to_u16(x))


def test_norm_preserved_and_conj_inverts():
    g = gen(4)
    S, H, D = 300, 4, 64
    x = randn_bf16((1, S, H, D), g)
    pos = np.arange(S, dtype=np.int64) * 13
    y = oracle.rope(to_u16(x), pos, pairing="interleaved", theta=10000.0)
    xv = x.double().numpy().reshape(1, S, H, D // 2, 2)
    yv = bf(y).reshape(1, S, H, D // 2, 2)
    nx, ny = np.hypot(xv[..., 0], xv[..., 1]), np.hypot(yv[..., 0], yv[..., 1])
    assert np.all(np.abs(nx - ny) <= 2 * 2.0**-8 * nx + 1e-30)
    back = oracle.rope(y, pos, pairing="interleaved", theta=10000.0, conj=True)
    assert np.all(np.abs(bf(back) - x.double().numpy()) <= 4 * 2.0**-8 * np.abs(x.double().numpy()).max())


def test_half_equals_interleaved_under_pair_permutation():
    g = gen(5)
    S, H, D = 50, 3, 128
    x = randn_bf16((1, S, H, D), g)
    perm = _perm_half_to_interleaved(D)
    yh = oracle.rope(to_u16(x), None, pairing="half", theta=500000.0)
    yi = oracle.rope(to_u16(x[..., perm].contiguous()), None, pairing="interleaved", theta=500000.0)
    assert np.array_equal(yh[..., perm], yi)


def test_out_of_table_positions():
    x = randn_bf16((1, 3, 2, 8), gen(6))
    freqs = np.ones((4, 4), np.complex64)
    out = oracle.rope(to_u16(x), np.array([[0, 4, -1]]), pairing="interleaved", freqs=freqs)
    assert np.array_equal(out[0, 0], to_u16(x[0, 0])) and not out[0, 1:].any()


def test_c64_matches_torch_complex128_multiply_with_gather():
    """oracle.rope_c64 (v1/075cb40f3d5d): x * table[pos] against torch's
    complex128 multiply of the gathered rows, positions repeated and out of
    order; a transposed or conjugated table would fail it."""
    g = torch.Generator().manual_seed(31)
    B, S, H, P = 2, 6, 3, 8
    x = torch.randn(B, S, H, P, dtype=torch.complex64, generator=g)
    t = torch.randn(10, P, dtype=torch.complex64, generator=g)
    pos = torch.tensor([[3, 3, 0, 9, 1, 5], [9, 8, 7, 6, 5, 4]])
    out = oracle.rope_c64(x.numpy(), t.numpy(), pos.numpy())
    ref = x.to(torch.complex128) * t.to(torch.complex128)[pos][:, :, None, :]
    np.testing.assert_array_equal(out, ref.numpy())
    # default positions: row s for position s
    out2 = oracle.rope_c64(x.numpy(), t.numpy())
    np.testing.assert_array_equal(out2, (x.to(torch.complex128) * t.to(torch.complex128)[:S][None, :, None, :]).numpy())


def test_c64_unit_rows_identity_norm_and_conj():
    g = torch.Generator().manual_seed(32)
    x = torch.randn(1, 5, 2, 16, dtype=torch.complex64, generator=g).numpy()
    ang = torch.rand(5, 16, generator=g).double().numpy() * 6.283
    t = np.exp(1j * ang)
    t[0] = 1.0
    out = oracle.rope_c64(x, t)
    np.testing.assert_array_equal(out[:, 0], x[:, 0].astype(np.complex128))  # position 0, unit row: identity
    np.testing.assert_allclose(np.abs(out), np.abs(x), rtol=1e-6)              # unit modulus keeps |x|
    back = oracle.rope_c64(out, t, conj=True)                                  # conj undoes the rotation
    np.testing.assert_allclose(back, x, rtol=0, atol=1e-6 * np.abs(x).max())
