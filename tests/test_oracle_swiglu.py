"""Pins the oracle's SwiGLU (v8/c68dae22972b, v8/385e1beb9bb9): against torch
CPU eager silu / mul / silu_backward (the reference op sequence), against an
independent fp64 evaluation (scipy's expit) over every bf16 gate value,
against central finite differences of silu, and against closed forms.  A
dropped term or flipped sign in either formula (x / (1 + e^x), sig * (1 +
sig), a missing bf16 rounding of silu or of g * b) fails at least one."""
import numpy as np
import pytest
import scipy.special
import torch

import oracle
from tests._util import bf, bf16_round_exact, from_u16, gen, randn_bf16, to_u16, ulp_bf16


def _same_value(a_u16, b_u16):
    """Equal as numbers (+0 == -0, NaN == NaN)."""
    av, bv = bf(a_u16), bf(b_u16)
    return (av == bv) | (np.isnan(av) & np.isnan(bv))


def _all_bf16(finite_only=False):
    pats = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    v = bf(pats)
    keep = ~np.isnan(v) if not finite_only else np.isfinite(v)
    return pats[keep]


def test_fwd_matches_torch_cpu_eager():
    g = gen(11)
    a, b = randn_bf16((64, 999), g, std=3.0), randn_bf16((64, 999), g)
    ref = torch.nn.functional.silu(a) * b           # eager bf16 silu, then bf16 mul
    out = oracle.swiglu_fwd(to_u16(a), to_u16(b))
    u = ulp_bf16(out, to_u16(ref))
    assert u.max() <= 1 and (u == 0).mean() > 0.999


def test_bwd_matches_torch_cpu_eager():
    g = gen(12)
    gr, s, b, a = (randn_bf16((64, 999), g, std=2.0) for _ in range(4))
    db_ref = gr * s
    da_ref = torch.ops.aten.silu_backward(gr * b, a)
    db, da = oracle.swiglu_bwd(to_u16(gr), to_u16(s), to_u16(b), to_u16(a))
    assert np.array_equal(db, to_u16(db_ref))       # one exact product, one rounding
    u = ulp_bf16(da, to_u16(da_ref))
    # torch evaluates 1 + a (1 - sig) in fp32; near silu's stationary point
    # (a ~ -1.2785) that cancellation leaves an absolute error ~ |t| 2^-23
    near_zero = np.abs(bf(to_u16(da_ref))) < 1e-5 * np.abs(bf(to_u16(gr * b))) + 1e-30
    assert (u[~near_zero] <= 1).all() and (u == 0).mean() > 0.999


def test_fwd_every_bf16_gate_value_fp64():
    """b = 1: out = bf16(silu(a)) for all 65536 - NaN patterns of a, against
    x * expit(x) in float64 rounded once (independent of the oracle's form)."""
    a = _all_bf16()
    out = oracle.swiglu_fwd(a, np.full_like(a, 0x3F80))
    x = bf(a)
    with np.errstate(invalid="ignore", over="ignore"):
        exact = x * scipy.special.expit(x)
    want = bf16_round_exact(exact)
    assert _same_value(out, want).all()


def test_fwd_closed_forms():
    a = _all_bf16(finite_only=True)
    one = np.full_like(a, 0x3F80)
    out = bf(oracle.swiglu_fwd(a, one))
    x = bf(a)
    assert np.all(out[x == 0] == 0)
    # saturation: silu(x) = x once e^-x is below half an ulp of 1 (x >= 17 in fp64 terms),
    # silu(x) -> -0 once x e^x underflows
    big = x >= 24
    assert np.array_equal(out[big], x[big])
    assert np.all(np.abs(out[x <= -200]) == 0)
    # silu(x) - silu(-x) = x; each output carries one bf16 rounding (half an ulp)
    mid = (np.abs(x) > 1e-3) & (np.abs(x) < 60)
    pos = bf(oracle.swiglu_fwd(a[mid], one[mid]))
    neg = bf(oracle.swiglu_fwd((a[mid] ^ 0x8000).astype(np.uint16), one[mid]))
    err = np.abs(pos - neg - x[mid])
    assert np.all(err <= 2.0**-8 * (np.abs(pos) + np.abs(neg)) + 1e-38)
    # silu(x) < x for x > 0, silu(x) in (-0.2785, 0) for x < 0
    assert np.all(out[(x > 0) & (x < 24)] <= x[(x > 0) & (x < 24)])
    assert np.all((out[x < 0] <= 0) & (out[x < 0] >= -0.28))


def test_fwd_rounds_silu_before_multiply():
    """out = bf16(bf16(silu(a)) * b): with b = 1 + 2^-7 the product is exact
    in fp32 and the result shows whether silu was rounded to bf16 first."""
    g = gen(13)
    a = to_u16(randn_bf16((4096,), g, std=3.0))
    b = np.full_like(a, 0x3F81)  # 1 + 2^-7
    out = oracle.swiglu_fwd(a, b)
    s16 = bf16_round_exact(bf(a) * scipy.special.expit(bf(a)))
    assert np.array_equal(out, bf16_round_exact(bf(s16) * (1 + 2.0**-7)))


def test_bwd_matches_finite_differences():
    """t = g * b = 1 (g = b = 1): da = bf16(silu'(a)); silu' from central
    differences of the fp64 silu, step 1e-6 (error ~1e-12, far below 2^-9)."""
    g = gen(14)
    a = np.concatenate([to_u16(randn_bf16((20000,), g, std=4.0)), _all_bf16(finite_only=True)[::7]])
    x = bf(a)
    keep = np.abs(x) < 80
    a, x = a[keep], x[keep]
    one = np.full_like(a, 0x3F80)
    _, da = oracle.swiglu_bwd(one, one, one, a)
    h = 1e-6
    silu = lambda v: v / (1.0 + np.exp(-v))
    fd = (silu(x + h) - silu(x - h)) / (2 * h)
    fd = np.where(np.abs(x) < 1e-30, 0.5, fd)  # the difference quotient loses all digits at denormal x
    diff = np.abs(bf(da) - fd)
    assert np.all(diff <= 2.0**-8 * np.abs(fd) + 1e-9)


def test_bwd_closed_forms():
    g = gen(15)
    t = to_u16(randn_bf16((512,), g, std=2.0))
    one = np.full_like(t, 0x3F80)
    zero = np.zeros_like(t)
    # silu'(0) = 1/2 exactly: da = bf16(t / 2) = t with the exponent lowered (exact)
    db, da = oracle.swiglu_bwd(t, zero, one, zero)
    assert np.array_equal(bf(da), bf(t) / 2)
    assert np.all(bf(db) == 0)
    # silu'(x) -> 1 for large x, -> 0 (from below) for very negative x
    _, da = oracle.swiglu_bwd(t, zero, one, np.full_like(t, 0x4200))   # a = 32
    assert np.array_equal(da, t)
    _, da = oracle.swiglu_bwd(t, zero, one, np.full_like(t, 0xC300))   # a = -128
    assert np.all(np.abs(bf(da)) < 1e-50 + 1e-40 * np.abs(bf(t)))
    # silu' changes sign at x0 = -1.27846454276107...: negative below, positive above
    lo, hi = bf16_round_exact(np.array([-1.3])), bf16_round_exact(np.array([-1.25]))
    _, d_lo = oracle.swiglu_bwd(one[:1], zero[:1], one[:1], lo)
    _, d_hi = oracle.swiglu_bwd(one[:1], zero[:1], one[:1], hi)
    assert bf(d_lo)[0] < 0 < bf(d_hi)[0]


def test_bwd_rounds_g_times_b():
    """da uses t = bf16(g * b): with g * b not representable in bf16 the
    result equals the one from the pre-rounded product fed as g (b = 1)."""
    g = gen(16)
    gr, b, a = (to_u16(randn_bf16((4096,), g)) for _ in range(3))
    zero = np.zeros_like(gr)
    _, da = oracle.swiglu_bwd(gr, zero, b, a)
    t = bf16_round_exact(bf(gr) * bf(b))
    _, da_t = oracle.swiglu_bwd(t, zero, np.full_like(gr, 0x3F80), a)
    assert np.array_equal(da, da_t)
    assert not np.array_equal(t, gr)  # the rounding point is actually exercised


@pytest.mark.parametrize("shape", [(0,), (1,), (3, 5), (2, 7, 11)])
def test_shapes_and_empty(shape):
    g = gen(17)
    a, b = randn_bf16(shape, g), randn_bf16(shape, g)
    out = oracle.swiglu_fwd(to_u16(a), to_u16(b))
    assert out.shape == tuple(shape)
    ref = to_u16(torch.nn.functional.silu(a) * b)
    assert (ulp_bf16(out, ref) <= 1).all()
    db, da = oracle.swiglu_bwd(to_u16(a), to_u16(b), to_u16(b), to_u16(a))
    assert db.shape == da.shape == tuple(shape)
    with pytest.raises(ValueError):
        oracle.swiglu_fwd(to_u16(a), np.zeros((5,), np.uint16))


def test_silu_every_bf16_value_matches_torch_cpu_eager():
    """oracle.silu (v7/58e7a4d6cde3) over all non-NaN bf16 values against
    torch's CPU bf16 silu, to one bf16 ulp (torch's CPU kernel evaluates
    in fp32 with its own exp).  Below x ~ -88.7 fp32 exp(-x) overflows and
    eager returns -0 where the fp64 value is a tiny number (< 1e-30)."""
    a = _all_bf16()
    out = oracle.silu(a)
    ref = to_u16(torch.nn.functional.silu(from_u16(a)))
    with np.errstate(invalid="ignore"):
        tiny = np.abs(bf(out) - bf(ref)) < 1e-30
    assert (_same_value(out, ref) | (ulp_bf16(out, ref) <= 1) | tiny).all()
    differ = ~_same_value(out, ref) & (ulp_bf16(out, ref) > 1)
    assert (bf(a)[differ] < -88.0).all()
    assert np.array_equal(out, oracle.swiglu_fwd(a, np.full_like(a, 0x3F80)))


def test_swiglu_fwd_bwd_is_the_composition():
    """(h, db, da) of v6/182d2dcd0652 against torch CPU eager silu / mul /
    silu_backward with silu materialised in bf16, as the fragment does."""
    g = gen(13)
    a, b, gr = (randn_bf16((32, 515), g, std=2.5) for _ in range(3))
    h, db, da = oracle.swiglu_fwd_bwd(to_u16(a), to_u16(b), to_u16(gr))
    s = torch.nn.functional.silu(a)
    assert (ulp_bf16(h, to_u16(s * b)) <= 1).all()
    assert (ulp_bf16(db, to_u16(gr * s)) <= 1).all()
    da_ref = to_u16(torch.ops.aten.silu_backward(gr * b, a))
    u = ulp_bf16(da, da_ref)
    assert (u <= 1).mean() > 0.999
    # db uses the bf16-rounded silu, not fp32 silu: a planted fp32 s differs
    s32 = a.float() * torch.sigmoid(a.float())
    assert not np.array_equal(db, to_u16((gr.float() * s32).to(torch.bfloat16)))
