"""Pins the oracle's bf16 rounding helpers: fp32 -> bf16 against torch's
conversion, fp64 -> bf16 against exhaustive nearest-even search (no double
rounding), and the eager bf16 add against torch's CPU add."""
import numpy as np
import torch

import oracle
from tests._util import bf, bf16_round_exact, to_u16


def _f32_specials():
    vals = [0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 1.1754942e-38, 3.4028235e38, -3.4028235e38,
            float("inf"), float("-inf")]
    # exact ties between adjacent bf16 values, both parities
    ties = [np.float32(1.0 + 2.0**-8), np.float32(1.0 + 3 * 2.0**-8), np.float32(-(1.0 + 2.0**-8))]
    return np.array(vals + ties, dtype=np.float32)


def test_f32_to_bf16_matches_torch():
    g = np.random.default_rng(0)
    bits = g.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = np.concatenate([x[np.isfinite(x)], _f32_specials()])
    ours = oracle.f32_to_bf16(x)
    ref = to_u16(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(ours, ref)
    nan = oracle.f32_to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(bf(nan)).all()


def test_f64_to_bf16_single_rounding():
    g = np.random.default_rng(1)
    # random doubles over a wide range, plus values a hair off bf16 midpoints
    # (a double -> fp32 -> bf16 chain rounds these to the wrong side)
    x = g.standard_normal(100000) * np.exp2(g.integers(-60, 60, 100000))
    base = bf(g.integers(0, 0x7F00, 20000).astype(np.uint16))
    base = base[np.isfinite(base) & (base > 0)]
    ulp = np.exp2(np.floor(np.log2(base)) - 7)
    mids = base + ulp / 2
    near = np.concatenate([mids, mids + ulp * 2.0**-30, mids - ulp * 2.0**-30, -(mids + ulp * 2.0**-30)])
    x = np.concatenate([x, near, [0.0, -0.0, 1.0, 3.3895313892515355e38, 1e39, -1e39]])
    ours = oracle.f64_to_bf16(x)
    ref = bf16_round_exact(x)
    bad = np.flatnonzero(ours != ref)
    assert bad.size == 0, f"{bad.size} mismatches, e.g. {x[bad[:3]]}: {ours[bad[:3]]} vs {ref[bad[:3]]}"


def test_f64_to_bf16_detects_double_rounding():
    """The midpoint-plus-epsilon inputs above do separate single from double
    rounding: the fp32-intermediate chain fails on them."""
    x = np.array([1.0 + 2.0**-8 + 2.0**-40], dtype=np.float64)  # just above a tie
    double_rounded = to_u16(torch.tensor(x.astype(np.float32)).to(torch.bfloat16))
    assert not np.array_equal(bf16_round_exact(x), double_rounded)
    assert np.array_equal(oracle.f64_to_bf16(x), bf16_round_exact(x))


def test_bf16_add_matches_torch():
    g = torch.Generator().manual_seed(2)
    a = (torch.randn(100000, generator=g) * torch.exp2(torch.randint(-20, 20, (100000,), generator=g))).bfloat16()
    b = (torch.randn(100000, generator=g) * torch.exp2(torch.randint(-20, 20, (100000,), generator=g))).bfloat16()
    assert np.array_equal(oracle.bf16_add(to_u16(a), to_u16(b)), to_u16(a + b))
