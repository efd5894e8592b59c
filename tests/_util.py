"""Shared helpers for the tests: bf16 <-> numpy bit patterns, seeded inputs,
tolerance checks.  bf16 data is exchanged with the oracle as uint16."""
from __future__ import annotations

import numpy as np
import torch

# North-star tolerance for bf16 outputs (fp32 accumulation).
BF16_RTOL = 1.6e-2
BF16_ATOL = 1e-2
# North-star tolerance for the fp32 weight gradient.
DW_RTOL = 1e-3


def to_u16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns (contiguous)."""
    assert t.dtype == torch.bfloat16
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_u16(a: np.ndarray, device=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return t.to(device) if device is not None else t


def bf(a: np.ndarray) -> np.ndarray:
    """uint16 bit patterns -> float64 values."""
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn_bf16(shape, g, mean=0.0, std=1.0) -> torch.Tensor:
    """Drawn in fp32 on the CPU, cast to bf16 (identical on every host)."""
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def ulp_bf16(a_u16: np.ndarray, b_u16: np.ndarray) -> np.ndarray:
    """Distance in bf16 units in the last place (monotone integer mapping)."""

    def key(x):
        x = np.asarray(x, dtype=np.uint16).astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + x)

    return np.abs(key(a_u16) - key(b_u16))


def assert_bf16_close(actual, expected, rtol=BF16_RTOL, atol=BF16_ATOL, what="", max_ulp=None, min_exact=None,
                      ulp_abs_slack=0.0):
    """actual / expected: uint16 bf16 bit patterns.  Checks the north-star
    tolerance |a - e| <= atol + rtol |e| on every element, and optionally a
    maximum ulp distance and a minimum fraction of bit-identical elements.
    Elements farther than max_ulp are still accepted when |a - e| <=
    ulp_abs_slack: near cancellation an fp32 rounding error proportional to
    the operands spans many ulps of a tiny result."""
    a, e = np.asarray(actual), np.asarray(expected)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    av, ev = bf(a), bf(e)
    bad = np.abs(av - ev) > atol + rtol * np.abs(ev)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {a.size} outside rtol={rtol} atol={atol}; "
        f"worst |diff|={np.max(np.abs(av - ev)):.4g}")
    if max_ulp is not None and a.size:
        u = ulp_bf16(a, e)
        far = (u > max_ulp) & (np.abs(av - ev) > ulp_abs_slack)
        assert not far.any(), (f"{what}: {int(far.sum())} elements beyond {max_ulp} ulp and {ulp_abs_slack} abs; "
                               f"max ulp {u.max()}")
    if min_exact is not None and a.size:
        frac = float(np.mean(a == e))
        assert frac >= min_exact, f"{what}: only {frac:.5f} of elements bit-identical (< {min_exact})"


def zipf_ids(n: int, vocab: int, s: float, g: torch.Generator) -> torch.Tensor:
    """Truncated Zipf(s) over ranks 1..vocab, id = rank - 1 (id 0 most frequent)."""
    r = torch.arange(1, vocab + 1, dtype=torch.float64)
    p = r.pow(-s)
    p /= p.sum()
    return torch.multinomial(p, n, replacement=True, generator=g).to(torch.int64)


_BF16_TABLE = None


def bf16_round_exact(v: np.ndarray) -> np.ndarray:
    """Correctly rounded (nearest, ties to even) float64 -> bf16 bit patterns,
    by search over the sorted table of all finite bf16 values; saturates to
    +-inf beyond the largest finite value's rounding boundary; NaN -> the
    quiet NaN 0x7FC0.  Independent of any float32 intermediate (no double
    rounding)."""
    global _BF16_TABLE
    if _BF16_TABLE is None:
        pats = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
        with np.errstate(invalid="ignore"):
            vals = bf(pats)
        keep = np.isfinite(vals) & ~((pats == 0x8000))  # one zero
        order = np.argsort(vals[keep], kind="stable")
        _BF16_TABLE = (vals[keep][order], pats[keep][order])
    tv, tp = _BF16_TABLE
    v = np.asarray(v, dtype=np.float64).ravel()
    out = np.empty(v.shape, dtype=np.uint16)
    hi_i = np.clip(np.searchsorted(tv, v, side="left"), 1, len(tv) - 1)
    lo_i = hi_i - 1
    lo, hi = tv[lo_i], tv[hi_i]
    d_lo, d_hi = v - lo, hi - v
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((tp[hi_i] & 1) == 0))
    res = np.where(pick_hi, tp[hi_i], tp[lo_i])
    exact = np.isin(v, tv)
    res = np.where(exact, tp[np.clip(np.searchsorted(tv, v), 0, len(tv) - 1)], res)
    # beyond the largest finite value: overflow boundary is max + half an ulp
    big = 3.3895313892515355e38  # 0x7F7F
    ulp = 2.0 ** (127 - 7)
    res = np.where(v >= big + ulp / 2, 0x7F80, res)
    res = np.where(v <= -(big + ulp / 2), 0xFF80, res)
    res = np.where(v == 0, np.where(np.signbit(v), 0x8000, 0x0000), res)
    res = np.where(np.isnan(v), 0x7FC0, res)
    out[:] = res
    return out.reshape(np.shape(v))
