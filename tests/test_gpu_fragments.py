"""Parity of every fragment drop-in (kernelproblems_amd.fragments) with the
fragment's own eager op sequence (oracle/fragments.py) on the same inputs,
at the reference's full shapes: same output arity, shapes, strides, dtypes,
the same aliasing between outputs, untouched inputs, and values within the
tolerance of each output's kind.
"""
import json
import os
from pathlib import Path

import pytest
import torch

import oracle.fragments as eager
from kernelproblems_amd import fragments as fr
from tests._util import BF16_ATOL, BF16_RTOL

# Outputs that are bit copies (gathered rows, unsharded parameters).
EXACT = {
    "v7/1e49beb8a123": {0},
    "v8/8e33a91b7364": {1},
    "v8/94985bdb7630": set(range(3, 10)),
    "v8/7815074de963": set(range(3, 10)),
    "v8/12545c1e9b06": set(range(3, 9)),
    "v5/013a3088b488": {1},
    "v1/2a844503364a": {2, 3, 4},
}
# Token-sum outputs of chains whose summed rows come from an earlier kernel
# of the chain: each summand may differ from eager's by one bf16 ulp, and the
# sum amplifies that near cancellation.  Their values are checked in
# tests/test_gpu_chain.py against a bound built from the summands themselves.
CHECKED_IN_CHAIN_TEST = {"v6/0b493aad68f0": {4}, "v5/118d525f44e0": {4}, "v8/f6251e84e3fa": {1}}
# Residual-epilogue outputs bf16(res + bf16(dx)): output index -> index of
# the residual input.  dx carries the backward's bf16 tolerance relative to
# dx itself, so where res and dx nearly cancel the bound is taken relative to
# the summands (|out| + |out - res| >= |dx| up to one rounding), not to the sum.
RESIDUAL_SUM = {
    "v4/363b7b58c971": {3: 5}, "v4/9c745ea697a7": {2: 5}, "v5/401b52261ef5": {2: 4},
    "v5/92ce4a0c7b2c": {3: 5}, "v6/408ac0979ac5": {2: 5}, "v6/822931829090": {3: 5},
    "v6/e9198b707240": {2: 4}, "v7/7f544ceb2120": {0: 5}, "v7/ed20955ec34b": {0: 6},
    "v8/d8f596b3df34": {0: 5}, "v8/43f0c930291e": {0: 6},
}
# fp32 outputs that carry no bf16 rounding (complex-multiply result):
# fp32 reassociation / contraction differences only.
F32_TOL = {"v7/0f38bc55457c": {0}}


# The reference harness's pass criterion (tests/golden/make_tol_tiers.py):
# max |out - ref| / (atol_eff + rtol |ref|) <= 1 with the fragment's tier.
# Fragments without a result record use their family's tier at its base atol
# (the RoPE captures: complex; the rest here: reduction).
TOL_TIERS = json.loads((Path(__file__).resolve().parent / "golden" / "tol_tiers.json").read_text())
BASE_TIERS = {"bitwise": (0.08, 1e-3), "reduction": (0.05, 1e-2), "complex": (0.05, 1e-2)}
COMPLEX_WITHOUT_RECORD = {"v8/7e38211c7f1c", "v1/075cb40f3d5d", "v1/9cd8f72e74ce", "v1/f23f9bb4567a",
                          "v1/d7efc428b2f5"}


def _tier(fid):
    for f in (fid, fr.SAME_AS.get(fid), fr.EQUIVALENT.get(fid), fr.EQUIVALENT.get(fr.SAME_AS.get(fid, ""))):
        if f in TOL_TIERS:
            t = TOL_TIERS[f]
            return t["tier"], t["atol_eff"], t["rtol"]
    canon = fr.EQUIVALENT.get(fr.SAME_AS.get(fid, fid), fr.SAME_AS.get(fid, fid))
    tier = "complex" if canon in COMPLEX_WITHOUT_RECORD else "reduction"
    return (tier, *BASE_TIERS[tier])


def max_tol_units(ours, ref, atol, rtol):
    worst = 0.0
    for a, e in zip(ours, ref):
        if a.is_complex():
            a, e = torch.view_as_real(a), torch.view_as_real(e)
        if a.numel() == 0:
            continue
        d = (a.double() - e.double()).abs() / (atol + rtol * e.double().abs())
        worst = max(worst, float(d.max()))
    return worst


def _tuple(o):
    return o if isinstance(o, tuple) else (o,)


def _storage(t):
    return t.untyped_storage().data_ptr()


def _clone(x):
    """A copy of one fragment input: a tensor, or the tuple a captured graph
    passes (e.g. a saved forward's (y, rstd))."""
    return tuple(_clone(t) for t in x) if isinstance(x, (tuple, list)) else x.clone()


def _same(x, y):
    if isinstance(x, (tuple, list)):
        return len(x) == len(y) and all(_same(a, b) for a, b in zip(x, y))
    return torch.equal(x, y)


def _check_close(fid, i, a, e, inputs):
    what = f"{fid} output {i}"
    fid = fr.SAME_AS.get(fid, fid)  # a repeated fragment's outputs are classed as its canonical's
    fid = fr.EQUIVALENT.get(fid, fid)
    assert a.shape == e.shape and a.dtype == e.dtype, f"{what}: {a.shape}/{a.dtype} vs {e.shape}/{e.dtype}"
    assert a.stride() == e.stride(), f"{what}: strides {a.stride()} vs {e.stride()}"
    if i in EXACT.get(fid, ()):
        assert torch.equal(a, e), f"{what}: not a bit-exact copy"
        return
    if i in CHECKED_IN_CHAIN_TEST.get(fid, ()):
        return
    if a.is_complex():
        # complex64 products in fp32, no bf16 rounding: contraction differences only
        a, e = torch.view_as_real(a), torch.view_as_real(e)
        rtol, atol = 1e-5, 1e-5
    elif a.dtype == torch.float32 and i in F32_TOL.get(fid, ()):
        rtol, atol = 1e-5, 1e-5
    else:
        rtol, atol = BF16_RTOL, BF16_ATOL
    af, ef = a.double(), e.double()
    scale = ef.abs()
    if i in RESIDUAL_SUM.get(fid, {}):
        res = inputs[RESIDUAL_SUM[fid][i]]
        assert res.numel() == ef.numel()
        res = res.double().reshape(ef.shape)
        scale = scale + (ef - res).abs()
    bad = (af - ef).abs() > atol + rtol * scale
    n_bad = int(bad.sum())
    assert n_bad == 0, f"{what}: {n_bad} of {a.numel()} outside rtol={rtol} atol={atol}; worst {(af - ef).abs().max():.4g}"


@pytest.mark.gpu
@pytest.mark.parametrize("fid", fr.FRAGMENTS)
def test_fragment_matches_eager(fid, gpu):
    print(f"[fragment] {fid}", flush=True)
    mod = fr.load(fid)
    g = torch.Generator(device=gpu).manual_seed(fr.FRAGMENTS.index(fid) + 1)
    inputs = mod.get_inputs(device=gpu, generator=g)
    before = [_clone(t) for t in inputs]
    ours = mod.kernel_function(*inputs)
    torch.cuda.synchronize()
    for t, b in zip(inputs, before):
        assert _same(t, b), f"{fid}: an input was modified"
    ref = eager.run(fid, inputs)
    assert isinstance(ours, tuple) == isinstance(ref, tuple), f"{fid}: tuple vs bare output"
    ours, ref = _tuple(ours), _tuple(ref)
    assert len(ours) == len(ref), f"{fid}: {len(ours)} outputs, expected {len(ref)}"
    for i, (a, e) in enumerate(zip(ours, ref)):
        assert a.device == e.device
        _check_close(fid, i, a, e, inputs)
    for i in range(len(ref)):
        for j in range(i + 1, len(ref)):
            same_ref = _storage(ref[i]) == _storage(ref[j])
            same_ours = _storage(ours[i]) == _storage(ours[j])
            assert same_ref == same_ours, f"{fid}: aliasing of outputs {i} and {j} differs from the fragment's"
    tier, atol, rtol = _tier(fid)
    units = max_tol_units(ours, ref, atol, rtol)
    print(f"[fragment] {fid}: max_tol_units {units:.4f} ({tier}, atol_eff {atol:g}, rtol {rtol:g})", flush=True)
    if os.environ.get("KP_TOL_REPORT"):
        with open(os.environ["KP_TOL_REPORT"], "a") as f:
            f.write(json.dumps({"fragment": fid, "tier": tier, "atol_eff": atol, "rtol": rtol,
                                "max_tol_units": units}) + "\n")
    assert units <= 1.0, f"{fid}: max_tol_units {units:.4f} > 1 (the reference harness's {tier} tier)"
