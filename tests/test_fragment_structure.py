"""oracle/fragments.py (the eager op sequences the GPU drop-ins are compared
with) against the reference fragments' own Model.forward, on the CPU.

tests/golden/fragment_outputs.json records, for every fragment with a
drop-in, what the reference's problem.py returned on seeded full-shape inputs
(tests/golden/make_fragment_fixtures.py, run in the build container): output
arity, tuple or bare, each output's dtype, shape, strides, storage offset,
which outputs share storage, which alias an input, and values at 48 seeded
positions.  Here the restatement runs on the same inputs (same layout, same
seed) and must reproduce all of it -- values bitwise, the two being the same
CPU operators in the same order.  A fragment that re-exports another's
drop-in (SAME_AS / EQUIVALENT) must have recorded exactly what that one
recorded: the reference's two problem.py files compute the same outputs from
the same inputs.
"""
import json
from pathlib import Path

import pytest
import torch

import oracle.fragments as eager
from kernelproblems_amd import fragments as fr
from tests.golden.fragment_inputs import describe, synth_inputs

FIXTURES = json.loads((Path(__file__).resolve().parent / "golden" / "fragment_outputs.json").read_text())
CANONICAL = [f for f in fr.FRAGMENTS if f not in fr.SAME_AS and f not in fr.EQUIVALENT]
ALIASES = [f for f in fr.FRAGMENTS if f in fr.SAME_AS or f in fr.EQUIVALENT]


def test_every_fragment_has_a_reference_record():
    assert set(FIXTURES) == set(fr.FRAGMENTS)
    errors = {f: r["error"] for f, r in FIXTURES.items() if "error" in r}
    assert not errors, f"reference forward failed when the fixtures were written: {errors}"


def _compare(fid, got, exp):
    assert got["tuple"] == exp["tuple"], f"{fid}: tuple vs bare output"
    assert len(got["outputs"]) == len(exp["outputs"]), f"{fid}: {len(got['outputs'])} outputs, reference has " \
                                                        f"{len(exp['outputs'])}"
    for k, (g, e) in enumerate(zip(got["outputs"], exp["outputs"])):
        for key in ("dtype", "shape", "stride", "storage_offset", "storage_group", "aliases_input", "positions"):
            assert g[key] == e[key], f"{fid} output {k}: {key} {g[key]} != reference {e[key]}"
        assert g["values"] == e["values"], f"{fid} output {k}: sampled values differ from the reference's"


@pytest.mark.parametrize("fid", CANONICAL)
def test_restatement_matches_reference_forward(fid):
    rec = FIXTURES[fid]
    inputs = synth_inputs(fr.load(fid), rec["seed"])
    with torch.no_grad(), eager.CpuDecompositions():
        out = eager.run(fid, inputs)
    _compare(fid, describe(out, inputs, rec["seed"]), rec)


@pytest.mark.parametrize("fid", ALIASES)
def test_repeated_fragment_records_equal_its_canonical(fid):
    canon = fr.SAME_AS.get(fid) or fr.EQUIVALENT[fid]
    canon = fr.EQUIVALENT.get(canon, canon)
    _compare(fid, FIXTURES[fid], FIXTURES[canon])


@pytest.mark.parametrize("mistake", ["dropped dy term", "outputs swapped", "output not viewed 2-D"])
def test_planted_mistakes_are_caught(mistake, monkeypatch):
    """Mistakes of the kind a hand transcription makes, planted in the
    restatement of v8/d8f596b3df34, each fail the comparison."""
    fid = "v8/d8f596b3df34"
    aten = torch.ops.aten
    good = eager._FRAGMENTS[fid]

    def bad(a, b, x, r, w, res):
        if mistake == "dropped dy term":
            return eager._rms_bwd_epilogue([aten.view.default(a, list(x.shape))], x, r, w, res, True)
        out, dw = good(a, b, x, r, w, res)
        if mistake == "outputs swapped":
            return dw, out
        return out.view(x.shape), dw

    monkeypatch.setitem(eager._FRAGMENTS, fid, bad)
    rec = FIXTURES[fid]
    inputs = synth_inputs(fr.load(fid), rec["seed"])
    with torch.no_grad(), eager.CpuDecompositions():
        out = eager.run(fid, inputs)
    with pytest.raises(AssertionError):
        _compare(fid, describe(out, inputs, rec["seed"]), rec)
