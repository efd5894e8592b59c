"""Writes tests/golden/fragment_outputs.json -- TEST INFRASTRUCTURE, run only
in the build container (it imports the reference's problem.py files from
/root/reference, which exists nowhere else; nothing of them is stored).

For each fragment with a drop-in (kernelproblems_amd.fragments), the
reference's own Model.forward (<round>/<id>/problem.py) runs on the CPU on
full-shape inputs with the drop-in's input layout, filled from a fixed seed
(tests/golden/fragment_inputs.py; a fragment that re-uses another's drop-in
takes that one's seed, so equal op sequences give equal records) --
the CUDA-only _fused_rms_norm_backward through torch's decomposition
(oracle.fragments.CpuDecompositions) -- and the fixture records, per output:
dtype, shape, strides, storage offset, which outputs share storage, which
alias an input, and values at 48 seeded flat positions.  Data only: no
reference text, code or bytecode is kept (bytecode writing is off, so the
import leaves /root/reference untouched).

    python tests/golden/make_fragment_fixtures.py [--only v8/d8f596b3df34 ...]

tests/test_fragment_structure.py checks oracle/fragments.py (the eager
restatements the GPU drop-ins are compared with) against these records.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import sys
import time
from pathlib import Path

sys.dont_write_bytecode = True
ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from tests.golden.fragment_inputs import describe, synth_inputs  # noqa: E402

REFERENCE = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "fragment_outputs.json"


def seed_of(fid: str) -> int:
    from kernelproblems_amd import fragments as fr
    canon = fr.EQUIVALENT.get(fr.SAME_AS.get(fid, fid), fr.SAME_AS.get(fid, fid))
    return int(canon.split("/")[1][:8], 16) % 100003


def reference_forward(fid, inputs):
    path = REFERENCE / fid / "problem.py"
    spec = importlib.util.spec_from_file_location("ref_" + fid.replace("/", "_"), path)
    mod = importlib.util.module_from_spec(spec)
    # the v1 captures call device(...) without the `from torch import device`
    # the later rounds' files carry; the name is provided up front
    mod.device = torch.device
    spec.loader.exec_module(mod)
    model = mod.Model(*mod.get_init_inputs())
    import oracle.fragments as eager
    with torch.no_grad(), eager.CpuDecompositions():
        return model(*inputs)


def main():
    from kernelproblems_amd import fragments as fr

    ap = argparse.ArgumentParser()
    ap.add_argument("--only", nargs="*")
    args = ap.parse_args()
    data = json.loads(OUT.read_text()) if OUT.exists() else {}
    ids = args.only or list(fr.FRAGMENTS)
    for fid in ids:
        t0 = time.time()
        seed = seed_of(fid)
        inputs = synth_inputs(fr.load(fid), seed)
        try:
            out = reference_forward(fid, inputs)
            rec = {"seed": seed, **describe(out, inputs, seed)}
        except Exception as e:  # recorded, not hidden: the test reports which fragments are unpinned
            rec = {"seed": seed, "error": f"{type(e).__name__}: {str(e).splitlines()[0][:200]}"}
        data[fid] = rec
        print(f"{fid}: {'ERROR ' + rec['error'] if 'error' in rec else str(len(rec['outputs'])) + ' outputs'} "
              f"({time.time() - t0:.1f} s)", flush=True)
        del inputs
    OUT.write_text(json.dumps(dict(sorted(data.items())), indent=0, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} fragments)")


if __name__ == "__main__":
    main()
