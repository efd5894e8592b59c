"""Writes tests/golden/tol_tiers.json -- TEST INFRASTRUCTURE, run only in the
build container (it reads /root/reference's benchmark.json result records,
plain JSON data).

The reference's harness passes a fragment when
    max_tol_units = max |out - ref| / (atol_eff + rtol * |ref|) <= 1,
with the tier's (atol, rtol) -- bitwise 0.08 / 1e-3, reduction 0.05 / 1e-2,
complex 0.05 / 1e-2 -- and atol_eff = max(tier atol, torch.compile's own
max_abs_err), the "trusted baseline" (e.g. v8/7884328a5557/benchmark.json:3-20).
For each fragment with a record this keeps its tier, rtol and atol_eff (the
harness's own, where a candidate's record carries one; else computed from
the torch.compile entry).  Fragments without a record get no entry; the
tests then use the tier of their family at the base atol.

It also writes tests/golden/reference_times.json: each record's eager time
and its fastest passing candidate (backend, time), the reference's own
per-fragment figures on its (H100) hardware, which bench.py --fragments
prints beside this build's times.

    python tests/golden/make_tol_tiers.py
"""
from __future__ import annotations

import json
from pathlib import Path

REFERENCE = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "tol_tiers.json"
TIMES = Path(__file__).resolve().parent / "reference_times.json"
TIERS = {"bitwise": (0.08, 1e-3), "reduction": (0.05, 1e-2), "complex": (0.05, 1e-2)}


def times(rec):
    best = None
    for k, v in rec.items():
        if isinstance(v, dict) and v.get("status") == "PASS" and "time_ms" in v:
            if best is None or v["time_ms"] < best[1]:
                best = (k, float(v["time_ms"]))
    out = {"eager_ms": float(rec["eager_ms"])} if rec.get("eager_ms") is not None else {}
    if best:
        out.update({"best_backend": best[0], "best_ms": best[1]})
    return out


def main():
    out, tm = {}, {}
    for f in sorted(REFERENCE.glob("v*/*/benchmark.json")):
        rec = json.loads(f.read_text())
        fid = f"{f.parent.parent.name}/{f.parent.name}"
        t = times(rec)
        if t:
            tm[fid] = t
        tier = atol_eff = rtol = compile_err = None
        for k, v in rec.items():
            if not isinstance(v, dict):
                continue
            tier = tier or v.get("tol_tier")
            if "atol_eff" in v and atol_eff is None:
                atol_eff, rtol = float(v["atol_eff"]), float(v["rtol"])
            if k == "torch_compile" and "max_abs_err" in v:
                compile_err = float(v["max_abs_err"])
        if tier is None:
            continue
        base_atol, base_rtol = TIERS[tier]
        if atol_eff is None:
            atol_eff = max(base_atol, compile_err) if compile_err is not None else base_atol
            rtol = base_rtol
        out[fid] = {"tier": tier, "atol_eff": atol_eff, "rtol": rtol, "compile_max_abs_err": compile_err}
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    TIMES.write_text(json.dumps(tm, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT}: {len(out)} fragments; {TIMES}: {len(tm)}")


if __name__ == "__main__":
    main()
