"""Writes tests/golden/golden.json: SHA-256 digests of the CPU oracle's
outputs for the seeded cases in tests/cases.py (inputs are regenerated from
the seeds, so the fixture stays a few KB).  Run from the repository root:
    python tests/golden/make_golden.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import numpy as np  # noqa: E402

import cases  # noqa: E402
import oracle as ora  # noqa: E402


def main():
    out = {"_comment": "sha256 of oracle outputs per seeded case (tests/cases.py); numpy "
                       + np.__version__ + " PCG64 inputs", "cases": {}}
    for name, (build, run) in cases.golden_cases().items():
        inp, meta = build()
        outs = run(ora, inp, meta)
        out["cases"][name] = {"meta": meta, "sha256": cases.digest(outs),
                              "head": [float(v) for v in np.asarray(outs[-1]).reshape(-1)[:8].astype(np.float64)]}
        print(name, out["cases"][name]["sha256"][:16])
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
