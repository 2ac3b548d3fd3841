"""Write tests/golden/schedule.json: the C structure and grouped pair schedule
of the reference's SpGEMM host planner (make_c_structure,
spmspm/bench_spmspm.cu:109-131; build_schedule, :137-243; PairEntry,
spmspm/spmspm.cu:40-46), run from the reference's own source text by
oracle/_ref/ref_schedule (built by `make -C oracle ref` where the reference
checkout exists; see oracle/Makefile).  The fixture pins the oracle's
restatement (orc_build_schedule).  Arrays of up to 4096 values are stored
whole, longer ones as their count and the SHA-256 of their int32
little-endian bytes.  Run in this container only:

    python tests/golden/make_schedule_golden.py
"""
from __future__ import annotations

import hashlib
import json
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
EXE = ROOT / "oracle" / "_ref" / "ref_schedule"
OUT = Path(__file__).resolve().parent / "schedule.json"


def run(*args) -> dict:
    text = subprocess.run([str(EXE), *map(str, args)], capture_output=True, check=True,
                          text=True).stdout
    out = {}
    for line in text.strip().split("\n"):
        name, cnt, *vals = line.split()
        assert int(cnt) == len(vals), name
        out[name] = np.array([int(v) for v in vals], np.int32)
    return out


def store(a: np.ndarray) -> dict:
    d = {"count": int(a.size),
         "sha256": hashlib.sha256(np.ascontiguousarray(a, np.int32).tobytes()).hexdigest()}
    if a.size <= 4096:
        d["values"] = a.tolist()
    return d


def cases():
    rng = np.random.default_rng(0)
    yield {"banded": [100000, 16, 1234, 5678]}             # the bench's own (:465-471)
    yield {"banded": [300, 3, 1, 2]}
    yield {"banded": [6, 4, 7, 8]}                          # offsets beyond n skipped
    yield {"n": 1 << 20, "A": list(range(-4, 5)),
           "B": [-16384, -128, -1, 0, 1, 128, 16384]}
    yield {"n": 1000, "A": rng.choice(np.arange(-999, 1000), 12, replace=False).tolist(),
           "B": rng.choice(np.arange(-999, 1000), 9, replace=False).tolist()}  # B unsorted
    yield {"n": 262144,                                     # BASELINE config 5 shape
           "A": sorted(rng.choice(np.arange(-4096, 4097), 128, replace=False).tolist()),
           "B": sorted(rng.choice(np.arange(-4096, 4097), 128, replace=False).tolist())}


def main() -> int:
    if not EXE.exists():
        print(f"{EXE} missing: run `make -C oracle ref` with the reference checkout present")
        return 1
    fx = {"generator": "oracle/_ref/ref_schedule (oracle/Makefile target ref)", "cases": []}
    for case in cases():
        if "banded" in case:
            res = run("banded", *case["banded"])
        else:
            res = run("offsets", case["n"], len(case["A"]), *case["A"], *case["B"])
        entry = dict(case)
        entry["scalars"] = res.pop("scalars").tolist()
        entry.update({k: store(v) for k, v in res.items()})
        fx["cases"].append(entry)
        print(case.get("banded", case.get("n")), entry["scalars"])
    OUT.write_text(json.dumps(fx, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
