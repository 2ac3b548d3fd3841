"""Regenerate the golden fixtures in this directory from the reference's own
host programs, built from the reference sources by `make -C oracle ref` into
oracle/_ref/ (this needs the reference checkout; the fixtures are committed,
so the GPU box never runs this).

  reconstruct_kat.json  -- output of spmv/test/test_reconstruct.cpp: the 5x5
                           matrix, x, DIA offsets, Recon offsets and rows, y,
                           parsed from its printout.
  gen_banded_n64.mtx    -- output of spmv/tools/gen_banded_mtx.cpp for N=64:
                           the SpMV bench's 9-diagonal hash band
                           (spmv/bench/bench_cusparse.cu:70-87).
"""
from __future__ import annotations

import json
import re
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REF = HERE.parents[1] / "oracle" / "_ref"


def _floats(line: str) -> list[float]:
    return [float(t) for t in re.findall(r"-?\d+\.\d+", line)]


def parse_reconstruct(text: str) -> dict:
    lines = text.splitlines()
    out: dict = {}
    i = 0
    while i < len(lines):
        ln = lines[i]
        if ln.startswith("1. ORIGINAL"):
            out["H"] = [_floats(lines[i + 1 + r]) for r in range(5)]
            i += 6
            continue
        if ln.strip().startswith("x  [5]"):
            out["x"] = _floats(lines[i + 1])
        if "DIA storage" in ln:
            out["dia_offsets"] = [int(t) for t in ln.split("{")[1].split("}")[0].split()]
        if "Recon offsets" in ln:
            out["recon_offsets"] = [int(t) for t in ln.split("{")[1].split("}")[0].split()]
        if ln.startswith("2. CONSTRUCT"):
            out["recon_rows"] = [_floats(lines[i + 1 + r]) for r in range(5)]
            i += 6
            continue
        if ln.startswith("3. RESULT"):
            out["y"] = _floats(lines[i + 1])
        if "[OK]" in ln or "[FAIL]" in ln:
            out.setdefault("checks", []).append("OK" if "[OK]" in ln else "FAIL")
        i += 1
    return out


def main() -> int:
    exe = REF / "test_reconstruct"
    gen = REF / "gen_banded_mtx"
    if not exe.exists() or not gen.exists():
        print("oracle/_ref programs missing: run `make -C oracle ref` first", file=sys.stderr)
        return 1
    text = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    kat = parse_reconstruct(text)
    kat["source"] = "spmv/test/test_reconstruct.cpp (built from the reference sources)"
    (HERE / "reconstruct_kat.json").write_text(json.dumps(kat, indent=1) + "\n")
    subprocess.run([str(gen), "64", str(HERE / "gen_banded_n64.mtx")], check=True,
                   capture_output=True)
    print("wrote reconstruct_kat.json, gen_banded_n64.mtx")
    return 0


if __name__ == "__main__":
    sys.exit(main())
