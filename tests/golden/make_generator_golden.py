"""Write tests/golden/generators.json: outputs of the reference's own input
generators, run from their source text by oracle/_ref/ref_generators (built
by `make -C oracle ref` where the reference checkout exists; see
oracle/Makefile).  The fixtures pin the oracle's restatements of

  hval, xval         spmv/bench/bench_cusparse.cu:70-82
  run_case's H, x    spmv/test/test_tc_spmv.cu:86-98 (the six cases of :168-179)
  make_banded        spmspm/bench_spmspm.cu:79-106 (seeds 1234 / 5678 of :465-466)
  pack_diag_matrix   gemm_diag/gemm_diag.cu:361-382 (seeds 42 / 137 of :485-486)

Values are stored as float32 bit patterns (uint32), whole for small cases;
full-size cases store the SHA-256 of the little-endian array bytes plus
their first 64 values.  Run in this container only:

    python tests/golden/make_generator_golden.py
"""
from __future__ import annotations

import hashlib
import json
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
EXE = ROOT / "oracle" / "_ref" / "ref_generators"
OUT = Path(__file__).resolve().parent / "generators.json"


def run(*args) -> bytes:
    proc = subprocess.run([str(EXE), *map(str, args)], capture_output=True, check=True)
    return proc.stdout


def bits(a: np.ndarray) -> list[int]:
    return np.ascontiguousarray(a, np.float32).view(np.uint32).tolist()


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def summary(a: np.ndarray, whole_below: int = 4096) -> dict:
    d = {"count": int(a.size), "sha256": digest(a)}
    if a.size <= whole_below:
        d["bits"] = bits(a)
    else:
        d["head_bits"] = bits(a[:64])
    return d


def band_entries(H: np.ndarray, offs) -> np.ndarray:
    """H[r, r + d] in the fill order of run_case: rows ascending, then the
    offsets in their given order, in-range entries only."""
    N = H.shape[0]
    return np.array([H[r, r + d] for r in range(N) for d in offs if 0 <= r + d < N],
                    np.float32)


# the six structural cases of spmv/test/test_tc_spmv.cu:168-179
LCG_CASES = [
    (48, [-1, 0, 1]), (37, [-1, 0, 1]), (64, [-2, -1, 0, 1, 2]),
    (80, [-9, -5, -2, -1, 0, 1, 2, 5, 9]), (71, [-3, 0, 2, 4, 7]), (16, [0]),
]
HASH_OFFSETS = [-9, -5, -2, -1, 0, 1, 2, 5, 9]      # bench_cusparse.cu:87


def main() -> int:
    if not EXE.exists():
        print(f"{EXE} missing: run `make -C oracle ref` with the reference checkout present")
        return 1
    fx: dict = {"generator": "oracle/_ref/ref_generators (oracle/Makefile target ref)"}
    fx["xval"] = [{"N": N, **summary(np.frombuffer(run("xval", N), np.float32))}
                  for N in (1000, 1 << 20)]
    fx["hval"] = [{"N": N, "offsets": HASH_OFFSETS,
                   **summary(np.frombuffer(run("hval", N, *HASH_OFFSETS), np.float32))}
                  for N in (64, 1 << 20)]
    fx["lcg"] = []
    for N, offs in LCG_CASES:
        raw = np.frombuffer(run("lcg", N, *offs), np.float32)
        H, x = raw[: N * N], raw[N * N:]
        band = band_entries(H.reshape(N, N), offs)
        fx["lcg"].append({"N": N, "offsets": offs, "H_sha256": digest(H),
                          "band_bits": bits(band), "x_bits": bits(x)})
    fx["make_banded"] = []
    for n, w, seed in [(20, 16, 1234), (10, 16, 5678), (300, 3, 1234),
                       (100000, 16, 1234), (100000, 16, 5678)]:
        raw = run("banded", n, w, seed)
        cnt = int(np.frombuffer(raw[:4], np.int32)[0])
        o = 4
        offs = np.frombuffer(raw[o: o + 4 * cnt], np.int32); o += 4 * cnt
        starts = np.frombuffer(raw[o: o + 8 * cnt], np.int64); o += 8 * cnt
        lens = np.frombuffer(raw[o: o + 4 * cnt], np.int32); o += 4 * cnt
        vals = np.frombuffer(raw[o:], np.float32)
        fx["make_banded"].append({"n": n, "w": w, "seed": seed, "offsets": offs.tolist(),
                                  "starts": starts.tolist(), "lengths": lens.tolist(),
                                  "values": summary(vals)})
    fx["pack_diag_matrix"] = []
    for n, offs, seed in [(32, list(range(-10, 11)), 42), (50, [-4, 0, 7], 137),
                          (4096, list(range(-10, 11)), 42), (4096, list(range(-10, 11)), 137)]:
        DA = np.frombuffer(run("pack", n, seed, *offs), np.float32)
        fx["pack_diag_matrix"].append({"n": n, "offsets": offs, "seed": seed,
                                       "DA": summary(DA)})
    OUT.write_text(json.dumps(fx, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
