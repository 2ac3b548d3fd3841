"""Build libdiagpu.so (all HIP sources under csrc/, gfx950) in-tree.

    python -m diagpu_amd.build            # library only
    python -m diagpu_amd.build --all      # + oracle, reference programs, C++ tests

Each source is compiled to an object in diagpu_amd/_build/ (in parallel),
then linked into diagpu_amd/libdiagpu.so.  Every call recompiles.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libdiagpu.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed FP32 VALU
# instructions (v_pk_*_f32) on gfx950.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libdiagpu)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n"
                           f"{proc.stdout}\n{proc.stderr}")


def build_library(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_run, [cc, *HIP_FLAGS, "-c", str(s), "-o", str(o)])
                for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "all"])


def build_cpp_tests() -> None:
    """C++ programs that use the drop-in header include/diagpu/dia.hpp."""
    src_dir = ROOT / "tests" / "cpp"
    out_dir = src_dir / "bin"
    if not src_dir.exists():
        return
    out_dir.mkdir(exist_ok=True)
    cc = hipcc()
    for src in sorted(src_dir.glob("*.cpp")):
        exe = out_dir / src.stem
        if src.stem.endswith("_cpu"):      # host-only: plain g++, no HIP
            _run(["g++", "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'include'}", f"-I{CSRC}", str(src),
                  f"-L{ROOT / 'oracle'}", "-loracle", "-Wl,-rpath,$ORIGIN/../../../oracle",
                  "-o", str(exe)])
            continue
        # tests/cpp/bin/<exe>: the library and the oracle sit three levels up
        _run([cc, "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'include'}", str(src),
              f"-L{PKG}", "-ldiagpu", f"-L{ROOT / 'oracle'}", "-loracle",
              "-Wl,-rpath,$ORIGIN/../../../diagpu_amd", "-Wl,-rpath,$ORIGIN/../../../oracle",
              "-o", str(exe)])


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--all", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=8)
    args = ap.parse_args(argv)
    lib = build_library(args.jobs)
    print(f"built {lib}")
    if args.all:
        build_oracle()
        build_cpp_tests()
        print("built oracle and C++ tests")
    return 0


if __name__ == "__main__":
    sys.exit(main())
