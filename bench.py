"""Benchmark of the MI355X DIA kernels (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--extras | --no-extras]

Prints ONE JSON line.  The headline is benchmark config 2: DIA SpMV of
the 2-D 5-point Poisson stencil on a 2048 x 2048 grid (n = 4,194,304, fp32);
one step = one SpMV y = H x.  `value` is achieved algorithmic HBM bandwidth

    bytes/step = s * (sum_k len(d_k) + cols + rows)     (values once, x once, y once)

divided by the step time measured with HIP events on the launch stream over
exactly K steps.  Each step uses the next of `--sets` independent buffer sets
(>= 512 MiB in total, twice the 256 MiB MALL), so no step finds its operands
in the Infinity Cache.  The "extras" object times the other benchmark configs
the same way (SpMV configs 1-3, SpGEMM configs 4-5 when built).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
FP32_PEAK_TFLOPS = 157.3
METRIC = "DIA SpMV achieved HBM GB/s (% peak); DIA SpGEMM GFLOP/s, 1 MI355X"
MALL_BYTES = 256 << 20


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--sets", type=int, default=0,
                    help="buffer sets rotated per step (0: enough for >= 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline time budget (0 disables)")
    ap.add_argument("--extras", dest="extras", action="store_true", default=True)
    ap.add_argument("--no-extras", dest="extras", action="store_false")
    ap.add_argument("--only", default="",
                    help="profiling aid: run just one workload (spmv2, spmv2d, spmv2c, "
                         "spmv2rc, spmv1, spmv3, spgemm1..spgemm3 (the squares of the SpMV "
                         "configs' matrices), spgemm4, spgemm5, spgemm4c, spgemm5c, taylor, krylov, "
                         "propagator, propagator2d, gemmdiag, gemmdiag20, spmvhash (the "
                         "reference SpMV bench's hash band), spgemmbanded (the reference "
                         "SpGEMM bench's make_banded operands), launch (the launch floor), copy, fill20) "
                         "and print its line")
    return ap.parse_args(argv)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


_SPIN_CYCLES_PER_US = None


def gpu_spin(stream, us: float = 150.0) -> None:
    """Hold `stream` busy for about `us` microseconds with torch's bounded
    spin kernel (untimed, before a timed region's first event), so that the
    launches the host queues next are waiting when that event runs: the
    host latency of the first launch then stays out of the timed region,
    which holds exactly the timed steps."""
    import torch
    global _SPIN_CYCLES_PER_US
    if _SPIN_CYCLES_PER_US is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(100_000)
            e0.record(stream)
            torch.cuda._sleep(1_000_000)
            e1.record(stream)
        e1.synchronize()
        _SPIN_CYCLES_PER_US = 1_000_000 / max(1.0, e0.elapsed_time(e1) * 1e3)
    with torch.cuda.stream(stream):
        torch.cuda._sleep(max(1, int(_SPIN_CYCLES_PER_US * us)))


# --------------------------------------------------------------------------
# SpMV
# --------------------------------------------------------------------------

def spmv_alg_bytes(R, elem: int, xelem: int | None = None) -> int:
    """Values once (matrix element size `elem`), x once and y once (vector
    element size `xelem`, default `elem`)."""
    xe = elem if xelem is None else xelem
    return elem * R.useful_terms() + xe * (R.cols + R.rows)


def time_spmv(cfg: int, dtype, steps: int, warmup: int, seed: int, sets: int, xdtype=None,
              R=None):
    """One SpMV per step over rotating buffer sets (>= 2x the MALL).  dtype is
    the matrix dtype, xdtype the vector dtype (default: dtype; complex64
    vectors with a float32 matrix use the real-matrix complex-state path).
    R: a prepared Recon matrix (default: benchmark config `cfg`)."""
    import torch
    from diagpu_amd import workloads
    from diagpu_amd.spmv import recon_view, _stream_handle, _SPMV
    from diagpu_amd import _lib
    import ctypes as C

    xdtype = xdtype or dtype
    base = torch.float64 if dtype == torch.float64 else torch.float32
    if R is None:
        R = workloads.spmv_config(cfg, seed=seed, device="cuda", dtype=base)
    if dtype == torch.complex64:        # complex values: (1 + 0.5i) times the real ones
        R.values = (R.values * (1 + 0.5j)).to(torch.complex64).contiguous()
    if xdtype == torch.complex64:
        R.x = torch.complex(R.x, torch.roll(R.x, 1)).contiguous()
    elem = R.values.element_size()
    xelem = R.x.element_size()
    per_set = R.values.numel() * elem + (R.x.numel() + R.rows) * xelem
    nsets = sets or max(3, -(-2 * MALL_BYTES // per_set))
    bufs = []
    for _ in range(nsets):
        vals = R.values.clone()
        x = R.x.clone()
        y = torch.empty(R.rows, dtype=xdtype, device="cuda")
        # the view holds raw pointers: the set keeps its values tensor alive
        # (else its memory returns to the allocator and later sets' x and y
        # land in it)
        bufs.append((recon_view(R.offsets, vals, R.rows, R.cols), x, y, vals))
    lib = _lib.load()
    fn = getattr(lib, _SPMV[(dtype, xdtype)])
    stream = torch.cuda.current_stream()
    sh = _stream_handle(stream)

    def step(i):
        v, x, y, _ = bufs[i % nsets]
        st = fn(C.byref(v), x.data_ptr(), x.numel(), y.data_ptr(), sh)
        if st:
            _lib.check(st)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    gpu_spin(stream)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    alg = spmv_alg_bytes(R, elem, xelem)
    flops = 2 * R.useful_terms() * (4 if dtype == torch.complex64 else
                                     2 if xdtype == torch.complex64 else 1)
    return {
        "R": R, "ms": ms, "alg_bytes": alg, "flops": flops, "sets": nsets,
        "set_bytes": per_set, "gbs": alg / (ms * 1e6), "gflops": flops / (ms * 1e6),
        "y": bufs[(steps - 1) % nsets][2] if steps else None,
    }


def host_cores() -> dict:
    """Host CPUs this process may run on: logical CPUs in its affinity mask,
    the physical cores (distinct package and core ids in sysfs) behind them,
    and the machine's logical CPU count."""
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        cpus = list(range(os.cpu_count() or 1))
    cores = set()
    for c in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            cores.add(((base / "physical_package_id").read_text().strip(),
                       (base / "core_id").read_text().strip()))
        except OSError:
            cores.add(("?", str(c)))
    return {"logical_cpus": len(cpus), "physical_cores": len(cores),
            "machine_logical_cpus": os.cpu_count()}


def cpu_spmv_baseline(R, seconds: float, y_gpu=None):
    """The oracle's OpenMP DIA loop over full SpMVs of the same matrix on the
    host cores, repeated until `seconds` elapse (1 warm-up run first).  With
    y_gpu (the GPU's y for the same matrix and x), the CPU leg also checks
    it, as the reference bench prints its difference from the CPU result
    (spmv/bench/bench_cusparse.cu:220-230): every row against the oracle's
    fp64 sum within tol * sum |terms| (1e-5 fp32, 1e-13 fp64), and the
    largest difference from the CPU loop's own y."""
    import numpy as np
    from oracle import binding as orc

    off = R.offsets.cpu().numpy()
    vals = R.values.cpu().numpy()
    x = R.x.cpu().numpy()
    y = np.empty(R.rows, dtype=vals.dtype)
    threads = orc.spmv_recon_omp(R.rows, R.cols, off, vals, x, y)
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.spmv_recon_omp(R.rows, R.cols, off, vals, x, y)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= 3:
            break
    ms = el * 1e3 / reps
    out = {"ms": ms, "threads": threads, "reps": reps,
           "gbs": spmv_alg_bytes(R, vals.itemsize) / (ms * 1e6)}
    if y_gpu is not None:
        g = y_gpu.cpu().numpy().astype(np.float64)
        y64, ab = orc.spmv_recon_ref64(R.rows, R.cols, off, vals, x)
        tol = 1e-13 if vals.dtype == np.float64 else 1e-5
        err = np.abs(g - y64)
        out["check"] = {
            "rows": int(R.rows),
            "max_err_over_term_sum": float(np.max(np.where(ab > 0, err / np.where(ab > 0, ab, 1), 0.0))),
            "tol": tol, "ok": bool(np.all(err <= tol * ab + 1e-300)),
            "max_abs_diff_vs_cpu": float(np.max(np.abs(g - y.astype(np.float64)))),
        }
    return out


def spmv_cpu_record(R, res, seconds: float, what: str) -> dict:
    """cpu_baseline object for an SpMV record (with the output check)."""
    c = cpu_spmv_baseline(R, seconds, res.get("y"))
    rec = {"value": round(c["gbs"], 2), "unit": "GB/s", "cores": c["threads"],
           **host_cores(), "kind": "port",
           "sample": f"{c['reps']} full SpMVs of {what} with the oracle's OpenMP DIA loop, "
                     f"{c['ms']:.3f} ms each"}
    if "check" in c:
        rec["check"] = c["check"]
    return rec


def load_traffic(name: str):
    """HBM bytes per launch measured offline with rocprofv3 --pmc
    (profiles/<name>_traffic.json), or None."""
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except (ValueError, OSError):
            return None
    return None


def spmv_record(cfg, dtype, res, xdtype=None):
    R = res["R"]
    names = {"torch.float32": "f32", "torch.float64": "f64", "torch.complex64": "c64"}
    vt = names[str(R.values.dtype)]
    xt = names[str(R.x.dtype)]
    return {
        "workload": f"spmv_cfg{cfg}",
        "dtype": vt if vt == xt else f"{vt}x{xt}",
        "n": R.rows, "K": R.K, "ms": round(res["ms"], 6),
        "GBs": round(res["gbs"], 1), "frac_hbm": round(res["gbs"] / HBM_PEAK_GBS, 4),
        "GFLOPs": round(res["gflops"], 1), "alg_bytes": res["alg_bytes"],
        "buffer_sets": res["sets"],
    }


def time_krylov(m: int = 30, t: float = 1.0, reps: int = 5):
    """exp(-i t H) psi_0 by Lanczos on config 2's 5-point stencil (real
    symmetric H, n = 2^22) with a complex state: one call = m SpMV+dot steps,
    m update+norm steps, one host sync and the combine pass."""
    import torch
    from diagpu_amd import workloads
    from diagpu_amd.krylov import expm_krylov, KrylovWorkspace
    R = workloads.spmv_config(2, seed=1, device="cuda", dtype=torch.float32)
    n = R.rows
    g = torch.Generator(device="cuda").manual_seed(1)
    psi0 = torch.complex(torch.randn(n, device="cuda", generator=g),
                         torch.randn(n, device="cuda", generator=g)).contiguous()
    ws = KrylovWorkspace(n, m)
    out = torch.empty_like(psi0)
    expm_krylov(R.offsets, R.values, n, psi0, t, m, out=out, workspace=ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        res = expm_krylov(R.offsets, R.values, n, psi0, t, m, out=out, workspace=ws)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    # algorithmic bytes: per step SpMV (values 4 B, x and y 8 B, x re-read by
    # the dot) + update (z, u_j, u_{j-1} read, z written); norm of psi_0 and
    # the combine (m vectors read, one written)
    spmv = 4 * R.useful_terms() + 8 * 3 * n
    upd = 8 * 4 * n
    alg = m * (spmv + upd) + 8 * n + 8 * (m + 1) * n
    return {"workload": "expm_krylov_cfg2", "n": n, "m": m, "t": t, "steps_used": res.steps,
            "err_estimate": res.err_estimate, "ms_per_call": round(ms, 4),
            "us_per_step": round(ms * 1e3 / m, 2), "alg_bytes": alg,
            "GBs": round(alg / (ms * 1e6), 1), "frac_hbm": round(alg / (ms * 1e6) / HBM_PEAK_GBS, 4)}


# --------------------------------------------------------------------------
# SpGEMM (configs 4 and 5)
# --------------------------------------------------------------------------

def cpu_spgemm_baseline(plan, A, B, seconds: float, C_gpu=None):
    """The oracle's OpenMP SpGEMM loop (schedule(dynamic) over C diagonals,
    each C diagonal's pairs resolved once, fp32 accumulation) on the host
    cores, over a bounded prefix of C diagonals (about `seconds` of work,
    growing the prefix until it takes at least a tenth of that); GFLOP/s and
    GB/s from the sample's own useful flops and algorithmic bytes.

    With C_gpu (the GPU's C for the same plan and operands) the CPU leg also
    checks it, as the reference bench prints each kernel's difference from
    the CPU result (spmspm/bench_spmspm.cu:779-796): up to 8 windows of C
    diagonals spread over the sampled prefix (about 2^20 values each)
    against the oracle's fp64 sum within 1e-5 * sum |terms|, and against
    the CPU loop's own fp32 values."""
    import numpy as np
    from oracle import binding as orc
    Av = A.values.cpu().numpy()
    Bv = B.values.cpu().numpy()
    c_len = plan.c_lengths().cpu().numpy().astype(np.int32)
    c_st = plan.c_starts().cpu().numpy()
    ptr = plan.pair_ptr().cpu().numpy()
    pairs = plan.pairs_numpy()
    nC = len(c_len)
    counts = np.diff(ptr)
    # useful flops per C diagonal: 2 * sum over its pairs of the overlap
    ov = (np.minimum(pairs["al"] - pairs["ash"], pairs["bl"] - pairs["bsh"])
          - np.maximum(0, np.maximum(-pairs["ash"], -pairs["bsh"])))
    ov = np.minimum(ov, np.repeat(c_len.astype(np.int64), counts)).clip(min=0)
    fl_k = 2 * np.add.reduceat(ov.astype(np.int64), ptr[:-1]) if nC else np.zeros(0)
    k = max(1, min(nC, 64))
    while True:
        out = np.empty(int(c_st[k - 1] + c_len[k - 1] - c_st[0]), np.float32)
        t0 = time.perf_counter()
        threads = orc.spgemm_pairs_omp_f32(Av, Bv, c_len, c_st, ptr, pairs, 0, k, out)
        el = time.perf_counter() - t0
        if el >= seconds / 10 or k == nC:
            break
        k = min(nC, k * 4)
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.spgemm_pairs_omp_f32(Av, Bv, c_len, c_st, ptr, pairs, 0, k, out)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 3 and el >= seconds / 2:
            break
    sec = el / reps
    flops = float(fl_k[:k].sum())
    # bytes: the sample's C values once plus the A and B values its pairs read
    byt = 4 * (2 * float(ov[: ptr[k]].sum()) + out.size)
    rec = {"value": round(flops / sec / 1e9, 2), "unit": "GFLOP/s", "GBs": round(byt / sec / 1e9, 2),
           "cores": threads, **host_cores(), "kind": "port",
           "sample": f"C diagonals 0..{k - 1} of {nC} ({100.0 * flops / max(1.0, float(fl_k.sum())):.1f}% "
                     f"of the flops), {reps} runs of {sec * 1e3:.1f} ms, oracle OpenMP loop"}
    if C_gpu is not None and k > 0:
        windows, e_prev = [], 0
        for s0 in np.unique(np.linspace(0, k - 1, min(k, 8)).astype(np.int64)):
            s0 = max(int(s0), e_prev)
            if s0 >= k:
                continue
            e = s0 + 1
            while e < k and c_st[e] + c_len[e] - c_st[s0] <= 1 << 20:
                e += 1
            windows.append((s0, e))
            e_prev = e
        worst, worst_cpu, nvals, ok = 0.0, 0.0, 0, True
        for s0, e in windows:
            lo, hi = int(c_st[s0]), int(c_st[e - 1] + c_len[e - 1])
            ref, ab = orc.spgemm_pairs_f64(Av, Bv, c_len, c_st, ptr, pairs, s0, e)
            g = C_gpu[lo:hi].cpu().numpy().astype(np.float64)
            err = np.abs(g - ref)
            ok &= bool(np.all(err <= 1e-5 * ab + 1e-30))
            worst = max(worst, float(np.max(np.where(ab > 0, err / np.where(ab > 0, ab, 1), 0.0))))
            cpu = out[lo - int(c_st[0]): hi - int(c_st[0])].astype(np.float64)
            worst_cpu = max(worst_cpu, float(np.max(np.abs(g - cpu))))
            nvals += hi - lo
        rec["check"] = {"windows": [[int(a), int(b)] for a, b in windows], "values": int(nvals),
                        "max_err_over_term_sum": worst, "tol": 1e-5, "ok": ok,
                        "max_abs_diff_vs_cpu": worst_cpu}
    return rec


def kernel_legs(plan, complex_values: bool = False) -> list[str]:
    """Every numeric kernel that takes this plan."""
    from diagpu_amd import _lib
    names = ["gather"]
    if not complex_values and plan.band_info()[1].eligible:
        names.append("band")
    if not complex_values and plan.band_info()[1].mfma_eligible:
        names.append("band_mfma")
    if plan.A.offsets.numel() <= (_lib.ASTAT_MAX_A_C64 if complex_values else _lib.ASTAT_MAX_A):
        try:
            plan.astat_records()
            names.append("astat")
        except _lib.DiagpuError:
            pass
    return names


CHECK_BYTES = 24 << 30     # C sizes whose outputs are compared bit for bit on the GPU


def compare_kernels(plan, sets, reps: int, alg: int, flops: int, complex_values: bool = False,
                    rounds: int = 10) -> tuple[dict, dict]:
    """The automatic choice and every numeric kernel that takes this plan
    (fp32 or complex64 values), forced, on the same rotated operand sets
    (the side-by-side run of spmspm/bench_spmspm.cu:518-653), timed in
    interleaved rounds (auto, k1, k2, ...; the order rotated by one leg each
    round, so every leg leads as many rounds, and reversed every other
    round, so every leg follows two different legs; each round opened behind
    a spin so the first leg's launch latency stays out of its window; reps /
    rounds products per leg per round) and reported as the median over
    rounds of the time per product, with GFLOP/s, the fraction of HBM peak,
    and whether C is bit for bit the gather's (where C fits CHECK_BYTES).
    The MFMA band kernel, opt-in and never the automatic choice, is timed
    in rounds of its own after the others: the launch that followed it ran
    up to 45 % slower (the A-stationary kernel on gemm_diag's band at n =
    2^20: 115 against 79 us for the launch after it), which would charge its
    neighbour in the interleaved order.
    Returns (auto record, {kernel: record})."""
    import statistics
    import torch
    names = kernel_legs(plan, complex_values)
    legs = ["auto"] + [k for k in names if k != "band_mfma"]
    alone = [k for k in names if k == "band_mfma"]
    stream = torch.cuda.current_stream()
    nsets = len(sets)
    rounds = max(1, min(rounds, reps))
    per = max(1, reps // rounds)
    for k in legs + alone:
        for i in range(2):
            plan.numeric(*sets[i % nsets], kernel=k)
    torch.cuda.synchronize()
    times = {k: [] for k in legs + alone}
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * len(legs))]

    # one counter over every launch, whatever its leg: consecutive launches
    # read different sets, so no leg reads a set the leg before it has just
    # brought into the MALL (with a per-leg index, each leg's second product
    # read the set its predecessor read last)
    launch = [0]

    def run_rounds(order_of):
        for r in range(rounds):
            gpu_spin(stream, 100.0)
            order = order_of(r)
            for j, k in enumerate(order):
                ev[2 * j].record(stream)
                for i in range(per):
                    plan.numeric(*sets[launch[0] % nsets], kernel=k)
                    launch[0] += 1
                ev[2 * j + 1].record(stream)
            torch.cuda.synchronize()
            for j, k in enumerate(order):
                times[k].append(ev[2 * j].elapsed_time(ev[2 * j + 1]) / per)

    def interleaved(r):
        # rounds 2s and 2s + 1: the order rotated by s legs, forward then
        # reversed (each leg leads about as many rounds either way)
        s = (r // 2) % len(legs)
        order = legs[s:] + legs[:s]
        return order[::-1] if r % 2 else order
    run_rounds(interleaved)
    for k in alone:
        run_rounds(lambda r, k=k: [k])
    esz = 8 if complex_values else 4
    check = plan.info.c_nnz * esz <= CHECK_BYTES
    ref = None
    out = {}
    for k in ["gather"] + [x for x in legs + alone if x != "gather"]:
        kms = statistics.median(times[k])
        rec = {"numeric_ms": round(kms, 5), "GFLOPs": round(flops / (kms * 1e6), 1),
               "frac_hbm": round(alg / (kms * 1e6) / HBM_PEAK_GBS, 4),
               "min_ms": round(min(times[k]), 5), "max_ms": round(max(times[k]), 5),
               "rounds": rounds, "products_per_round": per, "same_bits_as_gather": None}
        if k == "band_mfma":
            rec["mfma_utilisation"] = round(plan.mfma_utilisation(), 4)
            rec["mfma_blocks_per_16_rows"] = plan.band_info()[1].mfma_blocks
        if check:
            plan.numeric(*sets[0], kernel=k)
            torch.cuda.synchronize()
            c = sets[0][2][: plan.info.c_nnz]
            c = torch.view_as_real(c) if complex_values else c
            if ref is None:
                ref = c.clone()
            rec["same_bits_as_gather"] = bool(torch.equal(ref.view(torch.int32), c.view(torch.int32)))
            if not rec["same_bits_as_gather"]:
                rec["max_abs_diff_vs_gather"] = float((c - ref).abs().max())
        out[k] = rec
    del ref
    auto = out.pop("auto")
    return auto, out


def mfma_record(plan) -> dict:
    """Whether the fp32 MFMA band kernel (dense 16x16x4 tiles over the band)
    takes this plan, its utilisation if so, and the reason if not."""
    bi = plan.band_info()[1]
    if bi.mfma_eligible:
        return {"eligible": True, "utilisation": round(plan.mfma_utilisation(), 4),
                "blocks_per_16_rows": bi.mfma_blocks}
    na, nb = plan.A.offsets.numel(), plan.B.offsets.numel()
    sa = bi.a_off_max - bi.a_off_min
    sb = bi.b_off_max - bi.b_off_min
    dens = (na / (sa + 1)) * (nb / (sb + 1))
    return {"eligible": False,
            "reason": (f"A's {na} offsets span {sa + 1} columns and B's {nb} span {sb + 1} "
                       f"(the MFMA band kernel takes A spans up to 32 and A + B up to 48): "
                       f"a dense tile contraction over this band would find "
                       f"{100 * dens:.3g}% of its multiply-adds useful (about "
                       f"{1 / max(dens, 1e-12):.0f} issued per useful one), and C has "
                       f"{plan.info.n_pairs / max(1, plan.info.c_ndiag):.2f} plan entries per "
                       f"diagonal, so there is no dense tile to give the matrix cores"),
            "a_span": sa + 1, "b_span": sb + 1, "useful_fraction_dense": dens}


def time_spgemm(cfg: int, seed: int, reps: int, complex_values: bool = False,
                cpu_seconds: float = 0.0, operands=None, name: str | None = None,
                rounds: int = 10):
    """One SpGEMM configuration: the plan (symbolic phase timed on the
    device), then compare_kernels over rotated operand sets, the CPU
    baseline with its output check, and the MFMA record.  operands: (A, B)
    (default: benchmark config `cfg`)."""
    import torch
    from diagpu_amd import workloads
    from diagpu_amd.spgemm import SpgemmPlan
    if operands is None:
        A, B = workloads.spgemm_config(cfg, seed=seed, device="cuda")
    else:
        A, B = operands
    if complex_values:   # same structure, values v + i * roll(v)
        A = workloads.HM(A.n, A.offsets, A.lengths, A.starts,
                         torch.complex(A.values, torch.roll(A.values, 1)).contiguous())
        B = workloads.HM(B.n, B.offsets, B.lengths, B.starts,
                         torch.complex(B.values, torch.roll(B.values, 1)).contiguous())
    esz = A.values.element_size()
    stream = torch.cuda.current_stream()
    t0 = time.perf_counter()
    plan = SpgemmPlan(A, B)
    torch.cuda.synchronize()
    sym_wall_ms = (time.perf_counter() - t0) * 1e3
    # symbolic phase: a synchronous call (it returns with the counts on the
    # host), timed as a caller waits for it, 20 calls each timed (median;
    # the mean beside it); beside them the HIP-event span of 3 calls on the
    # stream (which also counts the idle stream while each call's launch
    # travels from the host)
    for _ in range(2):
        plan.symbolic()
    torch.cuda.synchronize()
    sym_calls = []
    for _ in range(20):
        t0 = time.perf_counter()
        plan.symbolic()
        sym_calls.append((time.perf_counter() - t0) * 1e3)
    sym_ms = statistics.median(sym_calls)
    sym_mean_ms = statistics.fmean(sym_calls)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(3):
        plan.symbolic()
    e1.record(stream)
    torch.cuda.synchronize()
    sym_ev_ms = e0.elapsed_time(e1) / 3
    # operand/result sets rotated so that together they exceed twice the MALL
    set_bytes = esz * (A.nnz + B.nnz + plan.info.c_nnz)
    nsets = 1 if set_bytes >= 2 * MALL_BYTES else max(3, -(-2 * MALL_BYTES // set_bytes))
    sets = [(A.values.clone(), B.values.clone(),
             torch.empty(plan.info.c_nnz, dtype=A.values.dtype, device="cuda"))
            for _ in range(nsets)]
    alg = esz * (A.nnz + B.nnz + plan.info.c_nnz)
    flops = plan.info.useful_flops * (4 if complex_values else 1)   # complex MAC = 4 real
    auto, kernels = compare_kernels(plan, sets, reps, alg, flops, complex_values, rounds)
    ms = auto["numeric_ms"]
    kern = plan.kernel_for(torch.complex64 if complex_values else torch.float32)
    rec = {
        "workload": name or (f"spgemm_cfg{cfg}" if cfg >= 4 else f"spgemm_HxH_cfg{cfg}"),
        "dtype": "c64" if complex_values else "f32", "n": A.n,
        "A_diags": A.ndiag, "B_diags": B.ndiag, "C_diags": plan.info.c_ndiag,
        "pairs": plan.info.n_pairs, "max_pairs_per_C": plan.info.max_pairs,
        "C_nnz": plan.info.c_nnz, "numeric_ms": round(ms, 5),
        "numeric_min_ms": auto["min_ms"], "numeric_max_ms": auto["max_ms"],
        "kernel": kern,
        "symbolic_ms": round(sym_ms, 5), "symbolic_mean_ms": round(sym_mean_ms, 5),
        "symbolic_event_span_ms": round(sym_ev_ms, 5),
        "symbolic_wall_ms_first": round(sym_wall_ms, 3),
        "GFLOPs": round(flops / (ms * 1e6), 1), "useful_flops": flops,
        "GBs": round(alg / (ms * 1e6), 1), "frac_hbm": round(alg / (ms * 1e6) / HBM_PEAK_GBS, 4),
        "alg_bytes": alg, "buffer_sets": nsets,
        "total_ms": round(ms + sym_ms, 5),
        "kernels": kernels,
    }
    if not complex_values:
        rec["mfma"] = mfma_record(plan)
    if cpu_seconds > 0 and not complex_values:
        plan.numeric(*sets[0])               # the automatic kernel's C, checked by the CPU leg
        torch.cuda.synchronize()
        rec["cpu_baseline"] = cpu_spgemm_baseline(
            plan, workloads.HM(A.n, A.offsets, A.lengths, A.starts, sets[0][0]),
            workloads.HM(B.n, B.offsets, B.lengths, B.starts, sets[0][1]), cpu_seconds,
            C_gpu=sets[0][2])
    else:
        rec["cpu_baseline"] = None
    return rec


def time_spgemm_banded(reps: int, cpu_seconds: float):
    """The reference SpGEMM bench's own operands (spmspm/bench_spmspm.cu:
    455-471): A = make_banded(100000, 16, 1234), B = make_banded(100000, 16,
    5678), 33 diagonals each, C on 65 diagonals; the reference times its
    kernels on this product (:518-653)."""
    from diagpu_amd import workloads
    n, w = 100_000, 16
    A = workloads.make_banded(n, w, 1234, device="cuda")
    B = workloads.make_banded(n, w, 5678, device="cuda")
    return time_spgemm(0, 0, reps, cpu_seconds=cpu_seconds, operands=(A, B),
                       name=f"spgemm_make_banded_n{n}_w{w}")


def time_taylor(order: int = 6, t: float = 0.05, chains: int = 9):
    """Taylor chain exp(tH) ~ sum_k (tH)^k/k! on the 7-point stencil of SpGEMM
    config 4 (n = 2^20): one warm-up chain, then `chains` chains each timed
    as a caller runs it (total_ms: their median), then one chain whose
    phases are stream-synchronised for the split (the plan of every product
    is built on the device)."""
    import torch
    from diagpu_amd import chain, workloads
    H = workloads.hm_stencil7(128, 128, 64, device="cuda")
    chain.taylor_expm(H, t, order)
    times = []
    for _ in range(chains):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        chain.taylor_expm(H, t, order)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    total = statistics.median(times)
    # the matrix-power chain H^6 on the same stencil: plans built beside the
    # products (chain.power), and each plan on the caller's stream after the
    # product before it (chain.multiply in a loop), medians of `chains` each
    def timed(fn):
        ts = []
        for _ in range(chains):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    def serial_power():
        P = H
        for _ in range(order - 1):
            P = chain.multiply(H, P)
        return P
    chain.power(H, order)
    serial_power()
    power_ms = timed(lambda: chain.power(H, order)) * 1e3
    power_serial_ms = timed(serial_power) * 1e3
    st = chain.ChainStats()
    t0 = time.perf_counter()
    S = chain.taylor_expm(H, t, order, st)
    torch.cuda.synchronize()
    total_split = time.perf_counter() - t0
    steps = [{"k": k + 2, "C_diags": st.c_ndiag[k], "pairs": st.n_pairs[k],
              "symbolic_ms": round(st.symbolic[k] * 1e3, 3),
              "numeric_ms": round(st.numeric[k] * 1e3, 3),
              "GFLOPs": round(st.useful_flops[k] / (st.numeric[k] * 1e9), 1)}
             for k in range(len(st.numeric))]
    flops = sum(st.useful_flops)
    return {"workload": "taylor_expm_stencil7_cfg4", "n": H.n, "order": order, "t": t,
            "S_diags": S.ndiag, "S_nnz": S.nnz, "total_ms": round(total * 1e3, 3),
            "total_min_ms": round(min(times) * 1e3, 3), "total_max_ms": round(max(times) * 1e3, 3),
            "chains": chains, "total_ms_phase_synced": round(total_split * 1e3, 3),
            "power_ms": round(power_ms, 3), "power_serial_ms": round(power_serial_ms, 3),
            "symbolic_ms": round(sum(st.symbolic) * 1e3, 3),
            "numeric_ms": round(sum(st.numeric) * 1e3, 3),
            "axpby_ms": round(sum(st.axpby) * 1e3, 3),
            "numeric_GFLOPs": round(flops / (sum(st.numeric) * 1e9), 1),
            "steps": steps}


def time_propagator(grid: str = "3d", order: int = 6, dt: float = 0.02, m: int = 12,
                    reps: int = 20):
    """The two propagation workflows of slides/transcript.md:10-18: build
    U = exp(-i dt H) once (complex Taylor chain + device HM->Recon) and apply
    it by the complex SpMV, against one Lanczos call per time step on H
    itself.  grid "3d": the 7-point stencil of SpGEMM config 4 (n = 2^20;
    U has 377 diagonals at order 6); "2d": config 2's 5-point stencil
    (n = 2^22; 85 diagonals).  Break-even = the number of steps after which
    building U has paid off."""
    import torch
    from diagpu_amd import chain, workloads
    from diagpu_amd.krylov import expm_krylov, KrylovWorkspace
    from diagpu_amd.spmv import spmv_recon
    if grid == "3d":
        H = workloads.hm_stencil7(128, 128, 64, device="cuda")
        name = "propagator_stencil7_cfg4"
    elif grid == "2d":
        H = workloads.recon_to_hm(workloads.spmv_config(2, seed=1, device="cuda"))
        name = "propagator_poisson5_cfg2"
    else:
        raise ValueError(f"unknown grid {grid}")
    n = H.n
    chain.to_recon(chain.propagator(H, dt, order))          # warm-up (plans, allocator)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    U = chain.propagator(H, dt, order)
    u_off, u_val = chain.to_recon(U)
    torch.cuda.synchronize()
    build_ms = (time.perf_counter() - t0) * 1e3
    del U
    g = torch.Generator(device="cuda").manual_seed(4)
    psi = torch.complex(torch.randn(n, device="cuda", generator=g),
                        torch.randn(n, device="cuda", generator=g)).contiguous()
    y = torch.empty_like(psi)
    for _ in range(3):
        spmv_recon(u_off, u_val, n, n, psi, y)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        spmv_recon(u_off, u_val, n, n, psi, y)
    e1.record()
    torch.cuda.synchronize()
    apply_ms = e0.elapsed_time(e1) / reps
    K = u_off.numel()
    apply_bytes = 8 * K * n + 8 * 2 * n                    # U values + x + y (padding included)
    h_off, h_val = chain.to_recon(H)
    ws = KrylovWorkspace(n, m)
    out = torch.empty_like(psi)
    expm_krylov(h_off, h_val, n, psi, dt, m, out=out, workspace=ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        res = expm_krylov(h_off, h_val, n, psi, dt, m, out=out, workspace=ws)
    torch.cuda.synchronize()
    kry_ms = (time.perf_counter() - t0) * 1e3 / reps
    nrm = torch.linalg.vector_norm(psi.to(torch.complex128)).item()
    rel = torch.linalg.vector_norm((y - out).to(torch.complex128)).item() / nrm
    return {"workload": name, "n": n, "order": order, "dt": dt,
            "U_diags": K, "U_bytes": 8 * K * n, "build_ms": round(build_ms, 3),
            "apply_ms": round(apply_ms, 4),
            "apply_GBs": round(apply_bytes / (apply_ms * 1e6), 1),
            "apply_frac_hbm": round(apply_bytes / (apply_ms * 1e6) / HBM_PEAK_GBS, 4),
            "krylov_m": m, "krylov_ms": round(kry_ms, 4), "krylov_steps": res.steps,
            "krylov_err_estimate": res.err_estimate, "rel_diff_U_vs_krylov": rel,
            "break_even_steps": (round(build_ms / (kry_ms - apply_ms), 1)
                                 if kry_ms > apply_ms else None)}


def time_gemm_diag(n: int = 4096, hb: int = 10, reps: int = 100, cpu_seconds: float = 0.0,
                   rotate: bool = False):
    """gemm_diag on row-packed operands (gemm_diag/gemm_diag.cu:9-15) with the
    reference driver's default shape (n = 4096, offsets -hb..hb, values
    U(0.5, 1.5), gemm_diag.cu:467-486): the plan once, then the automatic
    choice and every kernel that takes the plan in interleaved rounds of
    `reps` products each (compare_kernels), including the fp32 MFMA band
    kernel with its utilisation (useful / issued flops from its tile
    geometry).  One operand set, as the reference driver times its
    products, or with `rotate` the bench's rotated sets of at least twice
    the MALL (each product on operands no recent product touched): at n =
    2^20 one set (348 MB) stays partly in the 256 MB MALL, which favoured
    the A-stationary kernel (79 against 94 us for the band kernel; rotated,
    118 against 97 on compact operands of the same band).  The reference kernel has no
    tensor-core instructions (products in shared memory, a sequential
    reduction and atomicAdd).  With cpu_seconds > 0 the oracle's OpenMP
    SpGEMM loop runs the same plan over the same row-packed operands on the
    host cores beside it."""
    import types
    import torch
    from diagpu_amd.spgemm import gemm_diag
    offs = list(range(-hb, hb + 1))
    g = torch.Generator(device="cuda").manual_seed(42)

    def packed():
        D = torch.rand(len(offs), n, generator=g, device="cuda") + 0.5
        t = torch.arange(n, device="cuda")
        for i, d in enumerate(offs):       # zero where the row t + d leaves the matrix
            D[i].masked_fill_((t + d < 0) | (t + d >= n), 0)
        return D.reshape(-1).contiguous()
    off = torch.tensor(offs, dtype=torch.int32, device="cuda")
    DA, DB = packed(), packed()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan, C = gemm_diag(n, off, DA, off, DB)
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1e3
    nnz = sum(n - abs(d) for d in offs)
    alg = 4 * (2 * nnz + plan.info.c_nnz)
    flops = plan.info.useful_flops
    sets = [(DA, DB, C)]
    if rotate:
        set_bytes = 4 * (DA.numel() + DB.numel() + C.numel())
        nsets = 1 if set_bytes >= 2 * MALL_BYTES else max(3, -(-2 * MALL_BYTES // set_bytes))
        sets += [(DA.clone(), DB.clone(), torch.empty_like(C)) for _ in range(nsets - 1)]
    auto, kernels = compare_kernels(plan, sets, reps, alg, flops)
    ms = auto["numeric_ms"]
    kern = plan.kernel_for()
    rec = {"workload": f"gemm_diag_n{n}_hb{hb}", "n": n, "A_diags": len(offs),
           "B_diags": len(offs), "C_diags": plan.info.c_ndiag, "numeric_ms": round(ms, 5),
           "numeric_min_ms": auto["min_ms"], "numeric_max_ms": auto["max_ms"],
           "kernel": kern, "first_call_ms": round(first_ms, 3),
           "GFLOPs": round(flops / (ms * 1e6), 1),
           "GBs": round(alg / (ms * 1e6), 1), "frac_hbm": round(alg / (ms * 1e6) / HBM_PEAK_GBS, 4),
           "alg_bytes": alg,
           # useful / issued flops of the kernel that ran; None when that kernel
           # issues no MFMA (the MFMA band kernel's figure is under kernels)
           "mfma_utilisation": (round(plan.mfma_utilisation(), 4) if kern == "band_mfma" else None),
           "mfma": mfma_record(plan),
           "kernels": kernels, "cpu_baseline": None}
    if cpu_seconds > 0:
        plan.numeric(DA, DB, C)
        torch.cuda.synchronize()
        # the plan's pair starts index the row-packed arrays directly
        rec["cpu_baseline"] = cpu_spgemm_baseline(plan, types.SimpleNamespace(values=DA),
                                                  types.SimpleNamespace(values=DB), cpu_seconds,
                                                  C_gpu=C)
    return rec


def launch_floor(reps: int = 400) -> dict:
    """Time per launch of back-to-back near-empty kernels (torch's spin
    kernel with 0 cycles) on one stream, by HIP events: the floor under any
    single-launch product, for reading the launch-bound lines (config 1's
    SpMV and square, gemm_diag at n = 4096)."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(20):
        torch.cuda._sleep(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gpu_spin(stream)
    e0.record(stream)
    for _ in range(reps):
        torch.cuda._sleep(0)
    e1.record(stream)
    torch.cuda.synchronize()
    return {"workload": "launch_floor", "kernel": "torch spin kernel, 0 cycles", "launches": reps,
            "us_per_launch": round(e0.elapsed_time(e1) * 1e3 / reps, 3)}


def copy_calibration(steps: int):
    """A plain device copy of known size, for scaling rocprof FETCH/WRITE counters."""
    import torch
    nbytes = 1 << 30
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").normal_()
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"workload": "copy_1GiB", "bytes_read": nbytes, "bytes_written": nbytes, "ms": ms,
            "GBs": 2 * nbytes / (ms * 1e6)}


def fill_calibration(steps: int, nbytes: int = 20_000_000_000):
    """A plain device fill of known size (torch's vectorized fill kernel), for
    checking the WRITE_SIZE counter at the size of a large C (the square of
    config 3 writes 20.0 GB)."""
    import torch
    buf = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    for _ in range(2):
        buf.fill_(1.0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        buf.fill_(1.0)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"workload": f"fill_{nbytes}", "bytes_written": nbytes, "ms": ms,
            "GBs": nbytes / (ms * 1e6)}


# --------------------------------------------------------------------------

def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a code path)"}))
        return 2
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2
    from diagpu_amd import _lib, workloads
    _lib.load()

    if args.only:
        w = args.only
        if w == "copy":
            print(json.dumps(copy_calibration(args.steps)), flush=True)
        elif w == "fill20":
            print(json.dumps(fill_calibration(args.steps)), flush=True)
        elif w == "launch":
            print(json.dumps(launch_floor()), flush=True)
        elif w == "spmvhash":
            R = workloads.hash_band(device="cuda")
            res = time_spmv(0, torch.float32, args.steps, args.warmup, args.seed, args.sets, R=R)
            rec = spmv_record(0, torch.float32, res)
            rec["workload"] = "spmv_hash_band_N1048576"
            print(json.dumps(rec), flush=True)
        elif w == "spgemmbanded":
            print(json.dumps(time_spgemm_banded(args.steps, 0.0)), flush=True)
        elif w.startswith("spmv"):
            cfg = int(w[4])
            suffix = w[5:]
            dt, xt = {"": (torch.float32, None), "d": (torch.float64, None),
                      "c": (torch.complex64, None),
                      "rc": (torch.float32, torch.complex64)}[suffix]
            res = time_spmv(cfg, dt, args.steps, args.warmup, args.seed, args.sets, xt)
            print(json.dumps(spmv_record(cfg, dt, res, xt)), flush=True)
        elif w == "krylov":
            print(json.dumps(time_krylov()), flush=True)
        elif w.startswith("spgemm"):
            print(json.dumps(time_spgemm(int(w[6]), args.seed, args.steps, w.endswith("c"))),
                  flush=True)
        elif w == "taylor":
            print(json.dumps(time_taylor()), flush=True)
        elif w == "propagator":
            print(json.dumps(time_propagator("3d")), flush=True)
        elif w == "propagator2d":
            print(json.dumps(time_propagator("2d")), flush=True)
        elif w == "gemmdiag":
            print(json.dumps(time_gemm_diag()), flush=True)
        elif w == "gemmdiag20":
            print(json.dumps(time_gemm_diag(1 << 20, 10, 20, rotate=True)), flush=True)
        else:
            raise SystemExit(f"unknown --only {w}")
        return 0

    log(f"headline: SpMV config 2 fp32, {args.steps} steps after {args.warmup} warm-up")
    head = time_spmv(2, torch.float32, args.steps, args.warmup, args.seed, args.sets)
    R = head["R"]
    log(f"headline: {head['ms'] * 1e3:.2f} us/step, {head['gbs']:.1f} GB/s")

    cpu = None
    if args.cpu_seconds > 0:
        log(f"CPU baseline ({args.cpu_seconds:.0f} s budget)")
        cpu = spmv_cpu_record(R, head, args.cpu_seconds,
                              "the config-2 matrix (n=4194304, fp32)")
        cpu["sample"] += f", {os.cpu_count()} logical CPUs visible"
        log(f"CPU baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads, "
            f"GPU output check ok={cpu.get('check', {}).get('ok')}")
    head.pop("y", None)

    extras = {}
    if args.extras:
        for cfg, dt, xt in [(1, torch.float32, None), (2, torch.float64, None),
                            (3, torch.float32, None), (2, torch.complex64, None),
                            (2, torch.float32, torch.complex64)]:
            try:
                res = time_spmv(cfg, dt, 200, 20, args.seed, 0, xt)
                rec = spmv_record(cfg, dt, res, xt)
                if xt is None and dt != torch.complex64 and args.cpu_seconds > 0:
                    rec["cpu_baseline"] = spmv_cpu_record(
                        res["R"], res, min(2.0, args.cpu_seconds),
                        f"the config-{cfg} matrix ({rec['dtype']}, accumulation in "
                        f"{'fp64' if dt == torch.float64 else 'fp32'})")
                extras[f"spmv_cfg{cfg}_{rec['dtype']}"] = rec
                log(f"extra spmv cfg{cfg} {rec['dtype']}: {res['gbs']:.1f} GB/s")
                del res
                torch.cuda.empty_cache()
            except Exception as e:  # report, keep the headline
                extras[f"spmv_cfg{cfg}_{dt}_{xt}"] = {"error": repr(e)}
        # warm (MALL-resident) headline: one buffer set, the same matrix
        try:
            res = time_spmv(2, torch.float32, 400, 40, args.seed, 1)
            rec = spmv_record(2, torch.float32, res)
            rec["note"] = "warm: one buffer set (117 MB), reused every step from the MALL"
            extras["spmv_cfg2_f32_warm"] = rec
            log(f"extra spmv cfg2 warm: {res['gbs']:.1f} GB/s")
            del res
        except Exception as e:
            extras["spmv_cfg2_f32_warm"] = {"error": repr(e)}
        # the reference SpMV bench's own matrix (bench_cusparse.cu:84-144)
        try:
            Rh = workloads.hash_band(device="cuda")
            res = time_spmv(0, torch.float32, 400, 40, args.seed, 0, R=Rh)
            rec = spmv_record(0, torch.float32, res)
            rec["workload"] = "spmv_hash_band_N1048576"
            rec["offsets"] = workloads.HASH_BAND_OFFSETS
            if args.cpu_seconds > 0:
                rec["cpu_baseline"] = spmv_cpu_record(Rh, res, min(2.0, args.cpu_seconds),
                                                      "the reference bench's 9-diagonal hash band")
            extras["spmv_hash_band_N1048576"] = rec
            log(f"extra spmv hash band: {res['gbs']:.1f} GB/s")
            del res, Rh
        except Exception as e:
            extras["spmv_hash_band_N1048576"] = {"error": repr(e)}
        # configs 1-3 are SpMV matrices: their SpGEMM figure is H H
        for cfg, reps, rounds in ((1, 100, 10), (2, 50, 10), (3, 6, 3), (4, 50, 10), (5, 40, 10)):
            try:
                rec = time_spgemm(cfg, args.seed, reps, cpu_seconds=min(3.0, args.cpu_seconds),
                                  rounds=rounds)
                extras[rec["workload"]] = rec
                log(f"extra spgemm cfg{cfg}: {rec['GFLOPs']} GFLOP/s, {rec['GBs']} GB/s")
                torch.cuda.empty_cache()
            except Exception as e:
                extras[f"spgemm_cfg{cfg}"] = {"error": repr(e)}
            torch.cuda.empty_cache()
        try:
            rec = time_spgemm_banded(50, min(3.0, args.cpu_seconds))
            extras[rec["workload"]] = rec
            log(f"extra {rec['workload']}: {rec['GFLOPs']} GFLOP/s, {rec['GBs']} GB/s")
            torch.cuda.empty_cache()
        except Exception as e:
            extras["spgemm_make_banded"] = {"error": repr(e)}
        try:
            rec = time_krylov()
            extras["krylov_expm"] = rec
            log(f"extra krylov expm: {rec['ms_per_call']} ms per call, {rec['GBs']} GB/s")
            torch.cuda.empty_cache()
        except Exception as e:
            extras["krylov_expm"] = {"error": repr(e)}
        try:
            rec = time_taylor()
            extras["taylor_chain"] = rec
            log(f"extra taylor chain: {rec['total_ms']} ms, numeric {rec['numeric_GFLOPs']} GFLOP/s")
            torch.cuda.empty_cache()
        except Exception as e:
            extras["taylor_chain"] = {"error": repr(e)}
        for n_gd, reps_gd in ((4096, 100), (1 << 20, 20)):
            try:
                rec = time_gemm_diag(n_gd, 10, reps_gd, cpu_seconds=min(2.0, args.cpu_seconds),
                                     rotate=n_gd > 4096)
                extras[rec["workload"]] = rec
                log(f"extra {rec['workload']}: {rec['numeric_ms']} ms, {rec['GFLOPs']} GFLOP/s")
            except Exception as e:
                extras[f"gemm_diag_n{n_gd}"] = {"error": repr(e)}
        try:
            extras["launch_floor"] = launch_floor()
        except Exception as e:
            extras["launch_floor"] = {"error": repr(e)}
        for grid in ("3d", "2d"):
            try:
                rec = time_propagator(grid)
                extras[rec["workload"]] = rec
                log(f"extra {rec['workload']}: build {rec['build_ms']} ms, apply {rec['apply_ms']} ms, "
                    f"krylov {rec['krylov_ms']} ms")
            except Exception as e:
                extras[f"propagator_{grid}"] = {"error": repr(e)}
            torch.cuda.empty_cache()

    traffic = load_traffic("spmv_cfg2_f32")
    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 2: DIA SpMV, 2-D 5-point Poisson stencil, 2048x2048 "
                        "grid, n=4194304, offsets {2048,1,0,-1,-2048}, diag 4, off-diag -1 "
                        "(row wraps zeroed), x~N(0,1), fp32, Recon layout",
            "n": R.rows, "K": R.K, "seed": args.seed,
            "alg_bytes_per_step": head["alg_bytes"],
            "buffer_sets": head["sets"],
            "bytes_per_set": head["set_bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(head["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
