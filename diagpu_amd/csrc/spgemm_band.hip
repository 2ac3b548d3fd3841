// DIA x DIA SpGEMM numeric phase for narrow bands, with the operands staged
// in LDS: the LDS-tiled accumulation for products where each operand run is
// used by many plan entries (contiguous bands such as gemm_diag's defaults,
// gemm_diag/gemm_diag.cu:467-486: 21 x 21 diagonals, 10.8 entries per C
// diagonal).  The gather kernel (spgemm_numeric.hip) re-reads both operand
// runs from L2 for every entry; here a workgroup stages, for its block of
// kRB rows i,
//   A(i, i + da)          for every A diagonal          nA x kRB values
//   B(w, w + db)          for every B diagonal and       nB x (kRB + span)
//                         w in [i0 + min da, i0 + kRB + max da)
// once, then evaluates every C diagonal's entries from LDS:
//   C(i, i + dc) = sum over the plan entries (da, db) of dc
//                  A(i, i + da) * B(i + da, i + dc).
// Entries are taken in plan order (the pair order of
// spmspm/gather_flat.cuh:231-255) with one fused multiply-add each, and a
// term whose A element does not exist (row i + da outside [0, n)) is skipped
// -- the gather kernel's exact sequence of roundings, so both kernels return
// the same bits.  Row i's C element is written if column i + dc exists.
//
// Each plan entry becomes an int4 {A row's LDS offset, B window's LDS
// offset + the entry's shift, da, 0} (diagpu_spgemm_band_prepare, once per
// plan); the workgroup copies the table into LDS with the operands and reads
// it with uniform addresses (as global loads the compiler kept the entries
// in the vector memory queue, behind the staging loads).  The LDS footprint
// is 4 (nA kRB + nB WB) + 16 n_pairs bytes, WB = kRB + span rounded up to a
// multiple of 4, span = max da - min da.
#include <algorithm>
#include <type_traits>

#include "band_mfma.hpp"
#include "common.hpp"

namespace diagpu {
namespace {

constexpr int kRB = 256;                       // rows per block
constexpr int kThreads = 512;                  // lanes per workgroup: two halves of kRB
constexpr int kHalves = kThreads / kRB;
constexpr int64_t kLdsBudget = 64 * 1024;      // keeps two workgroups per CU

// Rows of one B diagonal's window in LDS: kRB + span, padded to a multiple
// of 4 (keeps the entry table after the windows 16-byte aligned).
__host__ __device__ constexpr int window_rows(int span) { return (kRB + span + 3) & ~3; }

// LDS bytes of one workgroup: A rows, B windows, the plan's entries.
int64_t band_lds_bytes(int32_t nA, int32_t nB, int64_t span, int64_t n_pairs)
{
    const int64_t wb = span > (int64_t)1 << 20 ? (int64_t)1 << 40 : window_rows((int)span);
    return 4 * ((int64_t)nA * kRB + (int64_t)nB * wb) + 16 * n_pairs;
}

// The band kernel takes the plan: its LDS footprint fits the budget.
bool band_fits(int64_t lds_bytes, int64_t n_pairs)
{
    return lds_bytes <= kLdsBudget && n_pairs <= 0x7fffffff;
}

// entries[g] = {a kRB, b WB + (da - min da), da, 0}, a and b the indices of
// pairs[g].ab in A_starts and of pairs[g].bb in B_starts, WB =
// window_rows(span).  span[0..1] = min, max da (k_span, which
// runs first on the stream); span[2] is set if an entry matches no diagonal
// or differs from the entry the symbolic phase makes for its two diagonals
// (the band kernel derives each term's shifts and bounds from the operand
// offsets, so it must be handed exactly that plan).
__global__ __launch_bounds__(256) void k_band_prepare(int32_t n,
                                                      const diagpu_gpair* __restrict__ pairs,
                                                      int64_t n_pairs,
                                                      const int32_t* __restrict__ A_off,
                                                      const int64_t* __restrict__ A_starts,
                                                      int32_t nA,
                                                      const int32_t* __restrict__ B_off,
                                                      const int64_t* __restrict__ B_starts,
                                                      int32_t nB, int4* __restrict__ entries,
                                                      int32_t* __restrict__ span)
{
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= n_pairs) return;
    // binary search (diagonals stored in offset order: starts ascend), then a
    // linear scan for operands stored in another order
    auto find = [](const int64_t* s, int32_t cnt, int64_t v) -> int {
        int lo = 0, hi = cnt - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s[mid] <= v) lo = mid; else hi = mid - 1;
        }
        if (s[lo] == v) return lo;
        for (int i = 0; i < cnt; ++i)
            if (s[i] == v) return i;
        return -1;
    };
    const diagpu_gpair p = pairs[g];
    const int a = find(A_starts, nA, (int64_t)p.ab);
    const int b = find(B_starts, nB, (int64_t)p.bb);
    bool ok = a >= 0 && b >= 0;
    int da = 0;
    if (ok) {
        da = A_off[a];
        const int db = B_off[b];
        const int64_t dc = (int64_t)da + db;
        auto min0 = [](int64_t x) { return x < 0 ? x : (int64_t)0; };
        auto absl = [](int64_t x) { return x < 0 ? -x : x; };
        ok = dc > -(int64_t)n && dc < n && (int64_t)p.ash == min0(da) - min0(dc) &&
             (int64_t)p.bsh == da + min0(db) - min0(dc) && (int64_t)p.al == n - absl(da) &&
             (int64_t)p.bl == n - absl(db);
    }
    if (!ok) {
        span[2] = 1;   // every writer stores the same value
        entries[g] = int4{0, 0, 0, 0};
        return;
    }
    const int lo = span[0], wb = window_rows(span[1] - span[0]);
    entries[g] = int4{a * kRB, b * wb + (da - lo), da, 0};
}

// min and max of A's offsets (out[0], out[1]) and of B's (out[3], out[4]),
// one workgroup; out[2] is the bad-entry flag, cleared here
__global__ __launch_bounds__(256) void k_span(const int32_t* __restrict__ off, int32_t cnt,
                                              const int32_t* __restrict__ boff, int32_t bcnt,
                                              int32_t* __restrict__ out)
{
    __shared__ int lo_s[256], hi_s[256], blo_s[256], bhi_s[256];
    int lo = 0x7fffffff, hi = -0x7fffffff - 1, blo = 0x7fffffff, bhi = -0x7fffffff - 1;
    for (int i = threadIdx.x; i < cnt; i += 256) {
        lo = off[i] < lo ? off[i] : lo;
        hi = off[i] > hi ? off[i] : hi;
    }
    for (int i = threadIdx.x; i < bcnt; i += 256) {
        blo = boff[i] < blo ? boff[i] : blo;
        bhi = boff[i] > bhi ? boff[i] : bhi;
    }
    blo_s[threadIdx.x] = blo;
    bhi_s[threadIdx.x] = bhi;
    lo_s[threadIdx.x] = lo;
    hi_s[threadIdx.x] = hi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            lo_s[threadIdx.x] = lo_s[threadIdx.x + s] < lo_s[threadIdx.x] ? lo_s[threadIdx.x + s] : lo_s[threadIdx.x];
            hi_s[threadIdx.x] = hi_s[threadIdx.x + s] > hi_s[threadIdx.x] ? hi_s[threadIdx.x + s] : hi_s[threadIdx.x];
            blo_s[threadIdx.x] = blo_s[threadIdx.x + s] < blo_s[threadIdx.x] ? blo_s[threadIdx.x + s] : blo_s[threadIdx.x];
            bhi_s[threadIdx.x] = bhi_s[threadIdx.x + s] > bhi_s[threadIdx.x] ? bhi_s[threadIdx.x + s] : bhi_s[threadIdx.x];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out[0] = lo_s[0];
        out[1] = hi_s[0];
        out[2] = 0;   // bad-entry flag, set by k_band_prepare (launched next)
        out[3] = blo_s[0];
        out[4] = bhi_s[0];
    }
}

// The persistent evaluation.  XCD x (workgroups b with b mod 8 == x) owns
// the row blocks [x per_xcd, (x + 1) per_xcd) and its L workgroups take
// blocks l, l + L, ... of that range in step, so the blocks in flight on one
// XCD are neighbours whose B windows overlap in its L2.  Per block a
// workgroup stages the operands with direct global-to-LDS loads (no
// registers, so every load of the block is in flight at once and one wait
// covers them all), then evaluates the block's C values from LDS.
//
// Staged elements that do not exist (rows outside [0, n), or columns
// outside it) hold whatever the clamped load brought: a term reads B(i + da,
// i + dc) only where C(i, i + dc) is written (so column i + dc exists) and
// A(i, i + da) exists (so row i + da does), and the evaluation skips every
// term whose A element is missing, so no such value reaches a C element.
__global__ __launch_bounds__(kThreads) void k_band(
    int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts, int32_t nA,
    const float* __restrict__ Av, const int32_t* __restrict__ B_off,
    const int64_t* __restrict__ B_starts, int32_t nB, const float* __restrict__ Bv,
    const int32_t* __restrict__ C_off, const int64_t* __restrict__ C_starts, int32_t nC,
    const int64_t* __restrict__ pair_ptr, const int4* __restrict__ entries, int32_t n_pairs,
    float* __restrict__ Cv, int32_t a_min, int32_t a_max, int32_t blocks, int32_t per_xcd,
    int32_t wg_per_xcd)
{
    extern __shared__ float lds[];
    const int xcd = (int)(blockIdx.x % kNumXcd);
    const int blk_end = (xcd + 1) * per_xcd < blocks ? (xcd + 1) * per_xcd : blocks;
    int blk = xcd * per_xcd + (int)(blockIdx.x / kNumXcd);
    if (blk >= blk_end) return;
    const int WB = window_rows(a_max - a_min);      // B window rows
    float* A_l = lds;                               // [nA][kRB]
    float* B_l = lds + (int64_t)nA * kRB;           // [nB][WB]
    int4* E_l = reinterpret_cast<int4*>(B_l + (int64_t)nB * WB);   // [n_pairs] plan entries
    const int r = (int)threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(r >> 6), lane = r & 63;
    // staging: half h of the workgroup (kRB lanes, one row each) takes the
    // diagonal groups h, h + kHalves, ...
    const int half = __builtin_amdgcn_readfirstlane(r / kRB), rr = r % kRB;
    const int hw = __builtin_amdgcn_readfirstlane(rr >> 6);   // wave within the half

    // the plan's entries, once per workgroup: read below with uniform LDS
    // addresses (as global loads the compiler kept them in the vector memory
    // queue, behind the staging loads)
    for (int g = r; g < n_pairs; g += kThreads) E_l[g] = entries[g];

    // One wave's 64 rows of one diagonal: lane l loads the element of row
    // w (its HM position clamped into the diagonal, so the address is
    // always valid) into dst[l].  Positions and rows fit int32 (n <= 2^30).
    auto load_row = [&](const float* __restrict__ vals, int64_t st, int o, int w, float* dst) {
        const int len = n - (o < 0 ? -o : o);
        const int pos = min(max(w + (o < 0 ? o : 0), 0), len - 1);   // HM position of (w, w + o)
        __builtin_amdgcn_global_load_lds(vals + st + pos, dst, 4, 0, 0);
    };
    // Diagonals kS at a time: their offsets and starts are read (scalar
    // loads, all in flight together) before any of their row loads is
    // issued -- the compiler does not move a scalar load across a direct
    // LDS load, so a load interleaved with them waits alone.
    constexpr int kS = 8;
    const int slots = (WB + kRB - 1) / kRB;         // kRB-row slots of a B window
    auto stage = [&](int i0) {
        for (int d0 = half * kS; d0 < nA; d0 += kHalves * kS) {   // A: rows i0 + rr
            int o[kS];
            int64_t st[kS];
#pragma unroll
            for (int u = 0; u < kS; ++u) {
                const int d = d0 + u < nA ? d0 + u : nA - 1;
                o[u] = at_byte(A_off, (uint32_t)d << 2);
                st[u] = at_byte(A_starts, (uint32_t)d << 3);
            }
#pragma unroll
            for (int u = 0; u < kS; ++u)
                if (d0 + u < nA) load_row(Av, st[u], o[u], i0 + rr, A_l + (d0 + u) * kRB + hw * 64);
        }
        for (int d0 = half * kS; d0 < nB; d0 += kHalves * kS) {   // B: window rows i0 + a_min + q
            int o[kS];
            int64_t st[kS];
#pragma unroll
            for (int u = 0; u < kS; ++u) {
                const int d = d0 + u < nB ? d0 + u : nB - 1;
                o[u] = at_byte(B_off, (uint32_t)d << 2);
                st[u] = at_byte(B_starts, (uint32_t)d << 3);
            }
            for (int sl = 0; sl < slots; ++sl) {
                const int q = rr + kRB * sl;
                if (q < WB) {
#pragma unroll
                    for (int u = 0; u < kS; ++u)
                        if (d0 + u < nB)
                            load_row(Bv, st[u], o[u], i0 + a_min + q,
                                     B_l + (d0 + u) * WB + kRB * sl + hw * 64);
                }
            }
        }
    };

    constexpr int kWaves = kThreads / 64, kR = kRB / 64;
    for (; blk < blk_end; blk += wg_per_xcd) {
        const int64_t i0 = (int64_t)blk * kRB;
        __syncthreads();                 // every wave is done with the previous block's LDS
        stage((int)i0);
        __builtin_amdgcn_s_waitcnt(0);   // this wave's direct loads have landed in LDS
        __syncthreads();

        // every A element of this block exists, for every diagonal: no predicate
        const bool interior =
            i0 + kRB <= n && i0 + a_min >= 0 && i0 + kRB + (int64_t)a_max <= n;
        const int row0 = (int)i0 + lane;             // n <= 2^30: rows fit int32
        // Wave w evaluates C diagonals w, w + kWaves, ... over all kRB rows, kR
        // rows per lane (lane l: rows l, l + 64, ...): each entry's lookup
        // then feeds kR independent pairs of LDS reads.
        auto evaluate = [&](auto interior_tag) {
            constexpr bool kInt = decltype(interior_tag)::value;
            for (int kc = wave; kc < nC; kc += kWaves) {
                // byte offsets 4 kc and 8 kc: small, since the plan's entries
                // (16 bytes each, at least one per C diagonal) fit the 64 KiB
                // LDS budget
                const int dc = at_byte(C_off, (uint32_t)kc << 2);
                const int g0 = (int)at_byte(pair_ptr, (uint32_t)kc << 3),
                          g1 = (int)at_byte(pair_ptr + 1, (uint32_t)kc << 3);
                float acc[kR];
#pragma unroll
                for (int j = 0; j < kR; ++j) acc[j] = 0.f;
                // entries in batches of kU: their LDS reads issued together,
                // then the multiply-adds in plan order
                constexpr int kU = 2;
                auto step = [&](const int4& e, const float (&a)[kR], const float (&b)[kR]) {
#pragma unroll
                    for (int j = 0; j < kR; ++j) {
                        const float t = __builtin_fmaf(a[j], b[j], acc[j]);
                        if constexpr (kInt) {
                            acc[j] = t;
                        } else {
                            const int ra = row0 + 64 * j + e.z;   // column of the A element
                            acc[j] = (ra >= 0 && ra < n) ? t : acc[j];
                        }
                    }
                };
                int g = g0;
                for (; g + kU <= g1; g += kU) {
                    int4 e[kU];
                    float a[kU][kR], b[kU][kR];
#pragma unroll
                    for (int u = 0; u < kU; ++u) e[u] = E_l[g + u];
#pragma unroll
                    for (int u = 0; u < kU; ++u)
#pragma unroll
                        for (int j = 0; j < kR; ++j) {
                            a[u][j] = A_l[e[u].x + lane + 64 * j];
                            b[u][j] = B_l[e[u].y + lane + 64 * j];
                        }
#pragma unroll
                    for (int u = 0; u < kU; ++u) step(e[u], a[u], b[u]);
                }
                for (; g < g1; ++g) {
                    const int4 e = E_l[g];
                    float a[kR], b[kR];
#pragma unroll
                    for (int j = 0; j < kR; ++j) {
                        a[j] = A_l[e.x + lane + 64 * j];
                        b[j] = B_l[e.y + lane + 64 * j];
                    }
                    step(e, a, b);
                }
                float* __restrict__ cp = Cv + at_byte(C_starts, (uint32_t)kc << 3) + (dc < 0 ? dc : 0);
#pragma unroll
                for (int j = 0; j < kR; ++j) {
                    const int ii = row0 + 64 * j;
                    if (ii < n && ii + dc >= 0 && ii + dc < n) __builtin_nontemporal_store(acc[j], cp + ii);
                }
            }
        };
        if (interior)
            evaluate(std::true_type{});
        else
            evaluate(std::false_type{});
    }
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spgemm_band_prepare(int32_t n, const int32_t* A_off,
                                          const int64_t* A_starts, int32_t nA,
                                          const int32_t* B_off, const int64_t* B_starts, int32_t nB,
                                          const diagpu_gpair* pairs, int64_t n_pairs,
                                          int32_t* entries, diagpu_band_info* info, void* stream)
{
    using namespace diagpu;
    const char* fn = "diagpu_spgemm_band_prepare";
    if (!info) return fail(DIAGPU_ERR_ARG, "%s: info is NULL", fn);
    *info = diagpu_band_info{};
    if (n < 1 || nA < 1 || nB < 1 || n_pairs < 0)
        return fail(DIAGPU_ERR_ARG, "%s: need n, nA, nB >= 1 and n_pairs >= 0", fn);
    if (nA > 65535 || nB > 32767)
        return fail(DIAGPU_ERR_ARG, "%s: at most 65535 A and 32767 B diagonals", fn);
    if (!A_off || !A_starts || !B_off || !B_starts || !entries || (n_pairs > 0 && !pairs))
        return fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
    hipStream_t s = as_stream(stream);
    int32_t* dev = entries + 4 * n_pairs;   // caller's 8 scratch ints: spans, bad-entry flag
    int32_t host[5] = {0, 0, 0, 0, 0};
    hipLaunchKernelGGL(k_span, dim3(1), dim3(256), 0, s, A_off, nA, B_off, nB, dev);
    int st = check_launch(fn);
    if (!st && n_pairs > 0) {
        hipLaunchKernelGGL(k_band_prepare, dim3((unsigned)ceil_div<int64_t>(n_pairs, 256)),
                           dim3(256), 0, s, n, pairs, n_pairs, A_off, A_starts, nA, B_off,
                           B_starts, nB, reinterpret_cast<int4*>(entries), dev);
        st = check_launch(fn);
    }
    if (!st) st = check_hip(hipMemcpyWithStream(host, dev, sizeof(host), hipMemcpyDeviceToHost, s), fn);
    if (st) return st;
    if (host[2])
        return fail(DIAGPU_ERR_ARG, "%s: a plan entry's starts are no operand diagonals' starts, or "
                    "its shifts or lengths are not the symbolic phase's for those diagonals", fn);
    if (host[0] <= -n || host[1] >= n)
        return fail(DIAGPU_ERR_OFFSET, "%s: an A offset is outside (-n, n)", fn);
    if (host[3] <= -n || host[4] >= n)
        return fail(DIAGPU_ERR_OFFSET, "%s: a B offset is outside (-n, n)", fn);
    info->a_off_min = host[0];
    info->a_off_max = host[1];
    info->b_off_min = host[3];
    info->b_off_max = host[4];
    const MfmaGeom g = mfma_geom(host[0], host[1], host[3], host[4]);
    info->mfma_blocks = g.ok ? g.nblk : 0;
    info->mfma_eligible = g.ok;
    info->mfma_lds_bytes = g.ok ? g.lds_bytes : 0;
    info->rows_per_block = kRB;
    info->n_pairs = n_pairs;
    info->lds_bytes = band_lds_bytes(nA, nB, host[1] - host[0], n_pairs);
    info->eligible = band_fits(info->lds_bytes, n_pairs) ? 1 : 0;
    return DIAGPU_OK;
}

DIAGPU_API int diagpu_spgemm_numeric_band_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    const int32_t* B_off, const int64_t* B_starts, int32_t nB, const float* B_vals,
    const int32_t* C_off, const int64_t* C_starts, int64_t c_ndiag, const int64_t* pair_ptr,
    const int32_t* entries, const diagpu_band_info* info, float* C_vals, void* stream)
{
    using namespace diagpu;
    const char* fn = "diagpu_spgemm_numeric_band_f32";
    if (!info) return fail(DIAGPU_ERR_ARG, "%s: info is NULL", fn);
    if (n < 1 || nA < 1 || nB < 1 || c_ndiag < 0 || c_ndiag > 2 * (int64_t)n - 1)
        return fail(DIAGPU_ERR_ARG, "%s: bad sizes (n=%d nA=%d nB=%d c_ndiag=%lld)", fn, n, nA,
                    nB, (long long)c_ndiag);
    const int64_t span = (int64_t)info->a_off_max - info->a_off_min;
    if (!info->eligible || info->rows_per_block != kRB || span < 0 || info->a_off_min <= -n ||
        info->a_off_max >= n || info->n_pairs < 0 ||
        info->lds_bytes != band_lds_bytes(nA, nB, span, info->n_pairs) ||
        !band_fits(info->lds_bytes, info->n_pairs))
        return fail(DIAGPU_ERR_CAPACITY, "%s: info is not an eligible band_prepare result for "
                    "these operands", fn);
    const int64_t n_pairs = info->n_pairs;
    if (c_ndiag == 0) return DIAGPU_OK;
    if (!A_off || !A_starts || !A_vals || !B_off || !B_starts || !B_vals || !C_off ||
        !C_starts || !pair_ptr || !entries || !C_vals)
        return fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
    const int32_t blocks = (int32_t)ceil_div<int64_t>(n, kRB);
    const int32_t per_xcd = ceil_div<int32_t>(blocks, kNumXcd);
    // persistent: as many workgroups per XCD as fit at once, at most one
    // per row block of its range
    int per_cu = 0;
    int st = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_band, kThreads,
                                                                    (size_t)info->lds_bytes), fn);
    if (st) return st;
    int64_t wg = (int64_t)(cu_count() / kNumXcd) * (per_cu > 0 ? per_cu : 1);
    if (wg > per_xcd) wg = per_xcd;
    hipLaunchKernelGGL(k_band, dim3((unsigned)(wg * kNumXcd)), dim3(kThreads), (size_t)info->lds_bytes,
                       as_stream(stream), n, A_off, A_starts, nA, A_vals, B_off, B_starts, nB,
                       B_vals, C_off, C_starts, (int32_t)c_ndiag, pair_ptr,
                       reinterpret_cast<const int4*>(entries), (int32_t)n_pairs, C_vals,
                       info->a_off_min, info->a_off_max, blocks, per_xcd, (int32_t)wg);
    return check_launch(fn);
}

}  // extern "C"
