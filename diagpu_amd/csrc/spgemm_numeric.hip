// DIA x DIA SpGEMM, numeric phase on the GPU (HM layout, fp32 or complex64).
//
//   C[k][p] = sum over the plan entries g of C diagonal k of
//             Av[g.ab + p + g.ash] * Bv[g.bb + p + g.bsh]
//   for 0 <= p < C_len[k], terms with p + ash outside [0, al) or p + bsh
//   outside [0, bl) dropped -- the shifted multiply-accumulate of
//   hm_structured_sparse_matmul_kernel (spmspm/paper_hm_kernel.cu:31-93) and
//   of gather_flat_kernel (spmspm/gather_flat.cuh:47-62), evaluated in plan
//   order with fp32 accumulation.  Every C value is written exactly once: no
//   atomics, no pre-zeroing, deterministic.  The complex64 variant (complex
//   Hamiltonians; the reference is real only) runs the same plan with
//   complex products; a lane then owns 2 positions instead of 4, so its loads
//   and stores stay 16 bytes.
//
// Work decomposition.  An item is (row block rb, C diagonal k): the 256 x E
// positions of diagonal k whose matrix rows fall in block rb (E = 4 for fp32,
// 2 for complex64; shifted back by less than one 128-byte line so the item's
// first C element starts a line).  Each lane owns E consecutive positions: one aligned
// 128-bit streaming store of C and, per plan entry, one 128-bit load each of A
// and B (dword aligned).  A workgroup
// takes a batch of up to 16 consecutive C diagonals of one row block (fewer
// when a small problem would otherwise leave CUs idle): their
// metadata and plan entries (1.7 per diagonal on average) are resolved once
// into LDS, then the flattened entry list is walked in chunks whose loads are
// all in flight together, across C-diagonal boundaries.  The C stores are
// non-temporal so the 10 GB output stream does not evict the operands from
// L2.
//
// Row-space locality.  In row coordinates the entry (da, db) of C row i
// reads A(i, i + da) and B(i + da, i + dc): every A diagonal at rows i, every
// B diagonal at rows i + da.  Items are ordered row block first, so the
// workgroups active on one XCD all work inside one row block and share an L2
// working set of |A| x 1024 A values and |B| x (1024 + spread of da) B
// values.  The launch is persistent: XCD x (workgroups b with b mod 8 == x)
// owns the row blocks [x * nbx, (x + 1) * nbx) and its workgroups stride
// through that range's items in order, so each XCD's L2 streams one
// contiguous band of rows.  Each workgroup's item loop ends at a fixed count.
#include <algorithm>

#include "common.hpp"
#include "elem.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;
constexpr int kBatch = 16;        // consecutive C diagonals per batch

// Positions per lane (16 bytes of T) and per item.
template <typename T> constexpr int epl() { return (int)(16 / sizeof(T)); }
template <typename T> constexpr int item_positions() { return kBlock * epl<T>(); }
// Positions per 128-byte line: items start on a line of C, so consecutive
// items of a C diagonal split it at line boundaries.  (A line written in two
// parts by two workgroups at different times costs a read-modify-write in
// HBM: measured, 4 KB store chunks that start 16-byte- but not line-aligned
// run at 3.5 TB/s against 5.4 aligned.)
template <typename T> constexpr int line_positions() { return (int)(128 / sizeof(T)); }

// acc + a * b over a lane's positions
__device__ __forceinline__ float mac(float acc, float a, float b) { return __builtin_fmaf(a, b, acc); }
__device__ __forceinline__ cf32 mac(cf32 acc, cf32 a, cf32 b) { return mad(acc, a, b); }

// One C diagonal of the current batch, for the current row block.
struct DiagRec {
    int64_t P0;     // first position of the item (may lie outside [0, len))
    int64_t cst;    // C_starts
    int32_t len;    // C_len
    int32_t pad0;
    int64_t pad1;
};

// One plan entry of the current batch, resolved for the current row block.
struct PairRec {
    int64_t a_base;   // A index of position 0 (ab + ash)
    int64_t b_base;   // B index of position 0 (bb + bsh)
    int32_t plo, phi; // positions where both operands exist, within [0, len)
    int32_t ci;       // C diagonal within the batch
    int32_t cover;    // 1: covers the whole item, 0: part of it, -1: none of it
};

// Item enumeration: XCD-partitioned (workgroup b on XCD b mod 8 strides
// through that XCD's row blocks) or, for problems with few row blocks, flat
// (workgroup b strides through all items).  `batch` (<= kBatch) C diagonals
// per item.
struct ItemSpace {
    int32_t NB;           // row blocks
    int32_t nb_per_xcd;   // XCD-partitioned: row blocks per XCD
    int32_t wg_per_xcd;   // XCD-partitioned: workgroups per XCD
    int32_t flat;         // 1: flat enumeration over gridDim.x workgroups
    int32_t batch;        // C diagonals per item, 1..kBatch
};

template <typename T, int PC>
__global__ __launch_bounds__(kBlock) void k_gather(
    const T* __restrict__ Av, const T* __restrict__ Bv,
    const int32_t* __restrict__ C_off, const int32_t* __restrict__ C_len,
    const int64_t* __restrict__ C_starts, int32_t nC, const int64_t* __restrict__ pair_ptr,
    const diagpu_gpair* __restrict__ pairs, T* __restrict__ Cv, ItemSpace is)
{
    constexpr int E = epl<T>();
    constexpr int TB = item_positions<T>();
    typedef Run<T, E> V;
    __shared__ DiagRec drec[kBatch];
    __shared__ int64_t ptr_s[kBatch + 1];
    __shared__ PairRec prec[kBlock];

    int rb0, rb_end, l, stride;
    if (is.flat) {
        rb0 = 0;
        rb_end = is.NB;
        l = (int)blockIdx.x;
        stride = (int)gridDim.x;
    } else {
        const int xcd = (int)(blockIdx.x % kNumXcd);
        rb0 = xcd * is.nb_per_xcd;
        rb_end = (rb0 + is.nb_per_xcd) < is.NB ? (rb0 + is.nb_per_xcd) : is.NB;
        l = (int)(blockIdx.x / kNumXcd);
        stride = is.wg_per_xcd;
    }
    if (rb0 >= rb_end || nC <= 0) return;
    const int batch = is.batch;
    const int nbat = (nC + batch - 1) / batch;
    const int t = (int)threadIdx.x;
    const int64_t p_lane = (int64_t)t * E;
    const int64_t nwork = (int64_t)(rb_end - rb0) * nbat;

    for (int64_t j = l; j < nwork; j += stride) {
        const int rb = rb0 + (int)(j / nbat);
        const int kb = (int)(j % nbat) * batch;
        const int gv = (nC - kb) < batch ? (nC - kb) : batch;

        __syncthreads();   // previous batch done with drec/ptr_s/prec
        if (t <= gv) ptr_s[t] = pair_ptr[kb + t];
        if (t < gv) {
            const int dc = C_off[kb + t];
            const int64_t cst = C_starts[kb + t];
            const int mc = dc < 0 ? dc : 0;
            DiagRec d;
            d.P0 = (int64_t)rb * TB + mc - (int)((cst + mc) & (line_positions<T>() - 1));
            d.cst = cst;
            d.len = C_len[kb + t];
            d.pad0 = 0;
            d.pad1 = 0;
            drec[t] = d;
        }
        __syncthreads();

        const int64_t gb = ptr_s[0], ge = ptr_s[gv];
        V acc;
#pragma unroll
        for (int e = 0; e < E; ++e) acc.v[e] = zero_of<T>();
        int cur = -1;   // C diagonal of the batch being accumulated
        auto flush = [&](int ci) {
            const DiagRec d = drec[ci];
            const int64_t p = d.P0 + p_lane;
            T* __restrict__ cp = Cv + d.cst;
            if (d.P0 >= 0 && d.P0 + TB <= d.len) {
                store_run_nt<T, E>(cp + p, acc);   // cst + P0 starts a 128-byte line
            } else if (d.P0 < d.len && d.P0 + TB > 0) {
#pragma unroll
                for (int e = 0; e < E; ++e)
                    if (p + e >= 0 && p + e < d.len) cp[p + e] = acc.v[e];
            }
        };
        // Close diagonal `cur` and move to diagonal `to` of the batch: the
        // diagonals in between have no plan entry and are written as zeros
        // (every C value is written, whatever the plan holds).
        auto advance = [&](int to) {
            if (cur >= 0) flush(cur);
#pragma unroll
            for (int e = 0; e < E; ++e) acc.v[e] = zero_of<T>();
            for (int z = cur + 1; z < to; ++z) flush(z);
            cur = to;
        };

        for (int64_t gq = gb; gq < ge; gq += kBlock) {
            const int cnt = (ge - gq) < kBlock ? (int)(ge - gq) : kBlock;
            __syncthreads();
            if (t < cnt) {
                const diagpu_gpair g = pairs[gq + t];
                int ci = 0;
                for (int c = 1; c < gv; ++c) ci += (ptr_s[c] <= gq + t) ? 1 : 0;
                const DiagRec d = drec[ci];
                PairRec r;
                r.a_base = (int64_t)g.ab + g.ash;
                r.b_base = (int64_t)g.bb + g.bsh;
                int lo = 0, hi = d.len;
                lo = -g.ash > lo ? -g.ash : lo;
                lo = -g.bsh > lo ? -g.bsh : lo;
                hi = g.al - g.ash < hi ? g.al - g.ash : hi;
                hi = g.bl - g.bsh < hi ? g.bl - g.bsh : hi;
                r.plo = lo;
                r.phi = hi;
                r.ci = ci;
                r.cover = (d.P0 >= lo && d.P0 + TB <= hi) ? 1
                          : ((d.P0 + TB > lo && d.P0 < hi) ? 0 : -1);
                prec[t] = r;
            }
            __syncthreads();

            for (int s0 = 0; s0 < cnt; s0 += PC) {
                // A chunk in which no entry covers only part of the item takes
                // the straight-line path: all 2*PC vector loads are issued
                // before the first multiply-add (a masked element path in the
                // same block would make the compiler drain the loads at its
                // merge point).
                bool fast = true;
#pragma unroll
                for (int c = 0; c < PC; ++c)
                    if (s0 + c < cnt && prec[s0 + c].cover == 0) fast = false;
                if (fast) {
                    V a[PC], b[PC];
#pragma unroll
                    for (int c = 0; c < PC; ++c) {
                        if (s0 + c < cnt && prec[s0 + c].cover > 0) {
                            const PairRec r = prec[s0 + c];
                            const int64_t p = drec[r.ci].P0 + p_lane;
                            a[c] = load_run<T, E, false>(Av + r.a_base + p);
                            b[c] = load_run<T, E, false>(Bv + r.b_base + p);
                        }
                    }
#pragma unroll
                    for (int c = 0; c < PC; ++c) {
                        if (s0 + c >= cnt) continue;
                        const PairRec r = prec[s0 + c];
                        if (r.ci != cur) advance(r.ci);
                        if (r.cover > 0) {
#pragma unroll
                            for (int e = 0; e < E; ++e) acc.v[e] = mac(acc.v[e], a[c].v[e], b[c].v[e]);
                        }
                    }
                } else {
                    for (int c = 0; c < PC && s0 + c < cnt; ++c) {
                        const PairRec r = prec[s0 + c];
                        if (r.ci != cur) advance(r.ci);
                        if (r.cover < 0) continue;
                        const int64_t p = drec[r.ci].P0 + p_lane;
                        T av[E], bv[E];
                        bool ok[E];
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            const int64_t x = p + e;
                            ok[e] = x >= r.plo && x < r.phi;
                            av[e] = ok[e] ? Av[r.a_base + x] : zero_of<T>();
                            bv[e] = ok[e] ? Bv[r.b_base + x] : zero_of<T>();
                        }
#pragma unroll
                        for (int e = 0; e < E; ++e)
                            acc.v[e] = ok[e] ? mac(acc.v[e], av[e], bv[e]) : acc.v[e];
                    }
                }
            }
        }
        advance(gv);
    }
}

template <typename T>
int numeric_launch(int32_t n, const T* A_vals, const T* B_vals, const int32_t* C_off,
                   const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
                   const int64_t* pair_ptr, const diagpu_gpair* pairs, int64_t max_pairs,
                   T* C_vals, void* stream, const char* fn)
{
    if (n < 1 || n > (1 << 30)) return fail(DIAGPU_ERR_ARG, "%s: n=%d outside [1, 2^30]", fn, n);
    if (c_ndiag < 0 || c_ndiag > 2 * (int64_t)n - 1)
        return fail(DIAGPU_ERR_ARG, "%s: c_ndiag=%lld outside [0, 2n-1]", fn, (long long)c_ndiag);
    if (max_pairs < 0) return fail(DIAGPU_ERR_ARG, "%s: negative max_pairs", fn);
    if (c_ndiag == 0) return DIAGPU_OK;
    if (!C_off || !C_len || !C_starts || !pair_ptr || !C_vals)
        return fail(DIAGPU_ERR_ARG, "%s: C structure, pair_ptr or C_vals is NULL", fn);
    if (max_pairs > 0 && (!pairs || !A_vals || !B_vals))
        return fail(DIAGPU_ERR_ARG, "%s: pairs or operand values are NULL", fn);

    constexpr int TB = item_positions<T>();
    ItemSpace is;
    is.NB = (int32_t)ceil_div<int64_t>((int64_t)n + line_positions<T>() - 1, TB);
    is.nb_per_xcd = ceil_div<int32_t>(is.NB, kNumXcd);
    // Many C diagonals (wide operands): 4 workgroups per
    // CU; few: 16 (8 fit at a time; the rest queue, and the lighter share of
    // items per workgroup balances the tail.  Measured against 8 with the
    // operands resident in the MALL: config 4 52.9 -> 46.0 us, the square of
    // config 2 80.6 -> 71.4 us; with cold operands, HBM-bound, about the
    // same).  8-entry chunks for the few-diagonal case (more loads in flight
    // per lane, half the workgroups resident) measured slower on the cold
    // lines: config 4 51.2 against 47.0 us, the square of config 1 16.9
    // against 15.2 us (the square of config 2 111.3 against 115.5 us).
    // With 2048 row blocks or more, 32: the batch then shrinks to smaller
    // items (measured: the square of config 2, 4096 row blocks, 115.6 ->
    // 99.8 us; config 4 with complex values, 2048, 146.7 -> 132.4 us; config
    // 4 in fp32, 1024, is 3.6% slower at 32, so it keeps 16).
    const bool wide = c_ndiag >= 1024;
    const int per_cu = wide ? 4 : (is.NB >= 2048 ? 32 : 16);
    const int64_t slots = (int64_t)cu_count() * per_cu;
    // Small problems with heavy items: fewer C diagonals per item until the
    // items can fill the GPU (a batch's entries are walked by one workgroup,
    // chunk after chunk, so an item of many entries is a long serial chain;
    // light items -- at most two chunks -- are left whole, their prologue
    // being the larger cost), and flat item enumeration when there are too
    // few row blocks to give every XCD a share.
    // Plans with up to 5 entries per C diagonal take 4-entry chunks; heavier
    // ones (e.g. powers of a 7-point stencil, 6-7 entries) 8-entry chunks:
    // the Taylor chain's products were 10% slower with 4 (k = 6: 1.255 ->
    // 1.452 ms).
    const int pc = (!wide && max_pairs >= 6) ? 8 : 4;
    is.batch = kBatch;
    while (is.batch > 1 && (int64_t)is.NB * ceil_div<int64_t>(c_ndiag, is.batch) < slots &&
           std::min<int64_t>(is.batch, c_ndiag) * max_pairs > 2 * pc)
        is.batch /= 2;
    is.flat = is.NB < 4 * kNumXcd ? 1 : 0;
    int64_t grid;
    if (is.flat) {
        grid = (int64_t)is.NB * ceil_div<int64_t>(c_ndiag, is.batch);
        if (grid > slots) grid = slots;
        is.wg_per_xcd = 0;
    } else {
        const int64_t items_per_xcd = (int64_t)is.nb_per_xcd * ceil_div<int64_t>(c_ndiag, is.batch);
        int64_t wg = (int64_t)(cu_count() / kNumXcd) * per_cu;
        if (wg > items_per_xcd) wg = items_per_xcd;
        if (wg < 1) wg = 1;
        is.wg_per_xcd = (int32_t)wg;
        grid = wg * kNumXcd;
    }
    if (pc == 8)
        hipLaunchKernelGGL((k_gather<T, 8>), dim3((unsigned)grid), dim3(kBlock), 0,
                           as_stream(stream), A_vals, B_vals, C_off, C_len, C_starts,
                           (int32_t)c_ndiag, pair_ptr, pairs, C_vals, is);
    else
        hipLaunchKernelGGL((k_gather<T, 4>), dim3((unsigned)grid), dim3(kBlock), 0,
                           as_stream(stream), A_vals, B_vals, C_off, C_len, C_starts,
                           (int32_t)c_ndiag, pair_ptr, pairs, C_vals, is);
    return check_launch(fn);
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spgemm_numeric_f32(
    int32_t n, const float* A_vals, const float* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const diagpu_gpair* pairs, int64_t max_pairs,
    float* C_vals, void* stream)
{
    return diagpu::numeric_launch<float>(n, A_vals, B_vals, C_off, C_len, C_starts, c_ndiag,
                                         pair_ptr, pairs, max_pairs, C_vals, stream,
                                         "diagpu_spgemm_numeric_f32");
}

DIAGPU_API int diagpu_spgemm_numeric_c64(
    int32_t n, const diagpu_complex64* A_vals, const diagpu_complex64* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const diagpu_gpair* pairs, int64_t max_pairs,
    diagpu_complex64* C_vals, void* stream)
{
    using diagpu::cf32;
    return diagpu::numeric_launch<cf32>(n, reinterpret_cast<const cf32*>(A_vals),
                                        reinterpret_cast<const cf32*>(B_vals), C_off, C_len,
                                        C_starts, c_ndiag, pair_ptr, pairs, max_pairs,
                                        reinterpret_cast<cf32*>(C_vals), stream,
                                        "diagpu_spgemm_numeric_c64");
}

}  // extern "C"
