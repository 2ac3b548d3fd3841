// DIA x DIA SpGEMM, symbolic (integer) phase on the GPU.
//
// Produces, bit for bit, what the reference's host planners produce:
//   C offsets   make_c_structure (spmspm/bench_spmspm.cu:109-131) /
//               compute_c_hm_structure (spmspm/paper_hm.cuh:87-117):
//               presence of every da + db with |da + db| < n, read out in
//               ascending offset order; lengths n - |dc|; starts = exclusive
//               prefix sum of the lengths (int64 here).
//   C lookup    build_c_diag_lookup (spmspm/paper_hm.cuh:121-130).
//   pair plan   build_pairs_only (spmspm/gather_flat.cuh:231-255): per C
//               diagonal, per B diagonal in B's order, the A diagonal with
//               da = dc - db (A offset lookup over the 2n - 1 offsets), as
//               GPair{A_starts[ai], B_starts[bi], min0(da) - min0(dc),
//               da + min0(db) - min0(dc), A_len[ai], B_len[bi]}.
//
// GPU formulation (every step is integer and order-independent, so the
// result does not depend on scheduling).  Two paths:
//
// One launch (k_sym_fast, below): for operand products of up to 2^20
// (a, b) pairs whose offset spans fit in a workgroup's LDS (bitmaps over the
// spans, not over the 2n - 1 offsets).  A kernel launch costs about 10 us of
// dispatch here, more than any of the small kernels of the path below, so
// this path's single launch plus one copy is the whole phase.
//
// Multi-launch, for everything else:
//   1 init        fill the A lookup with -1 and clear the bitmaps
//   2 operands    validate A/B offsets and lengths, scatter the A lookup,
//                 detect duplicates (atomicExch / atomicOr old values)
//   3 mark        one lane per (a, b): set bit dc + n - 1 of the C bitmap
//   4 word sums   popcount per 256-word block
//   5 word scan   one workgroup: exclusive scan of the block counts -> nC
//   6 emit        per word: block scan of popcounts, write C_off/C_len for
//                 each set bit in ascending order, keep the word prefix
//   7 lookup      (optional) one lane per offset: C index or -1
//   8 count       one lane per C diagonal: pairs (loop over B) and useful
//                 flops, block sums of lengths and counts
//   9 scan top    one workgroup: exclusive scan of the block sums
//  10 scan final  C_starts and pair_ptr
//  11 fill        one lane per C diagonal: the GPairs in B order
// then one synchronous device-to-host copy of the counts on the stream.
#include <climits>
#include <mutex>

#include "common.hpp"
#include "scan.hpp"
#include "spgemm_internal.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;

// One-launch path (k_sym_fast): workgroup size, dynamic LDS per workgroup,
// largest grid, and the largest operand product it takes.
constexpr int kFastBlock = 512;
constexpr int kFastWaves = kFastBlock / 64;
constexpr int kFastLdsBytes = 128 * 1024;
constexpr int kFastLdsWords = kFastLdsBytes / 4;
constexpr int kMaxFastGroups = 1024;
constexpr int64_t kFastMaxProducts = int64_t(1) << 20;

enum : int32_t {
    kFlagAOffset = 1,
    kFlagBOffset = 2,
    kFlagADup = 4,
    kFlagBDup = 8,
    kFlagCCapacity = 16,
    kFlagPairCapacity = 32,
    kFlagFallback = 64,   // the one-launch path cannot hold the operands in LDS
};

struct SymState {
    int64_t c_ndiag;
    int64_t c_nnz;
    int64_t n_pairs;
    int64_t max_pairs;
    int64_t useful_flops;
    int32_t flags;
    int32_t pad;
    int64_t a_extent;     // values A's starts and lengths address: max(start + length)
    int64_t b_extent;
};
static_assert(sizeof(SymState) == 64, "state is one 64-byte record");

struct Layout {
    int64_t nlk = 0;       // 2n - 1 offsets
    int64_t nwords = 0;    // 32-bit words of one bitmap
    int64_t nwblocks = 0;  // workgroups over the words
    int64_t cmax = 0;      // upper bound of the C diagonal count
    int64_t nkblocks = 0;  // workgroups over C diagonals
    size_t off_alk = 0, off_bbits = 0, off_cbits = 0, off_wprefix = 0, off_wsum = 0,
           off_part = 0, off_state = 0, total = 0;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

Layout layout_for(int32_t n, int32_t na, int32_t nb)
{
    Layout L;
    L.nlk = 2 * (int64_t)n - 1;
    L.nwords = ceil_div<int64_t>(L.nlk, 32);
    L.nwblocks = ceil_div<int64_t>(L.nwords, kBlock);
    const int64_t pairs = (int64_t)na * nb;
    L.cmax = pairs < L.nlk ? pairs : L.nlk;
    L.nkblocks = ceil_div<int64_t>(L.cmax + 1, kBlock);
    size_t o = 0;
    L.off_alk = o;     o = align256(o + sizeof(int32_t) * L.nlk);
    L.off_bbits = o;   o = align256(o + sizeof(uint32_t) * L.nwords);
    L.off_cbits = o;   o = align256(o + sizeof(uint32_t) * L.nwords);
    L.off_wprefix = o; o = align256(o + sizeof(int32_t) * L.nwords);
    L.off_wsum = o;    o = align256(o + sizeof(int64_t) * L.nwblocks);
    L.off_part = o;    o = align256(o + 2 * sizeof(int64_t) * L.nkblocks);
    L.off_state = o;   o = align256(o + sizeof(SymState) + 2 * sizeof(int32_t) * kMaxFastGroups);
    L.total = o;
    return L;
}

__device__ __forceinline__ int iabs_(int x) { return x < 0 ? -x : x; }
__device__ __forceinline__ int imin0(int x) { return x < 0 ? x : 0; }

__device__ __forceinline__ void raise_flag(SymState* st, int32_t f) { atomicOr(&st->flags, f); }

__global__ __launch_bounds__(kBlock) void k_init(int32_t* __restrict__ alk, int64_t nlk,
                                                 uint32_t* __restrict__ bbits,
                                                 uint32_t* __restrict__ cbits, int64_t nwords,
                                                 SymState* __restrict__ st)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = t0; i < nlk; i += stride) alk[i] = -1;
    for (int64_t i = t0; i < nwords; i += stride) {
        bbits[i] = 0;
        cbits[i] = 0;
    }
    if (t0 == 0) {
        st->c_ndiag = 0;
        st->c_nnz = 0;
        st->n_pairs = 0;
        st->max_pairs = 0;
        st->useful_flops = 0;
        st->flags = 0;
        st->pad = 0;
        st->a_extent = 0;
        st->b_extent = 0;
    }
}

__global__ __launch_bounds__(kBlock) void k_operands(int32_t n, const int32_t* __restrict__ A_off,
                                                     const int32_t* __restrict__ A_len,
                                                     const int64_t* __restrict__ A_starts, int32_t na,
                                                     const int32_t* __restrict__ B_off,
                                                     const int32_t* __restrict__ B_len,
                                                     const int64_t* __restrict__ B_starts, int32_t nb,
                                                     int32_t* __restrict__ alk,
                                                     uint32_t* __restrict__ bbits,
                                                     SymState* __restrict__ st)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < na) {
        const int d = A_off[t];
        if (d <= -n || d >= n || A_len[t] != n - iabs_(d)) {
            raise_flag(st, kFlagAOffset);
        } else {
            if (atomicExch(&alk[d + (n - 1)], t) != -1) raise_flag(st, kFlagADup);
            atomicMax((unsigned long long*)&st->a_extent,
                      (unsigned long long)(A_starts[t] + A_len[t]));
        }
    }
    if (t < nb) {
        const int d = B_off[t];
        if (d <= -n || d >= n || B_len[t] != n - iabs_(d)) {
            raise_flag(st, kFlagBOffset);
        } else {
            const int64_t pos = d + (int64_t)(n - 1);
            const uint32_t m = 1u << (pos & 31);
            if (atomicOr(&bbits[pos >> 5], m) & m) raise_flag(st, kFlagBDup);
            atomicMax((unsigned long long*)&st->b_extent,
                      (unsigned long long)(B_starts[t] + B_len[t]));
        }
    }
}

__global__ __launch_bounds__(kBlock) void k_mark(int32_t n, const int32_t* __restrict__ A_off,
                                                 int32_t na, const int32_t* __restrict__ B_off,
                                                 int32_t nb, uint32_t* __restrict__ cbits)
{
    const int64_t total = (int64_t)na * nb;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
        const int a = (int)(t / nb), b = (int)(t - (int64_t)a * nb);
        const int64_t dc = (int64_t)A_off[a] + B_off[b];
        if (dc > -(int64_t)n && dc < n) {
            const int64_t pos = dc + (n - 1);
            atomicOr(&cbits[pos >> 5], 1u << (pos & 31));
        }
    }
}

__global__ __launch_bounds__(kBlock) void k_word_sums(const uint32_t* __restrict__ cbits,
                                                      int64_t nwords, int64_t* __restrict__ wsum)
{
    __shared__ int64_t lds[kBlock / 64];
    const int64_t w = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    int64_t c = w < nwords ? __popc(cbits[w]) : 0;
    c = wave_sum(c);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t s = 0;
        for (int i = 0; i < kBlock / 64; ++i) s += lds[i];
        wsum[blockIdx.x] = s;
    }
}

// One workgroup: exclusive scan of `count` int64 values in place (chunks of
// kBlock with a running carry); the total goes to *total.
__device__ void scan_in_place(int64_t* __restrict__ v, int64_t count, int64_t* total)
{
    __shared__ int64_t lds[kBlock / 64];
    int64_t carry = 0;
    for (int64_t base = 0; base < count; base += kBlock) {
        const int64_t i = base + threadIdx.x;
        const int64_t x = i < count ? v[i] : 0;
        int64_t sum;
        const int64_t ex = block_exclusive_scan<int64_t, kBlock>(x, sum, lds);
        if (i < count) v[i] = carry + ex;
        carry += sum;
    }
    if (threadIdx.x == 0) *total = carry;
}

__global__ __launch_bounds__(kBlock) void k_word_scan(int64_t* __restrict__ wsum, int64_t nwb,
                                                      SymState* __restrict__ st)
{
    scan_in_place(wsum, nwb, &st->c_ndiag);
}

__global__ __launch_bounds__(kBlock) void k_emit(int32_t n, const uint32_t* __restrict__ cbits,
                                                 int64_t nwords, const int64_t* __restrict__ wsum,
                                                 int32_t* __restrict__ wprefix,
                                                 int32_t* __restrict__ C_off,
                                                 int32_t* __restrict__ C_len, int64_t c_cap,
                                                 SymState* __restrict__ st)
{
    __shared__ int64_t lds[kBlock / 64];
    const int64_t w = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const uint32_t bits = w < nwords ? cbits[w] : 0u;
    int64_t tot;
    const int64_t ex = block_exclusive_scan<int64_t, kBlock>((int64_t)__popc(bits), tot, lds);
    if (w >= nwords) return;
    int64_t ci = wsum[blockIdx.x] + ex;
    wprefix[w] = (int32_t)ci;
    uint32_t m = bits;
    while (m) {
        const int bit = __ffs(m) - 1;
        m &= m - 1;
        const int dc = (int)(w * 32 + bit - (n - 1));
        if (ci < c_cap) {
            C_off[ci] = dc;
            C_len[ci] = n - iabs_(dc);
        } else {
            raise_flag(st, kFlagCCapacity);
        }
        ++ci;
    }
}

__global__ __launch_bounds__(kBlock) void k_lookup(const uint32_t* __restrict__ cbits,
                                                   const int32_t* __restrict__ wprefix,
                                                   int64_t nlk, int32_t* __restrict__ lookup)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < nlk; p += stride) {
        const uint32_t bits = cbits[p >> 5];
        const uint32_t m = 1u << (p & 31);
        lookup[p] = (bits & m) ? wprefix[p >> 5] + __popc(bits & (m - 1)) : -1;
    }
}

__device__ __forceinline__ int64_t c_count(const SymState* st, int64_t c_cap)
{
    const int64_t nc = st->c_ndiag;
    return nc < c_cap ? nc : c_cap;
}

__global__ __launch_bounds__(kBlock) void k_pair_count(
    int32_t n, const int32_t* __restrict__ C_off, const int32_t* __restrict__ C_len,
    int64_t c_cap, const int32_t* __restrict__ B_off, int32_t nb,
    const int32_t* __restrict__ alk, int64_t* __restrict__ pair_ptr,
    int64_t* __restrict__ part, int64_t nkb, SymState* __restrict__ st)
{
    __shared__ int64_t red[2][kBlock / 64];
    const int64_t nc = c_count(st, c_cap);
    const int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    int64_t cnt = 0, len = 0, flops = 0;
    if (k < nc) {
        const int dc = C_off[k];
        len = C_len[k];
        for (int b = 0; b < nb; ++b) {
            const int db = B_off[b];
            const int64_t da = (int64_t)dc - db;
            if (da <= -(int64_t)n || da >= n) continue;
            if (alk[da + (n - 1)] < 0) continue;
            ++cnt;
            int m = iabs_((int)da);
            m = iabs_(db) > m ? iabs_(db) : m;
            m = iabs_(dc) > m ? iabs_(dc) : m;
            flops += 2 * (int64_t)(n - m);
        }
        pair_ptr[k] = cnt;
        atomicMax((unsigned long long*)&st->max_pairs, (unsigned long long)cnt);
    }
    const int64_t s_len = wave_sum(len), s_cnt = wave_sum(cnt), s_fl = wave_sum(flops);
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = s_len;
        red[1][threadIdx.x >> 6] = s_cnt;
        if (s_fl) atomicAdd((unsigned long long*)&st->useful_flops, (unsigned long long)s_fl);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t a = 0, c = 0;
        for (int i = 0; i < kBlock / 64; ++i) {
            a += red[0][i];
            c += red[1][i];
        }
        part[blockIdx.x] = a;
        part[nkb + blockIdx.x] = c;
    }
}

__global__ __launch_bounds__(kBlock) void k_scan_top(int64_t* __restrict__ part, int64_t nkb,
                                                     SymState* __restrict__ st)
{
    scan_in_place(part, nkb, &st->c_nnz);
    __syncthreads();
    scan_in_place(part + nkb, nkb, &st->n_pairs);
}

__global__ __launch_bounds__(kBlock) void k_scan_final(const int32_t* __restrict__ C_len,
                                                       int64_t* __restrict__ pair_ptr,
                                                       int64_t* __restrict__ C_starts,
                                                       const int64_t* __restrict__ part,
                                                       int64_t nkb, int64_t c_cap,
                                                       const SymState* __restrict__ st)
{
    __shared__ int64_t lds[kBlock / 64];
    const int64_t nc = c_count(st, c_cap);
    const int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t len = k < nc ? (int64_t)C_len[k] : 0;
    const int64_t cnt = k < nc ? pair_ptr[k] : 0;
    int64_t t0, t1;
    const int64_t ex_len = block_exclusive_scan<int64_t, kBlock>(len, t0, lds);
    const int64_t ex_cnt = block_exclusive_scan<int64_t, kBlock>(cnt, t1, lds);
    if (k < nc) {
        C_starts[k] = part[blockIdx.x] + ex_len;
        pair_ptr[k] = part[nkb + blockIdx.x] + ex_cnt;
    } else if (k == nc) {
        pair_ptr[k] = st->n_pairs;
    }
}

__global__ __launch_bounds__(kBlock) void k_pair_fill(
    int32_t n, const int32_t* __restrict__ C_off, int64_t c_cap,
    const int32_t* __restrict__ A_len, const int64_t* __restrict__ A_starts,
    const int32_t* __restrict__ B_off, const int32_t* __restrict__ B_len,
    const int64_t* __restrict__ B_starts, int32_t nb, const int32_t* __restrict__ alk,
    const int64_t* __restrict__ pair_ptr, diagpu_gpair* __restrict__ pairs, int64_t p_cap,
    SymState* __restrict__ st)
{
    const int64_t nc = c_count(st, c_cap);
    const int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (k >= nc) return;
    const int dc = C_off[k], minc = imin0(dc);
    int64_t slot = pair_ptr[k];
    for (int b = 0; b < nb; ++b) {
        const int db = B_off[b];
        const int64_t da64 = (int64_t)dc - db;
        if (da64 <= -(int64_t)n || da64 >= n) continue;
        const int da = (int)da64;
        const int ai = alk[da + (n - 1)];
        if (ai < 0) continue;
        if (slot < p_cap) {
            diagpu_gpair g;
            g.ab = (uint64_t)A_starts[ai];
            g.bb = (uint64_t)B_starts[b];
            g.ash = imin0(da) - minc;
            g.bsh = da + imin0(db) - minc;
            g.al = A_len[ai];
            g.bl = B_len[b];
            pairs[slot] = g;
        } else {
            raise_flag(st, kFlagPairCapacity);
        }
        ++slot;
    }
}

// ---------------------------------------------------------------------------
// One-launch symbolic phase.
//
// Every workgroup builds, in LDS, presence bitmaps over the span of A's
// offsets, of B's offsets and of the pair sums [min da + min db, max da +
// max db] clipped to (-n, n), each with an exclusive popcount prefix per
// 32-bit word (rank of an offset = prefix + popcount of the lower bits),
// plus A's index by rank (perm).  Spans, not n, size these structures, so
// they are small for banded operands at any n.  The C diagonals are then
// split into G equal slices, one per workgroup; a workgroup computes the
// global prefixes its slice starts from directly:
//   pair_ptr base  = #{(a, b) : -n < da + db < dc_k0} = sum over A of
//                    rank_B(dc_k0 - da) - rank_B(1 - n - da)
//   C_starts base  = sum over the C offsets below dc_k0 of n - |dc|
// so no workgroup waits for another (no grid barrier, no device-scope
// fence, no global atomics).  Within the slice each wave takes a contiguous
// run of C diagonals: it counts each one's entries (B diagonals 64 at a
// time, da = dc - db present in A, counted with a ballot), the waves
// exchange their totals once, and each wave then writes its diagonals'
// starts, pair_ptr and GPairs (slot ranks from the same ballot: B order).
// Everything a workgroup combines goes through one LDS exchange and one
// barrier per step (eight in all, nine with the A-stationary records).
// Counts, nnz, useful flops and the operands' value extents are computed by
// every workgroup and written by workgroup 0; each workgroup writes its
// largest entry count (wg_max) and, with the records, its flag word (wg_rec),
// and the host combines them.  If the structures exceed the LDS budget the
// kernel only raises kFlagFallback.
// ---------------------------------------------------------------------------

template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op)
{
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v = op(v, __shfl_xor(v, s, 64));
    return v;
}

// Combination of the kFastWaves per-wave values in slot[] (after a barrier).
template <typename T, typename Op>
__device__ __forceinline__ T combine_waves(const T* slot, Op op)
{
    T r = slot[0];
#pragma unroll
    for (int w = 1; w < kFastWaves; ++w) r = op(r, slot[w]);
    return r;
}

// Set bits of `bits` below position q (q >= 0 within the span).
__device__ __forceinline__ int32_t fast_rank(const uint32_t* bits, const int32_t* pfx, int64_t q)
{
    const int64_t w = q >> 5;
    return pfx[w] + __popc(bits[w] & ((1u << (q & 31)) - 1u));
}

__device__ __forceinline__ bool fast_test(const uint32_t* bits, int64_t q)
{
    return (bits[q >> 5] >> (q & 31)) & 1u;
}

// Position (within the span) of the k-th set bit, 0 <= k < total.
__device__ int64_t fast_select(const uint32_t* bits, const int32_t* pfx, int32_t nwords, int64_t k)
{
    int32_t lo = 0, hi = nwords - 1;
    while (lo < hi) {                     // last word whose prefix is <= k
        const int32_t mid = (lo + hi + 1) >> 1;
        if (pfx[mid] <= k) lo = mid; else hi = mid - 1;
    }
    uint32_t m = bits[lo];
    for (int64_t r = k - pfx[lo]; r > 0; --r) m &= m - 1u;
    return (int64_t)lo * 32 + (__ffs(m) - 1);
}

__device__ __forceinline__ int32_t i32min(int32_t x, int32_t y) { return x < y ? x : y; }
__device__ __forceinline__ int32_t i32max(int32_t x, int32_t y) { return x > y ? x : y; }
__device__ __forceinline__ int32_t i32or(int32_t x, int32_t y) { return x | y; }
__device__ __forceinline__ int64_t i64add(int64_t x, int64_t y) { return x + y; }
__device__ __forceinline__ int64_t i64max(int64_t x, int64_t y) { return x > y ? x : y; }

// Words of LDS the operand tables take: A and B starts (int64), lengths,
// offsets, and A's index by rank.
__host__ __device__ constexpr int64_t fast_table_words(int64_t na, int64_t nb)
{
    return 5 * na + 4 * nb;
}

__global__ __launch_bounds__(kFastBlock) void k_sym_fast(
    int32_t n, const int32_t* __restrict__ A_off, const int32_t* __restrict__ A_len,
    const int64_t* __restrict__ A_starts, int32_t na, const int32_t* __restrict__ B_off,
    const int32_t* __restrict__ B_len, const int64_t* __restrict__ B_starts, int32_t nb,
    int32_t* __restrict__ C_off, int32_t* __restrict__ C_len, int64_t* __restrict__ C_starts,
    int64_t c_cap, int64_t* __restrict__ pair_ptr, diagpu_gpair* __restrict__ pairs,
    int64_t p_cap, int32_t* __restrict__ lookup, SymState* __restrict__ st,
    int32_t* __restrict__ wg_max, int32_t* __restrict__ records, int32_t* __restrict__ wg_rec)
{
    extern __shared__ uint32_t lds[];
    __shared__ int32_t s32[8][kFastWaves];        // one slot per combined value
    __shared__ int64_t s64[10][kFastWaves];
    __shared__ int32_t sscan[3][kFastWaves];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = (int)gridDim.x, wg = (int)blockIdx.x;
    const bool lane0 = lane == 0;

    // LDS: the operand tables, then the bitmaps and this slice's C offsets
    int64_t* ast = reinterpret_cast<int64_t*>(lds);
    int64_t* bst = ast + na;
    int32_t* alen = reinterpret_cast<int32_t*>(bst + nb);
    int32_t* blen = alen + na;
    int32_t* aoff = blen + nb;
    int32_t* boff = aoff + na;
    int32_t* perm = boff + nb;
    uint32_t* bitbase = reinterpret_cast<uint32_t*>(perm + na);
    const int64_t free_words = kFastLdsWords - fast_table_words(na, nb);

    // 1. operand tables into LDS; validity, ranges, value extents.  The
    //    bitmap area is cleared meanwhile (whatever part the spans use).
    int32_t amin = INT_MAX, amax = INT_MIN, bmin = INT_MAX, bmax = INT_MIN, bad = 0;
    int64_t aext = 0, bext = 0;
    for (int a = tid; a < na; a += kFastBlock) {
        const int d = A_off[a], l = A_len[a];
        const int64_t s0 = A_starts[a];
        aoff[a] = d;
        alen[a] = l;
        ast[a] = s0;
        if (d <= -n || d >= n || l != n - iabs_(d)) {
            bad |= kFlagAOffset;
        } else {
            amin = i32min(amin, d);
            amax = i32max(amax, d);
            aext = i64max(aext, s0 + l);
        }
    }
    for (int b = tid; b < nb; b += kFastBlock) {
        const int d = B_off[b], l = B_len[b];
        const int64_t s0 = B_starts[b];
        boff[b] = d;
        blen[b] = l;
        bst[b] = s0;
        if (d <= -n || d >= n || l != n - iabs_(d)) {
            bad |= kFlagBOffset;
        } else {
            bmin = i32min(bmin, d);
            bmax = i32max(bmax, d);
            bext = i64max(bext, s0 + l);
        }
    }
    {   // bitbase is 16-byte aligned when the tables are (5 na + 4 nb words)
        const int64_t lead = (4 - (fast_table_words(na, nb) & 3)) & 3;
        for (int64_t w = tid; w < lead && w < free_words; w += kFastBlock) bitbase[w] = 0u;
        uint4* q = reinterpret_cast<uint4*>(bitbase + lead);
        const int64_t nq = (free_words - lead) >> 2;
        for (int64_t w = tid; w < nq; w += kFastBlock) q[w] = uint4{0u, 0u, 0u, 0u};
        for (int64_t w = lead + 4 * nq + tid; w < free_words; w += kFastBlock) bitbase[w] = 0u;
    }
    bad = wave_reduce(bad, i32or);
    amin = wave_reduce(amin, i32min);
    amax = wave_reduce(amax, i32max);
    bmin = wave_reduce(bmin, i32min);
    bmax = wave_reduce(bmax, i32max);
    aext = wave_reduce(aext, i64max);
    bext = wave_reduce(bext, i64max);
    if (lane0) {
        s32[0][wave] = bad;
        s32[1][wave] = amin;
        s32[2][wave] = amax;
        s32[3][wave] = bmin;
        s32[4][wave] = bmax;
        s64[0][wave] = aext;
        s64[1][wave] = bext;
    }
    __syncthreads();                                                   // barrier 1
    bad = combine_waves(s32[0], i32or);
    amin = combine_waves(s32[1], i32min);
    amax = combine_waves(s32[2], i32max);
    bmin = combine_waves(s32[3], i32min);
    bmax = combine_waves(s32[4], i32max);
    aext = combine_waves(s64[0], i64max);
    bext = combine_waves(s64[1], i64max);
    auto report = [&](int32_t flags, int64_t nc, int64_t nnz, int64_t np, int64_t fl) {
        if (wg == 0 && tid == 0) {
            st->c_ndiag = nc;
            st->c_nnz = nnz;
            st->n_pairs = np;
            st->max_pairs = 0;
            st->useful_flops = fl;
            st->flags = flags;
            st->pad = 0;
            st->a_extent = aext;
            st->b_extent = bext;
        }
    };
    if (bad) {
        report(bad, 0, 0, 0, 0);
        return;
    }

    // 2. bitmaps of the A, B and sum spans, their word prefixes, and room for
    //    the slice's C offsets (at most ceil(min(na nb, span) / G) of them)
    const int64_t SA = na ? (int64_t)amax - amin + 1 : 0;
    const int64_t SB = nb ? (int64_t)bmax - bmin + 1 : 0;
    int64_t clo = 0, chi = -1;
    if (na && nb) {
        clo = (int64_t)amin + bmin;
        chi = (int64_t)amax + bmax;
        if (clo < 1 - (int64_t)n) clo = 1 - (int64_t)n;
        if (chi > (int64_t)n - 1) chi = (int64_t)n - 1;
    }
    const int64_t SC = chi >= clo ? chi - clo + 1 : 0;
    const int64_t wa = (SA + 31) >> 5, wb = (SB + 31) >> 5, wc = (SC + 31) >> 5;
    const int64_t cmax = (int64_t)na * nb < SC ? (int64_t)na * nb : SC;
    const int64_t rmax = (cmax + G - 1) / G;
    if (2 * (wa + wb + wc) + rmax > free_words) {
        report(kFlagFallback, 0, 0, 0, 0);
        return;
    }
    uint32_t* abits = bitbase;
    int32_t* apfx = reinterpret_cast<int32_t*>(abits + wa);
    uint32_t* bbits = reinterpret_cast<uint32_t*>(apfx + wa);
    int32_t* bpfx = reinterpret_cast<int32_t*>(bbits + wb);
    uint32_t* cbits = reinterpret_cast<uint32_t*>(bpfx + wb);
    int32_t* cpfx = reinterpret_cast<int32_t*>(cbits + wc);
    int32_t* rows = cpfx + wc;                       // the slice's C offsets

    // a bit already set is a repeated offset
    int32_t dup = 0;
    for (int a = tid; a < na; a += kFastBlock) {
        const int64_t q = (int64_t)aoff[a] - amin;
        const uint32_t m = 1u << (q & 31);
        if (atomicOr(&abits[q >> 5], m) & m) dup |= kFlagADup;
    }
    for (int b = tid; b < nb; b += kFastBlock) {
        const int64_t q = (int64_t)boff[b] - bmin;
        const uint32_t m = 1u << (q & 31);
        if (atomicOr(&bbits[q >> 5], m) & m) dup |= kFlagBDup;
    }
    // sums: lanes over B (offsets held in registers, 4 per lane at a time),
    // waves over A; pair count, useful flops
    int64_t np = 0, fl = 0;
    for (int b0 = 0; b0 < nb; b0 += 4 * 64) {
        int db[4];
        bool has[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = b0 + j * 64 + lane;
            has[j] = b < nb;
            db[j] = has[j] ? boff[b] : 0;
        }
        // this wave's A offsets (a = wave + kFastWaves i) one per lane, then
        // taken lane by lane with readlane: no LDS read between the atomics
        for (int a0 = wave; a0 < na; a0 += 64 * kFastWaves) {
            const int ai = a0 + lane * kFastWaves;
            const int mine = ai < na ? aoff[ai] : 0;
            const int cnt = (na - a0 + kFastWaves - 1) / kFastWaves < 64
                                ? (na - a0 + kFastWaves - 1) / kFastWaves : 64;
            for (int i = 0; i < cnt; ++i) {
                const int da = __builtin_amdgcn_readlane(mine, i);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t dc = (int64_t)da + db[j];
                    if (has[j] && dc > -(int64_t)n && dc < n) {
                        const int64_t q = dc - clo;
                        atomicOr(&cbits[q >> 5], 1u << (q & 31));
                        ++np;
                        int m = iabs_(da) > iabs_(db[j]) ? iabs_(da) : iabs_(db[j]);
                        m = iabs_((int)dc) > m ? iabs_((int)dc) : m;
                        fl += 2 * (int64_t)(n - m);
                    }
                }
            }
        }
    }
    dup = wave_reduce(dup, i32or);
    np = wave_reduce(np, i64add);
    fl = wave_reduce(fl, i64add);
    if (lane0) {
        s32[5][wave] = dup;
        s64[2][wave] = np;
        s64[3][wave] = fl;
    }
    __syncthreads();                                                   // barrier 2
    dup = combine_waves(s32[5], i32or);
    np = combine_waves(s64[2], i64add);
    fl = combine_waves(s64[3], i64add);
    if (dup) {
        report(dup, 0, 0, 0, 0);
        return;
    }

    // word prefixes of the three bitmaps together: each thread takes kPer
    // consecutive words per step
    constexpr int kPer = 4;
    int32_t carry[3] = {0, 0, 0};
    const int64_t wmax = wa > wb ? (wa > wc ? wa : wc) : (wb > wc ? wb : wc);
    for (int64_t base = 0; base < wmax; base += (int64_t)kFastBlock * kPer) {
        const int64_t w0 = base + (int64_t)tid * kPer;
        const uint32_t* bm[3] = {abits, bbits, cbits};
        int32_t* pf[3] = {apfx, bpfx, cpfx};
        const int64_t nw[3] = {wa, wb, wc};
        int32_t loc[3][kPer], tot[3], incl[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            int32_t t = 0;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                loc[j][i] = t;
                t += (w0 + i < nw[j]) ? __popc(bm[j][w0 + i]) : 0;
            }
            tot[j] = t;
            incl[j] = wave_inclusive_scan(t);
            if (lane == 63) sscan[j][wave] = incl[j];
        }
        __syncthreads();
        int32_t before[3] = {0, 0, 0}, sum[3] = {0, 0, 0};
        for (int v = 0; v < kFastWaves; ++v)
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int32_t t = sscan[j][v];
                before[j] += v < wave ? t : 0;
                sum[j] += t;
            }
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int32_t first = carry[j] + before[j] + incl[j] - tot[j];
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (w0 + i < nw[j]) pf[j][w0 + i] = first + loc[j][i];
            carry[j] += sum[j];
        }
        __syncthreads();   // sscan is rewritten by the next step
    }
    const int64_t nC = carry[2];
    if (wmax == 0) __syncthreads();                 // the prefix step's barrier

    // 3. A index by rank; this workgroup's C diagonals [k0, k1) into `rows`
    //    and the prefixes they start from; the C value count
    for (int a = tid; a < na; a += kFastBlock) perm[fast_rank(abits, apfx, (int64_t)aoff[a] - amin)] = a;
    auto rank_b = [&](int64_t x) -> int64_t {       // B offsets below x
        if (x <= bmin) return 0;
        if (x > bmax) return nb;
        return fast_rank(bbits, bpfx, x - bmin);
    };
    const int64_t k0 = nC * wg / G, k1 = nC * (wg + 1) / G;
    int64_t lb = 0, nz = 0;
    for (int64_t w = tid; w < wc; w += kFastBlock) {
        int64_t r = cpfx[w];
        for (uint32_t m = cbits[w]; m; m &= m - 1u, ++r) {
            const int64_t o = clo + w * 32 + (__ffs(m) - 1);
            const int64_t len = (int64_t)n - (o < 0 ? -o : o);
            nz += len;
            lb += r < k0 ? len : 0;
            if (r >= k0 && r < k1) rows[r - k0] = (int32_t)o;
        }
    }
    lb = wave_reduce(lb, i64add);
    nz = wave_reduce(nz, i64add);
    if (lane0) {
        s64[5][wave] = lb;
        s64[6][wave] = nz;
    }
    __syncthreads();                                                   // barrier 3
    const int64_t nnz = combine_waves(s64[6], i64add);
    int64_t pbase = np, lbase = nnz;
    if (k0 < nC) {
        const int64_t d0 = rows[0];
        int64_t pb = 0;
        for (int a = tid; a < na; a += kFastBlock)
            pb += rank_b(d0 - aoff[a]) - rank_b(1 - (int64_t)n - aoff[a]);
        pb = wave_reduce(pb, i64add);
        if (lane0) s64[4][wave] = pb;
        lbase = combine_waves(s64[5], i64add);
    }
    int32_t flags = 0;
    if (nC > c_cap) flags |= kFlagCCapacity;
    if (np > p_cap) flags |= kFlagPairCapacity;
    report(flags, nC, nnz, np, fl);
    if (flags) return;
    if (records && wg == 0 && tid == 0)   // the 4 ints after the records
        reinterpret_cast<int4*>(records)[np] = int4{0, 0, amin, amax};

    // 4. each wave's run of C diagonals: counts, then one exchange
    const int64_t R = k1 - k0;
    const int64_t r0 = R * wave / kFastWaves, r1 = R * (wave + 1) / kFastWaves;
    auto entry = [&](int dc, int b, int64_t& da) -> bool {   // B diagonal b feeds dc
        if (b >= nb) return false;
        da = (int64_t)dc - boff[b];
        return da >= amin && da <= amax && fast_test(abits, da - amin);
    };
    int64_t wcnt = 0, wlen = 0;
    int32_t wmx = 0;
    for (int64_t r = r0; r < r1; ++r) {
        const int dc = rows[r];
        int32_t cnt = 0;
        for (int b0 = 0; b0 < nb; b0 += 64) {
            int64_t da;
            cnt += __popcll(__ballot(entry(dc, b0 + lane, da)));
        }
        wcnt += cnt;
        wlen += n - iabs_(dc);
        wmx = cnt > wmx ? cnt : wmx;
    }
    if (lane0) {
        s64[7][wave] = wcnt;
        s64[8][wave] = wlen;
        s32[6][wave] = wmx;
    }
    __syncthreads();                                                   // barrier 4
    if (k0 < nC) pbase = combine_waves(s64[4], i64add);
    int64_t slot = pbase, lpos = lbase;
    for (int v = 0; v < wave; ++v) {
        slot += s64[7][v];
        lpos += s64[8][v];
    }
    if (tid == 0) wg_max[wg] = combine_waves(s32[6], i32max);
    if (wg == G - 1 && tid == 0) pair_ptr[nC] = np;

    // 5. the run's starts, pair_ptr, C offsets and lengths, and GPairs (B
    //    order within each C diagonal); with `records`, each entry's record
    //    as diagpu_spgemm_astat_prepare forms it ({A index, lo, hi, b}; every
    //    entry here is in the symbolic form), rflag set for a B index beyond
    //    2^30 - 1
    int32_t rflag = 0;
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t k = k0 + r;
        const int dc = rows[r];
        const int minc = imin0(dc);
        if (lane0) {
            C_off[k] = dc;
            C_len[k] = n - iabs_(dc);
            C_starts[k] = lpos;
            pair_ptr[k] = slot;
        }
        lpos += n - iabs_(dc);
        for (int b0 = 0; b0 < nb; b0 += 64) {
            const int b = b0 + lane;
            int64_t da = 0;
            const bool v = entry(dc, b, da);
            const uint64_t m = __ballot(v);
            if (v) {
                const int ai = perm[fast_rank(abits, apfx, da - amin)];
                const int db = boff[b];
                diagpu_gpair g;
                g.ab = (uint64_t)ast[ai];
                g.bb = (uint64_t)bst[b];
                g.ash = imin0((int)da) - minc;
                g.bsh = (int)da + imin0(db) - minc;
                g.al = alen[ai];
                g.bl = blen[b];
                const int64_t at = slot + __popcll(m & ((1ull << lane) - 1ull));
                pairs[at] = g;
                if (records) {
                    const int plo = i32max(0, i32max(-g.ash, -g.bsh));
                    const int phi = i32min(g.al - g.ash, g.bl - g.bsh);
                    const int64_t bq = (int64_t)g.bb + g.bsh;
                    int4 rec = int4{ai, plo, phi, (int)bq};
                    if (plo >= phi) {
                        rec = int4{ai, 1, 1, 0};    // never fires (see k_astat_prepare)
                    } else if (bq < INT_MIN || bq + phi > ((int64_t)1 << 30)) {
                        rec = int4{0, 0, 0, 0};
                        rflag = 1;
                    }
                    reinterpret_cast<int4*>(records)[at] = rec;
                }
            }
            slot += __popcll(m);
        }
    }
    if (records) {   // one word per workgroup: the host ORs them
        rflag = wave_reduce(rflag, i32or);
        if (lane0) s32[7][wave] = rflag;
        __syncthreads();
        if (tid == 0) wg_rec[wg] = combine_waves(s32[7], i32or);
    }

    // 6. lookup: every offset of the 2n - 1, grid-stride over all workgroups
    if (lookup) {
        const int64_t nlk = 2 * (int64_t)n - 1;
        for (int64_t p = (int64_t)wg * kFastBlock + tid; p < nlk; p += (int64_t)G * kFastBlock) {
            const int64_t o = p - (n - 1);
            int32_t v = -1;
            if (o >= clo && o <= chi && fast_test(cbits, o - clo)) v = fast_rank(cbits, cpfx, o - clo);
            lookup[p] = v;
        }
    }
}

int grid_for(int64_t work, int64_t cap = 65536)
{
    int64_t g = ceil_div<int64_t>(work, kBlock);
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

// Scratch of diagpu_spgemm_symbolic_noalloc: the workspace of the symbolic
// phase held in a file-scope device array, for callers that cannot allocate.
// Each device that runs the library holds its own copy until the process ends.
// Host code never uses the name `scratch` as an address (on the host it names
// a stand-in, not device memory); it uses the per-device address from
// hipGetSymbolAddress that scratch_ptr() keeps.
constexpr size_t kScratchBytes = DIAGPU_SYMBOLIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_ptr(const char* fn, void** out)
{
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), fn);
    if (rc) return rc;
    if (dev < 0 || dev >= 64) return fail(DIAGPU_ERR_ARG, "%s: device %d out of range", fn, dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), fn);
        if (rc) return rc;
        if (!p) return fail(DIAGPU_ERR_HIP, "%s: no device address for the scratch array", fn);
        addr[dev] = p;
    }
    *out = addr[dev];
    return DIAGPU_OK;
}

// One lock per device over that device's scratch array: a no-alloc call holds
// it from before its first launch until its stream has drained, so calls that
// overlap in one process (other host threads, other streams) run one after
// the other instead of racing for the array.
std::mutex& scratch_lock(int dev)
{
    static std::mutex mu[64];
    return mu[dev];
}

// Waits for `s` when armed: on an error return after a launch, the queued
// kernels may still use the scratch array, so the lock is released only after
// they finish.  Declared after the lock, so it runs before the unlock.
struct DrainOnExit {
    hipStream_t s = nullptr;
    bool armed = false;
    ~DrainOnExit()
    {
        if (armed) (void)hipStreamSynchronize(s);
    }
};

// k_sym_fast takes kFastLdsBytes of dynamic LDS; more than 64 KiB must be
// allowed explicitly (once per device).
int fast_lds_allowed(const char* fn)
{
    static std::mutex mu;
    static bool done[64] = {};
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), fn);
    if (rc) return rc;
    if (dev < 0 || dev >= 64) return fail(DIAGPU_ERR_ARG, "%s: device %d out of range", fn, dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!done[dev]) {
        rc = check_hip(hipFuncSetAttribute((const void*)k_sym_fast,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kFastLdsBytes), fn);
        if (rc) return rc;
        done[dev] = true;
    }
    return DIAGPU_OK;
}

// The two entry points below share this runner.  workspace == nullptr asks
// for the file-scope scratch array (diagpu_spgemm_symbolic_noalloc).
int run_symbolic(
    const char* fn, int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup, bool use_scratch,
    void* workspace, size_t workspace_bytes,
    int32_t* records, int32_t* records_status,
    diagpu_spgemm_info* info, void* stream)
{
    if (!info) return fail(DIAGPU_ERR_ARG, "%s: info is NULL", fn);
    if (records && !records_status) return fail(DIAGPU_ERR_ARG, "%s: records_status is NULL", fn);
    if (n < 1 || n > (1 << 30))
        return fail(DIAGPU_ERR_ARG, "%s: n=%d outside [1, 2^30]", fn, n);
    if (a_ndiag < 0 || b_ndiag < 0 || c_capacity < 0 || pair_capacity < 0)
        return fail(DIAGPU_ERR_ARG, "%s: negative count", fn);
    if (a_ndiag > 0 && (!A_off || !A_len || !A_starts))
        return fail(DIAGPU_ERR_ARG, "%s: A arrays are NULL", fn);
    if (b_ndiag > 0 && (!B_off || !B_len || !B_starts))
        return fail(DIAGPU_ERR_ARG, "%s: B arrays are NULL", fn);
    if (!pair_ptr) return fail(DIAGPU_ERR_ARG, "%s: pair_ptr is NULL", fn);
    if (c_capacity > 0 && (!C_off || !C_len || !C_starts))
        return fail(DIAGPU_ERR_ARG, "%s: C arrays are NULL", fn);
    if (pair_capacity > 0 && !pairs) return fail(DIAGPU_ERR_ARG, "%s: pairs is NULL", fn);
    const Layout L = layout_for(n, a_ndiag, b_ndiag);
    std::unique_lock<std::mutex> scratch_guard;
    if (use_scratch) {
        if (L.total > kScratchBytes)
            return fail(DIAGPU_ERR_CAPACITY,
                        "%s: n=%d with %d x %d diagonals needs %zu bytes of scratch, more than "
                        "the %zu the library holds (use diagpu_spgemm_symbolic with a workspace)",
                        fn, n, a_ndiag, b_ndiag, L.total, kScratchBytes);
        int dev = 0;
        int rc = check_hip(hipGetDevice(&dev), fn);
        if (rc) return rc;
        if (dev < 0 || dev >= 64)
            return fail(DIAGPU_ERR_ARG, "%s: device %d out of range", fn, dev);
        scratch_guard = std::unique_lock<std::mutex>(scratch_lock(dev));
        rc = scratch_ptr(fn, &workspace);
        if (rc) return rc;
        workspace_bytes = kScratchBytes;
    }
    if (!workspace) return fail(DIAGPU_ERR_ARG, "%s: workspace is NULL", fn);
    if (workspace_bytes < L.total)
        return fail(DIAGPU_ERR_CAPACITY, "%s: workspace has %zu bytes, needs %zu", fn,
                    workspace_bytes, L.total);

    char* ws = static_cast<char*>(workspace);
    int32_t* alk = reinterpret_cast<int32_t*>(ws + L.off_alk);
    uint32_t* bbits = reinterpret_cast<uint32_t*>(ws + L.off_bbits);
    uint32_t* cbits = reinterpret_cast<uint32_t*>(ws + L.off_cbits);
    int32_t* wprefix = reinterpret_cast<int32_t*>(ws + L.off_wprefix);
    int64_t* wsum = reinterpret_cast<int64_t*>(ws + L.off_wsum);
    int64_t* part = reinterpret_cast<int64_t*>(ws + L.off_part);
    SymState* st = reinterpret_cast<SymState*>(ws + L.off_state);
    hipStream_t s = as_stream(stream);
    int32_t* wg_max = reinterpret_cast<int32_t*>(st + 1);   // after the state record
    struct {
        SymState h;
        int32_t m[2 * kMaxFastGroups];   // wg_max[0 .. G), then wg_rec[0 .. G)
    } back;
    int32_t rec_flags = 0;   // the records step's flags (1: form, 2: B index)
    SymState& h = back.h;
    int rc = DIAGPU_OK;
    DrainOnExit drain;
    drain.s = s;

    // The one-launch path where the operand product is small enough for each
    // workgroup to enumerate (it reports kFlagFallback when the spans do not
    // fit in its LDS); the multi-launch path below otherwise.
    bool done = false;
    if ((int64_t)a_ndiag * b_ndiag <= kFastMaxProducts &&
        fast_table_words(a_ndiag, b_ndiag) <= kFastLdsWords / 2) {
        rc = fast_lds_allowed(fn);
        if (rc) return rc;
        int64_t ub = (int64_t)a_ndiag * b_ndiag;
        if (ub > 2 * (int64_t)n - 1) ub = 2 * (int64_t)n - 1;
        int64_t G = ceil_div<int64_t>(ub, 32);
        const int64_t gmax = cu_count() < kMaxFastGroups ? cu_count() : kMaxFastGroups;
        G = G < 1 ? 1 : (G > gmax ? gmax : G);
        drain.armed = use_scratch;
        // the kernel writes the records itself (with each entry), and one
        // flag word per workgroup after wg_max
        int32_t* wg_rec = wg_max + G;
        hipLaunchKernelGGL(k_sym_fast, dim3((unsigned)G), dim3(kFastBlock), kFastLdsBytes, s, n,
                           A_off, A_len, A_starts, a_ndiag, B_off, B_len, B_starts, b_ndiag,
                           C_off, C_len, C_starts, c_capacity, pair_ptr, pairs, pair_capacity,
                           c_lookup, st, wg_max, records, wg_rec);
        rc = check_launch(fn);
        if (rc) return rc;
        // one synchronous, stream-ordered copy: the kernel and everything
        // before it on `s` are complete when it returns (it costs about
        // 9 us less than an asynchronous copy plus a stream synchronisation)
        const size_t words = (records ? 2 : 1) * (size_t)G;
        rc = check_hip(hipMemcpyWithStream(&back, st, sizeof(SymState) + sizeof(int32_t) * words,
                                           hipMemcpyDeviceToHost, s), fn);
        if (rc) return rc;
        drain.armed = false;
        if (!(h.flags & kFlagFallback)) {
            int32_t mx = 0;
            for (int64_t g = 0; g < G && !h.flags; ++g) mx = back.m[g] > mx ? back.m[g] : mx;
            h.max_pairs = mx;
            if (records && !h.flags)
                for (int64_t g = 0; g < G; ++g) rec_flags |= back.m[G + g] ? 2 : 0;
            done = true;
        }
    }
    if (!done) {
        const int64_t c_cap = c_capacity < L.cmax ? c_capacity : L.cmax;
        const int64_t nkb = ceil_div<int64_t>(c_cap + 1, kBlock);

        drain.armed = use_scratch;
        hipLaunchKernelGGL(k_init, dim3(grid_for(L.nlk, 4096)), dim3(kBlock), 0, s, alk, L.nlk, bbits,
                           cbits, L.nwords, st);
        hipLaunchKernelGGL(k_operands, dim3(grid_for(a_ndiag > b_ndiag ? a_ndiag : b_ndiag)),
                           dim3(kBlock), 0, s, n, A_off, A_len, A_starts, a_ndiag, B_off, B_len,
                           B_starts, b_ndiag, alk, bbits, st);
        hipLaunchKernelGGL(k_mark, dim3(grid_for((int64_t)a_ndiag * b_ndiag, 8192)), dim3(kBlock), 0,
                           s, n, A_off, a_ndiag, B_off, b_ndiag, cbits);
        hipLaunchKernelGGL(k_word_sums, dim3((unsigned)L.nwblocks), dim3(kBlock), 0, s, cbits,
                           L.nwords, wsum);
        hipLaunchKernelGGL(k_word_scan, dim3(1), dim3(kBlock), 0, s, wsum, L.nwblocks, st);
        hipLaunchKernelGGL(k_emit, dim3((unsigned)L.nwblocks), dim3(kBlock), 0, s, n, cbits, L.nwords,
                           wsum, wprefix, C_off, C_len, c_cap, st);
        if (c_lookup)
            hipLaunchKernelGGL(k_lookup, dim3(grid_for(L.nlk, 8192)), dim3(kBlock), 0, s, cbits,
                               wprefix, L.nlk, c_lookup);
        hipLaunchKernelGGL(k_pair_count, dim3((unsigned)nkb), dim3(kBlock), 0, s, n, C_off, C_len,
                           c_cap, B_off, b_ndiag, alk, pair_ptr, part, nkb, st);
        hipLaunchKernelGGL(k_scan_top, dim3(1), dim3(kBlock), 0, s, part, nkb, st);
        hipLaunchKernelGGL(k_scan_final, dim3((unsigned)nkb), dim3(kBlock), 0, s, C_len, pair_ptr,
                           C_starts, part, nkb, c_cap, st);
        hipLaunchKernelGGL(k_pair_fill, dim3((unsigned)nkb), dim3(kBlock), 0, s, n, C_off, c_cap,
                           A_len, A_starts, B_off, B_len, B_starts, b_ndiag, alk, pair_ptr, pairs,
                           pair_capacity, st);
        rc = check_launch(fn);
        if (rc) return rc;
        if (records) {
            rc = launch_astat_records(s, n, A_off, A_starts, a_ndiag, B_off, B_starts, b_ndiag,
                                      C_off, pair_ptr, c_cap, c_capacity, pairs, pair_capacity,
                                      &st->c_ndiag, &st->flags, records);
            if (rc) return rc;
        }
        rc = check_hip(hipMemcpyWithStream(&h, st, sizeof(h), hipMemcpyDeviceToHost, s), fn);
        if (rc) return rc;
        drain.armed = false;
        rec_flags = h.pad;
    }
    info->c_ndiag = h.c_ndiag;
    info->c_nnz = h.c_nnz;
    info->n_pairs = h.n_pairs;
    info->max_pairs = h.max_pairs;
    info->useful_flops = h.useful_flops;
    info->a_extent = h.a_extent;
    info->b_extent = h.b_extent;
    if (h.flags & (kFlagAOffset | kFlagBOffset))
        return fail(DIAGPU_ERR_OFFSET, "%s: an %s offset has |d| >= n=%d or length != n - |d|",
                    fn, (h.flags & kFlagAOffset) ? "A" : "B", n);
    if (h.flags & (kFlagADup | kFlagBDup))
        return fail(DIAGPU_ERR_DUPLICATE, "%s: repeated diagonal offset in %s", fn,
                    (h.flags & kFlagADup) ? "A" : "B");
    if (h.flags & kFlagCCapacity || h.c_ndiag > c_capacity)
        return fail(DIAGPU_ERR_CAPACITY, "%s: %lld C diagonals exceed c_capacity=%lld", fn,
                    (long long)h.c_ndiag, (long long)c_capacity);
    if (h.flags & kFlagPairCapacity || h.n_pairs > pair_capacity)
        return fail(DIAGPU_ERR_CAPACITY, "%s: %lld pairs exceed pair_capacity=%lld", fn,
                    (long long)h.n_pairs, (long long)pair_capacity);
    if (records) {
        *records_status =
            (rec_flags & 1) ? fail(DIAGPU_ERR_ARG,
                                   "%s: a plan entry is not in the symbolic plan's form", fn)
            : (rec_flags & 2) ? fail(DIAGPU_ERR_CAPACITY, "%s: B indices beyond 2^30 - 1", fn)
                              : DIAGPU_OK;
    }
    return DIAGPU_OK;
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spgemm_symbolic_workspace(int32_t n, int32_t a_ndiag, int32_t b_ndiag,
                                                size_t* bytes)
{
    using namespace diagpu;
    if (!bytes) return fail(DIAGPU_ERR_ARG, "diagpu_spgemm_symbolic_workspace: bytes is NULL");
    if (n < 1 || n > (1 << 30) || a_ndiag < 0 || b_ndiag < 0)
        return fail(DIAGPU_ERR_ARG,
                    "diagpu_spgemm_symbolic_workspace: need 1 <= n <= 2^30 and counts >= 0 "
                    "(n=%d a=%d b=%d)", n, a_ndiag, b_ndiag);
    *bytes = layout_for(n, a_ndiag, b_ndiag).total;
    return DIAGPU_OK;
}

DIAGPU_API int diagpu_spgemm_symbolic(
    int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup,
    void* workspace, size_t workspace_bytes,
    diagpu_spgemm_info* info, void* stream)
{
    return diagpu::run_symbolic("diagpu_spgemm_symbolic", n, A_off, A_len, A_starts, a_ndiag,
                                B_off, B_len, B_starts, b_ndiag, C_off, C_len, C_starts,
                                c_capacity, pair_ptr, pairs, pair_capacity, c_lookup, false,
                                workspace, workspace_bytes, nullptr, nullptr, info, stream);
}

DIAGPU_API int diagpu_spgemm_symbolic_astat(
    int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup,
    void* workspace, size_t workspace_bytes,
    int32_t* records, int32_t* records_status,
    diagpu_spgemm_info* info, void* stream)
{
    if (!records)
        return diagpu::fail(DIAGPU_ERR_ARG, "diagpu_spgemm_symbolic_astat: records is NULL");
    return diagpu::run_symbolic("diagpu_spgemm_symbolic_astat", n, A_off, A_len, A_starts,
                                a_ndiag, B_off, B_len, B_starts, b_ndiag, C_off, C_len, C_starts,
                                c_capacity, pair_ptr, pairs, pair_capacity, c_lookup, false,
                                workspace, workspace_bytes, records, records_status, info, stream);
}

DIAGPU_API int diagpu_spgemm_symbolic_noalloc(
    int32_t n,
    const int32_t* A_off, const int32_t* A_len, const int64_t* A_starts, int32_t a_ndiag,
    const int32_t* B_off, const int32_t* B_len, const int64_t* B_starts, int32_t b_ndiag,
    int32_t* C_off, int32_t* C_len, int64_t* C_starts, int64_t c_capacity,
    int64_t* pair_ptr, diagpu_gpair* pairs, int64_t pair_capacity,
    int32_t* c_lookup, diagpu_spgemm_info* info, void* stream)
{
    return diagpu::run_symbolic("diagpu_spgemm_symbolic_noalloc", n, A_off, A_len, A_starts,
                                a_ndiag, B_off, B_len, B_starts, b_ndiag, C_off, C_len, C_starts,
                                c_capacity, pair_ptr, pairs, pair_capacity, c_lookup, true,
                                nullptr, 0, nullptr, nullptr, info, stream);
}

}  // extern "C"
