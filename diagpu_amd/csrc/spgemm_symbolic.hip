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
// result does not depend on scheduling):
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
// then one 64-byte device-to-host copy of the counts and a stream sync.
#include <climits>
#include <mutex>

#include "common.hpp"
#include "scan.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;

enum : int32_t {
    kFlagAOffset = 1,
    kFlagBOffset = 2,
    kFlagADup = 4,
    kFlagBDup = 8,
    kFlagCCapacity = 16,
    kFlagPairCapacity = 32,
};

struct SymState {
    int64_t c_ndiag;
    int64_t c_nnz;
    int64_t n_pairs;
    int64_t max_pairs;
    int64_t useful_flops;
    int32_t flags;
    int32_t pad;
    int64_t reserved[2];
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
    L.off_state = o;   o = align256(o + sizeof(SymState));
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
    }
}

__global__ __launch_bounds__(kBlock) void k_operands(int32_t n, const int32_t* __restrict__ A_off,
                                                     const int32_t* __restrict__ A_len, int32_t na,
                                                     const int32_t* __restrict__ B_off,
                                                     const int32_t* __restrict__ B_len, int32_t nb,
                                                     int32_t* __restrict__ alk,
                                                     uint32_t* __restrict__ bbits,
                                                     SymState* __restrict__ st)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < na) {
        const int d = A_off[t];
        if (d <= -n || d >= n || A_len[t] != n - iabs_(d)) {
            raise_flag(st, kFlagAOffset);
        } else if (atomicExch(&alk[d + (n - 1)], t) != -1) {
            raise_flag(st, kFlagADup);
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
    diagpu_spgemm_info* info, void* stream)
{
    if (!info) return fail(DIAGPU_ERR_ARG, "%s: info is NULL", fn);
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
    if (use_scratch) {
        if (L.total > kScratchBytes)
            return fail(DIAGPU_ERR_CAPACITY,
                        "%s: n=%d with %d x %d diagonals needs %zu bytes of scratch, more than "
                        "the %zu the library holds (use diagpu_spgemm_symbolic with a workspace)",
                        fn, n, a_ndiag, b_ndiag, L.total, kScratchBytes);
        const int rc = scratch_ptr(fn, &workspace);
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
    const int64_t c_cap = c_capacity < L.cmax ? c_capacity : L.cmax;
    const int64_t nkb = ceil_div<int64_t>(c_cap + 1, kBlock);

    hipLaunchKernelGGL(k_init, dim3(grid_for(L.nlk, 4096)), dim3(kBlock), 0, s, alk, L.nlk, bbits,
                       cbits, L.nwords, st);
    hipLaunchKernelGGL(k_operands, dim3(grid_for(a_ndiag > b_ndiag ? a_ndiag : b_ndiag)),
                       dim3(kBlock), 0, s, n, A_off, A_len, a_ndiag, B_off, B_len, b_ndiag, alk,
                       bbits, st);
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
    int rc = check_launch(fn);
    if (rc) return rc;
    SymState h;
    rc = check_hip(hipMemcpyAsync(&h, st, sizeof(h), hipMemcpyDeviceToHost, s), fn);
    if (rc) return rc;
    rc = check_hip(hipStreamSynchronize(s), fn);
    if (rc) return rc;
    info->c_ndiag = h.c_ndiag;
    info->c_nnz = h.c_nnz;
    info->n_pairs = h.n_pairs;
    info->max_pairs = h.max_pairs;
    info->useful_flops = h.useful_flops;
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
                                workspace, workspace_bytes, info, stream);
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
                                nullptr, 0, info, stream);
}

}  // extern "C"
