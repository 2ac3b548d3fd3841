// DIA x DIA SpGEMM numeric phase with A held in LDS ("A-stationary"), for
// products whose A diagonals each feed many plan entries but whose B window
// is too wide for the band kernel -- e.g. the square of a 64-diagonal band
// spread over +-512 (4096 entries over 64 A diagonals: each A run is used by
// 64 C diagonals).  The gather kernel (spgemm_numeric.hip) reads both
// operand runs of every entry from L2; here a workgroup stages, for a block
// of kRB rows i and the kLead rows before it,
//   A(i, i + da)        for every A diagonal           nA x kStage values
// with direct global-to-LDS loads, then evaluates every C diagonal of the
// block: the A operand of each term comes from LDS and only the B operand
// from memory, which halves the L2 -> CU operand stream.
//
//   C(i, i + dc) = sum over the plan entries (da, db) of dc
//                  A(i, i + da) * B(i + da, i + dc)
//
// Entries are taken in plan order (spmspm/gather_flat.cuh:231-255) with one
// fused multiply-add each, and a term is skipped where either operand lacks
// the element: the gather kernel's exact sequence of roundings, so both
// kernels return the same bits.
//
// Per C diagonal the rows a wave evaluates start s rows before the block,
// s = (C start + min(dc, 0)) mod kLead, kLead = the elements of a 128-byte
// line: the block's C values then start on a line, so no line is written in
// two parts by two workgroups (a read-modify-write in HBM).  The kLead rows
// staged before the block cover that shift.  The rows the shift leaves after
// the last block (at most kLead - 1 per diagonal) are covered in one of two
// layouts chosen per launch: ceil((n + kLead) / kRB) blocks, the last
// covering them, or ceil(n / kRB) blocks, the last taking the rows
// [i0 + kRB - s, n) as one more row per lane (its staged window holds them,
// since n <= i0 + kRB).
//
// A workgroup has W = kWaves waves, or one per C diagonal for plans of
// fewer; wave w evaluates C diagonals w, w + W, ... over the block's kRB =
// 64 R rows, R rows per lane (lane l: rows l, l + 64, ..., l + 64 (R - 1)
// of the shifted window; R + 1 in the longer last block), R = 2, 4, 8 or 16
// chosen per launch from the plan's shape and occupancy (launch_astat).  The plan entries come as records
// {a, lo, hi, b} (diagpu_spgemm_astat_prepare): a the A diagonal's index,
// [lo, hi) the C positions where both operands hold an element, b the B
// index of C position 0.  Each term's B load is clamped into [lo, hi) and
// its multiply-add kept by a select, except on a C diagonal whose rows in
// the block lie inside the matrix for every A offset (tested once per
// diagonal from A's smallest and largest offset, which the prepare step
// stores after the records): there every entry takes every term, with no
// clamp and no select.
#include <algorithm>
#include <atomic>
#include <climits>
#include <type_traits>

#include "common.hpp"
#include "elem.hpp"
#include "spgemm_internal.hpp"

namespace diagpu {
namespace {

constexpr int kWaves = 16;                // waves per workgroup
constexpr int kForceR = 0;                // rows per lane forced (0: chosen per launch)
constexpr int kPrefetchDiagsPerWave = 4;  // C diagonals per wave from which the metadata is prefetched

// Per element type T (fp32 or complex fp32) and R rows per lane: blocks of
// kRB = 64 R rows, kLead rows staged before the block (one 128-byte line of
// C), kStage staged rows per A diagonal, kMax A diagonals in 160 KiB of LDS
// and kMax2 in 80 KiB (two workgroups per CU).
template <typename T, int R = 4> struct Astat {
    static constexpr int kRB = 64 * R;
    static constexpr int kLead = (int)(128 / sizeof(T));
    static constexpr int kStage = kRB + kLead;
    static constexpr int kWords = (int)(sizeof(T) / 4);   // dwords per element
    static constexpr int kMax = (160 * 1024) / (kStage * (int)sizeof(T));
    static constexpr int kMax2 = (80 * 1024) / (kStage * (int)sizeof(T));
};
// The A-diagonal capacity: fp32 at 4 rows per lane; complex at 2, the
// blocks that take more than 4 rows' worth of complex A diagonals.
template <typename T> constexpr int astat_cap()
{
    return sizeof(T) == 4 ? Astat<T, 4>::kMax : Astat<T, 2>::kMax;
}
static_assert(astat_cap<float>() == DIAGPU_ASTAT_MAX_A, "fp32 A diagonals in 160 KiB of LDS");
static_assert(astat_cap<cf32>() == DIAGPU_ASTAT_MAX_A_C64, "complex A diagonals in 160 KiB of LDS");

// records[g] = {a, lo, hi, b} for plan entry g; flag[0] set if an entry is
// not in the symbolic plan's form (its A or B start is no diagonal's start,
// da + db is not its C diagonal's offset, or its shifts or lengths differ
// from min0(da) - min0(dc), da + min0(db) - min0(dc), n - |da|, n - |db|) or
// pair_ptr is not a partition of the entries, flag[1] if its B indices
// reach 2^30 (the numeric kernel forms their byte offsets in 32 bits).  The
// kernel builds each A row from A_off and C_off but takes each term's range
// from the record, so an entry of another form would give a different C
// without an error.
//
// One thread per C diagonal k walks its entries [pair_ptr[k], pair_ptr[k +
// 1]), so no entry searches pair_ptr; each entry's A and B diagonals are
// found by their starts, in tables staged in LDS when both fit (kPrepTable
// diagonals each), else in global memory.
constexpr int kPrepBlock = 256;
constexpr int kPrepTable = 1024;

__device__ __forceinline__ int find_start(const int64_t* s, int32_t cnt, int64_t v)
{
    // binary search (diagonals stored in offset order: starts ascend), then a
    // linear scan for operands stored in another order
    int lo = 0, hi = cnt - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s[mid] <= v) lo = mid; else hi = mid - 1;
    }
    if (s[lo] == v) return lo;
    for (int i = 0; i < cnt; ++i)
        if (s[i] == v) return i;
    return -1;
}

// A's and B's starts and offsets, staged in LDS by every workgroup of a
// prepare kernel when both fit (kPrepTable diagonals each).
struct PrepTables {
    int64_t sa[kPrepTable], sb[kPrepTable];
    int32_t oa[kPrepTable], ob[kPrepTable];
};

// Stages the tables (every lane of the workgroup calls it); true if staged.
__device__ __forceinline__ bool stage_tables(PrepTables& t, const int32_t* __restrict__ A_off,
                                             const int64_t* __restrict__ A_starts, int32_t nA,
                                             const int32_t* __restrict__ B_off,
                                             const int64_t* __restrict__ B_starts, int32_t nB)
{
    const bool staged = nA <= kPrepTable && nB <= kPrepTable;
    if (staged) {
        for (int i = (int)threadIdx.x; i < nA; i += kPrepBlock) {
            t.sa[i] = A_starts[i];
            t.oa[i] = A_off[i];
        }
        for (int i = (int)threadIdx.x; i < nB; i += kPrepBlock) {
            t.sb[i] = B_starts[i];
            t.ob[i] = B_off[i];
        }
        __syncthreads();
    }
    return staged;
}

// The records of C diagonal k's entries [pair_ptr[k], pair_ptr[k + 1]) of a
// plan with c_ndiag diagonals and n_pairs entries; raise(1) for an entry not
// in the symbolic form or a pair_ptr that is no partition, raise(2) for a B
// index beyond 2^30 - 1.
template <typename Raise>
__device__ __forceinline__ void prepare_diag(
    int64_t k, int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts,
    int32_t nA, const int32_t* __restrict__ B_off, const int64_t* __restrict__ B_starts, int32_t nB,
    const int32_t* __restrict__ C_off, const int64_t* __restrict__ pair_ptr, int64_t c_ndiag,
    const diagpu_gpair* __restrict__ pairs, int64_t n_pairs, int4* __restrict__ records,
    const PrepTables& t, bool staged, Raise raise)
{
    const int64_t g0 = pair_ptr[k], g1 = pair_ptr[k + 1];
    if (g0 < 0 || g1 < g0 || g1 > n_pairs || (k == 0 && g0 != 0) ||
        (k == c_ndiag - 1 && g1 != n_pairs)) {
        raise(1);
        return;
    }
    const int64_t dc = C_off[k];
    auto min0 = [](int64_t x) { return x < 0 ? x : (int64_t)0; };
    auto absl = [](int64_t x) { return x < 0 ? -x : x; };
    for (int64_t g = g0; g < g1; ++g) {
        const diagpu_gpair p = pairs[g];
        const int a = find_start(staged ? t.sa : A_starts, nA, (int64_t)p.ab);
        const int bi = find_start(staged ? t.sb : B_starts, nB, (int64_t)p.bb);
        bool ok = a >= 0 && bi >= 0;
        if (ok) {
            const int64_t da = staged ? t.oa[a] : A_off[a], db = staged ? t.ob[bi] : B_off[bi];
            ok = da + db == dc && dc > -(int64_t)n && dc < n &&
                 (int64_t)p.ash == min0(da) - min0(dc) &&
                 (int64_t)p.bsh == da + min0(db) - min0(dc) && (int64_t)p.al == n - absl(da) &&
                 (int64_t)p.bl == n - absl(db);
        }
        const int plo = max(0, max(-p.ash, -p.bsh));
        const int phi = min(p.al - p.ash, p.bl - p.bsh);
        const int64_t b = (int64_t)p.bb + p.bsh;
        int4 r = int4{0, 0, 0, 0};
        if (!ok) {
            raise(1);
        } else if (plo >= phi) {
            // No position holds both operands (an entry of the symbolic form
            // always has one; kept so that no record can read past B): a
            // record that never fires, whose clamped B load
            // min(max(p, 1), 0) = 0 reads B[0].
            r = int4{a, 1, 1, 0};
        } else if (b < INT_MIN || b + phi > ((int64_t)1 << 30)) {
            raise(2);   // the kernel forms 4 (b + c) in 32 bits
        } else {
            r = int4{a, plo, phi, (int)b};
        }
        records[g] = r;
    }
}

__global__ __launch_bounds__(kPrepBlock) void k_astat_prepare(
    int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts, int32_t nA,
    const int32_t* __restrict__ B_off, const int64_t* __restrict__ B_starts, int32_t nB,
    const int32_t* __restrict__ C_off, const int64_t* __restrict__ pair_ptr, int64_t c_ndiag,
    const diagpu_gpair* __restrict__ pairs, int64_t n_pairs, int4* __restrict__ records,
    int32_t* __restrict__ flag)
{
    __shared__ PrepTables t;
    const bool staged = stage_tables(t, A_off, A_starts, nA, B_off, B_starts, nB);
    const int64_t k = (int64_t)blockIdx.x * kPrepBlock + threadIdx.x;
    if (k >= c_ndiag) return;
    // every writer of a flag stores the same value
    prepare_diag(k, n, A_off, A_starts, nA, B_off, B_starts, nB, C_off, pair_ptr, c_ndiag, pairs,
                 n_pairs, records, t, staged, [&](int bit) { flag[bit - 1] = 1; });
}

// The same records built inside the symbolic call
// (diagpu_spgemm_symbolic_astat) when it takes the multi-launch path (the
// one-launch kernel writes them with the entries), queued behind that phase
// on its stream, so one read-back returns both.  The plan's counts come from
// the phase's state record on the device: state_counts[0] C diagonals,
// state_counts[2] entries (each bounded by its capacity).  Nothing runs when
// the phase raised a flag (state_flags[0]: its plan is incomplete).  Errors
// are ORed into state_flags[1] (zeroed by the symbolic phase): 1 an entry not
// in the symbolic form, 2 a B index beyond 2^30 - 1.
// Workgroup 0 also writes the 4 ints after the records, {0, 0, smallest,
// largest A offset}.
__global__ __launch_bounds__(kPrepBlock) void k_astat_records(
    int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts, int32_t nA,
    const int32_t* __restrict__ B_off, const int64_t* __restrict__ B_starts, int32_t nB,
    const int32_t* __restrict__ C_off, const int64_t* __restrict__ pair_ptr, int64_t c_cap,
    const diagpu_gpair* __restrict__ pairs, int64_t p_cap, const int64_t* state_counts,
    int32_t* state_flags, int32_t* __restrict__ records)
{
    if (state_flags[0]) return;
    const int64_t c_ndiag = min(state_counts[0], c_cap);
    const int64_t n_pairs = min(state_counts[2], p_cap);
    if (blockIdx.x == 0 && threadIdx.x < 64) {
        int lo = INT_MAX, hi = INT_MIN;
        for (int d = (int)threadIdx.x; d < nA; d += 64) {
            lo = min(lo, A_off[d]);
            hi = max(hi, A_off[d]);
        }
        for (int m = 32; m >= 1; m >>= 1) {
            lo = min(lo, __shfl_xor(lo, m));
            hi = max(hi, __shfl_xor(hi, m));
        }
        if (threadIdx.x == 0)
            reinterpret_cast<int4*>(records)[n_pairs] = int4{0, 0, lo, hi};
    }
    __shared__ PrepTables t;
    const bool staged = stage_tables(t, A_off, A_starts, nA, B_off, B_starts, nB);
    const int64_t k = (int64_t)blockIdx.x * kPrepBlock + threadIdx.x;
    if (k >= c_ndiag) return;
    prepare_diag(k, n, A_off, A_starts, nA, B_off, B_starts, nB, C_off, pair_ptr, c_ndiag, pairs,
                 n_pairs, reinterpret_cast<int4*>(records), t, staged,
                 [&](int bit) { atomicOr(state_flags + 1, bit); });
}

// flag[0..1] = 0 (the error flags above); flag[2..3] = the smallest and
// largest of A's offsets, which the numeric kernel reads.
__global__ __launch_bounds__(64) void k_astat_init(int32_t* __restrict__ flag,
                                                   const int32_t* __restrict__ A_off, int32_t nA)
{
    int lo = INT_MAX, hi = INT_MIN;
    for (int d = (int)threadIdx.x; d < nA; d += 64) {
        lo = min(lo, A_off[d]);
        hi = max(hi, A_off[d]);
    }
    for (int m = 32; m >= 1; m >>= 1) {
        lo = min(lo, __shfl_xor(lo, m));
        hi = max(hi, __shfl_xor(hi, m));
    }
    if (threadIdx.x < 2) flag[threadIdx.x] = 0;
    if (threadIdx.x == 0) {
        flag[2] = lo;
        flag[3] = hi;
    }
}

// Keeps a value in registers at this point: the compiler cannot sink its
// load into a branch past it.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(cf32& v) { asm volatile("" : "+v"(v.re), "+v"(v.im)); }

template <typename T>
__device__ __forceinline__ void store_elem_nt(T* p, T v)
{
    typedef typename ElemRaw<T>::type Raw;
    Raw r;
    __builtin_memcpy(&r, &v, sizeof(T));
    __builtin_nontemporal_store(r, reinterpret_cast<Raw*>(p));
}

// B element b + c, b the B index of the entry's C position 0 and c the C
// position (0 <= b + c < 2^30, the prepare step's bound on B indices).
// fp32: a buffer load through one descriptor over all of B (rB), with the
// byte offset 4 (b + c) formed in 32-bit arithmetic (exact, since it is
// below 2^32): an entry costs one scalar shift, not a descriptor of its own.
// Complex: a global load (this toolchain compiles the 64-bit raw buffer load
// builtin to a single-dword load).
__device__ __forceinline__ float load_b(const float*, __amdgpu_buffer_rsrc_t rB, int b, int c)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rB, ((uint32_t)c << 2) + ((uint32_t)b << 2), 0, 0));
}
__device__ __forceinline__ cf32 load_b(const cf32* B, __amdgpu_buffer_rsrc_t, int b, int c)
{
    return load_elem<cf32, false>(B + (int64_t)b + c);
}

// Stores a wave's RR values of one C diagonal cd[0, len): lane l holds
// positions pb + 64 j, those in [0, len) are written.  fp32: buffer stores
// that always issue, the descriptor spanning the diagonal (4 len bytes,
// below 2^32 for len < 2^30) and a lane outside [0, len) given an offset
// past it (dropped by the hardware): no branch around the stores (config 5
// 2.33 -> 2.25 ms against branched global stores).  Complex: branched global
// stores.
//
// The test 0 <= p < len takes one of two equivalent forms, which compile to
// different schedules of the whole diagonal loop: two signed compares
// (TwoCmp, the kernels of four-entry batches) or one unsigned compare.
// Measured in interleaved rounds on two boxes: config 3's square (four-entry
// batches) 7.04-7.07 / 6.67-6.88 ms with two compares against 7.43-7.49 /
// 7.24-7.27 with one; config 5, config 4, config 2's square and complex
// config 4 0.5-2 % faster with one.  Counters on config 3's square: with two
// compares the vector L1 hit rate is 78 % against 72 % and L2 read requests
// 427 M against 536 M per launch; why the schedule moves the hit rate is not
// established.
template <typename T, int RR, bool TwoCmp = false>
__device__ __forceinline__ void store_c(T* cd, int pb, int len, const T (&acc)[RR])
{
    if constexpr (sizeof(T) == 4) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            cd, (short)0, (int)((uint32_t)len * 4u), 0x00020000);
#pragma unroll
        for (int j = 0; j < RR; ++j) {
            const int p = pb + 64 * j;
            const bool in = TwoCmp ? (p >= 0 && p < len) : (uint32_t)p < (uint32_t)len;
            const uint32_t off = in ? (uint32_t)p << 2 : 0xFFFFFFFFu;
            // cache policy 2: non-temporal, as store_elem_nt
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc[j]), r, off, 0, 2);
        }
    } else {
#pragma unroll
        for (int j = 0; j < RR; ++j) {
            const int p = pb + 64 * j;
            if (p >= 0 && p < len) store_elem_nt(cd + p, acc[j]);
        }
    }
}

// Prefetch: each diagonal's metadata loaded while the one before it runs
// (for waves that walk many diagonals).  tail5: the last block also takes
// the rows the line-aligned shift leaves after it, R + 1 rows per lane (else
// one more block of at most kLead - 1 rows per diagonal covers them).
// Epi: C = (alpha A) B + sigma I -- the staged A rows are scaled in LDS
// (scale_, once per staged element, before any term reads them), so the
// terms are those of the plain kernel on the operand alpha A, and sigma is
// added to the main diagonal's sums before they are stored.
template <typename T, bool Prefetch, int R, bool Quad = false, bool Epi = false>
__global__ __launch_bounds__(64 * kWaves) void k_astat(
    int32_t n, const int32_t* __restrict__ A_off, const int64_t* __restrict__ A_starts, int32_t nA,
    const T* __restrict__ Av, const T* __restrict__ Bv, const int32_t* __restrict__ C_off,
    const int32_t* __restrict__ C_len, const int64_t* __restrict__ C_starts, int32_t nC,
    const int64_t* __restrict__ pair_ptr, const int4* __restrict__ records,
    const int32_t* __restrict__ aext, T* __restrict__ Cv, int32_t blocks, int32_t groups,
    int32_t per_xcd, int32_t tail5, T alpha, T sigma)
{
    // A's smallest and largest offset (written by diagpu_spgemm_astat_prepare
    // after the records)
    const int amin = aext[0], amax = aext[1];
    const __amdgpu_buffer_rsrc_t rB =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(Bv), (short)0, -1, 0x00020000);
    constexpr int kRB = Astat<T, R>::kRB, kLead = Astat<T, R>::kLead;
    constexpr int kStage = Astat<T, R>::kStage, kWords = Astat<T, R>::kWords;
    extern __shared__ float A_l[];   // [nA][kStage] elements: rows i0 - kLead .. i0 + kRB - 1
    const T* A_t = reinterpret_cast<const T*>(A_l);
    // workgroup b on XCD b mod 8: each XCD owns a contiguous range of work
    // units, so neighbouring blocks (whose B windows overlap) share its L2.
    // Unit = (block, group): a block's C diagonals are split over `groups`
    // workgroups (more than one only when the blocks alone cannot fill the
    // GPU), each staging the block's A rows.
    const int unit = (int)(blockIdx.x % kNumXcd) * per_xcd + (int)(blockIdx.x / kNumXcd);
    if (unit >= blocks * groups) return;
    // with tail5 the last block (R + 1 rows per lane) goes first: dispatched
    // with the first wave of workgroups, its longer work overlaps the others'
    const int blk = tail5 ? (unit / groups + blocks - 1) % blocks : unit / groups;
    const int grp = unit % groups;
    const int r = (int)threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(r >> 6), lane = r & 63;
    const int nw = (int)(blockDim.x >> 6);          // waves in this workgroup
    const int i0 = blk * kRB;                       // n < 2^30: rows fit int32

    // Stage A: one wave-instruction per 64 dwords of a diagonal's window
    // (kWords dwords per element), each lane's HM position clamped into the
    // diagonal (the address is always valid; a staged element that does not
    // exist is never used: its terms are outside [lo, hi)).
    const float* Aw = reinterpret_cast<const float*>(Av);
    for (int d = wave; d < nA; d += nw) {
        const int o = A_off[d];
        const int64_t st = A_starts[d];
        const int len = n - (o < 0 ? -o : o);
        for (int q0 = 0; q0 < kStage * kWords; q0 += 64) {
            const int f = q0 + lane;                // dword of the window
            if (f < kStage * kWords) {
                const int w = i0 - kLead + f / kWords;
                const int pos = min(max(w + (o < 0 ? o : 0), 0), len - 1);
                __builtin_amdgcn_global_load_lds(Aw + (st + pos) * kWords + f % kWords,
                                                 A_l + d * kStage * kWords + q0, 4, 0, 0);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // this wave's direct loads have landed in LDS
    __syncthreads();
    if constexpr (Epi) {
        T* A_s = reinterpret_cast<T*>(A_l);
        for (int e = r; e < nA * kStage; e += 64 * nw) A_s[e] = scale_(alpha, A_s[e]);
        __syncthreads();
    }

    // RR rows per lane: R, and with tail5 R + 1 in the last block, whose
    // staged window also holds the rows [i0 + kRB - s, n) that no later block
    // covers (n <= i0 + kRB there).
    auto run = [&](auto rows) {
        constexpr int RR = decltype(rows)::value;
        // With Prefetch, a diagonal's metadata is loaded while the diagonal
        // before it runs (index clamped rather than tested: a load under a
        // branch is waited for where the branch joins).
        const int stride = groups * nw;
        int kc = grp * nw + wave;
        if (kc >= nC) return;
        // The metadata of diagonal k sits at byte offsets 4 k (C_off, C_len)
        // and 8 k (C_starts, pair_ptr), below 2^32 for nC < 2^29.
        int dcn = at_byte(C_off, (uint32_t)kc << 2), lenn = at_byte(C_len, (uint32_t)kc << 2);
        int64_t cstn = at_byte(C_starts, (uint32_t)kc << 3), g0n = at_byte(pair_ptr, (uint32_t)kc << 3),
                g1n = at_byte(pair_ptr + 1, (uint32_t)kc << 3);
        // The block-wide part of the every-term test below: whatever a
        // diagonal's shift s (0 <= s < kLead), its rows [i0 - s, i0 - s + 64
        // RR) lie in [i0 - kLead + 1, i0 + 64 RR), inside the matrix for
        // every A offset when blk_in holds; they then meet 0 <= i + dc < n
        // for dc - dlo in [0, dspan] (dlo = kLead - 1 - i0, dspan = n - 64 RR
        // - kLead + 1, which is >= 0 where blk_in holds).
        const bool blk_in = i0 >= kLead - 1 - min(amin, 0) && n - i0 - 64 * RR >= max(amax, 0);
        const int dlo = kLead - 1 - i0;
        const uint32_t dspan = (uint32_t)(n - 64 * RR - kLead + 1);
        for (; kc < nC; kc += stride) {
            int dc, len, g0, g1;
            int64_t cst;
            if constexpr (Prefetch) {
                dc = dcn;
                len = lenn;
                cst = cstn;
                g0 = (int)g0n;
                g1 = (int)g1n;
                const uint32_t kn = (uint32_t)min(kc + stride, nC - 1);
                dcn = at_byte(C_off, kn << 2);
                lenn = at_byte(C_len, kn << 2);
                cstn = at_byte(C_starts, kn << 3);
                g0n = at_byte(pair_ptr, kn << 3);
                g1n = at_byte(pair_ptr + 1, kn << 3);
            } else {
                dc = at_byte(C_off, (uint32_t)kc << 2);
                len = at_byte(C_len, (uint32_t)kc << 2);
                cst = at_byte(C_starts, (uint32_t)kc << 3);
                g0 = (int)at_byte(pair_ptr, (uint32_t)kc << 3);
                g1 = (int)at_byte(pair_ptr + 1, (uint32_t)kc << 3);
            }
            const int mc = dc < 0 ? dc : 0;
            // C(i0 - s, ...) starts a line (the low bits of the start suffice)
            const int s = ((int)(uint32_t)cst + mc) & (kLead - 1);
            const int pb = i0 - s + lane + mc;          // C position of the lane's first row
            const int ab = kLead - s + lane;            // its staged A row
            T acc[RR];
#pragma unroll
            for (int j = 0; j < RR; ++j) acc[j] = zero_of<T>();
            // A element of entry a at the lane's row j: staged row ab + 64 j
            // (row R of a lane past the window, p >= len there, reads row 0),
            // addressed as the lane's byte offset plus the entry's (one add
            // per entry, the rows' 256 j bytes an instruction offset)
            const char* A_c = reinterpret_cast<const char*>(A_t);
            const int abx = ab * (int)sizeof(T);
            auto a_at = [&](int a, int j) -> T {
                const int rb = j < R || lane < s ? abx + 64 * j * (int)sizeof(T) : abx;
                return *reinterpret_cast<const T*>(A_c + (a * kStage * (int)sizeof(T) + rb));
            };
            // one term: B at the position clamped into the entry's range
            // [e.y, e.z) (an always valid load: 0 <= c < n), A from LDS, the
            // multiply-add kept where the clamp leaves the position as it is
            // and the range is not empty: where both operands hold the element
            // (positions p >= len take terms too, but are never stored)
            auto term = [&](const int4& e, int j, T& b, T& a, bool& ok) {
                const int p = pb + 64 * j;
                const int c = min(max(p, e.y), e.z - 1);
                ok = c == p && e.y < e.z;
                b = load_b(Bv, rB, e.w, c);
                a = a_at(e.x, j);
            };
            // Every entry of this diagonal takes every term of the wave's
            // rows [r0, r0 + 64 RR), r0 = i0 - s, where each row i has
            // 0 <= i, i + da, i + dc < n for all of A's offsets da (the
            // rows where an entry's A and B elements and C's exist; tested
            // by blk_in and the bounds on dc above, which hold for any s
            // and so miss at most the kLead - 1 rows at an edge): then
            // the B loads need no clamp and the multiply-adds no select,
            // about a fifth of the vector instructions of the general form,
            // with the same multiply-adds in the same order.  Measured
            // against the general form alone: make_banded(100000, 16) squared
            // 34.7 -> 28.2 us, config 3's square 7.62 -> 7.43 ms, config 5
            // 2.28 -> 2.23 ms (fp32, 4 rows per lane); at 16 rows per lane
            // config 1's square 15.4 -> 14.8 us and config 4 42.5 -> 42.05
            // us, at 8 the Taylor chain's products 1.83 -> 1.81 ms, complex
            // config 5 5.95 -> 5.85 ms.  (Before the scalar loads at byte
            // offsets the path lost 2-3 % at 8 rows per lane and 1 % for
            // complex values.)
            const bool inner = blk_in && (uint32_t)(dc - dlo) <= dspan;
            // A batch of NU entries: their loads issued together, then the
            // multiply-adds in plan order.  The values are pinned once all
            // loads are issued, so the compiler cannot turn a masked
            // multiply-add into a branch around its own load (each such
            // branch ends in a full vmcnt(0) drain: gfx9 counts loads in
            // order).
            auto batch = [&](auto nu, auto every, int g) {
                constexpr int NU = decltype(nu)::value;
                constexpr bool kEvery = decltype(every)::value;
                T bv[NU][RR], av[NU][RR];
                bool ok[NU][RR];
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    // byte offset 16 g (below 2^32 for n_pairs < 2^28) from
                    // records + u: u's 16 bytes an immediate offset, so the
                    // batch's loads merge into one
                    const int4 e = at_byte(records + u, (uint32_t)g << 4);
#pragma unroll
                    for (int j = 0; j < RR; ++j) {
                        if constexpr (kEvery) {
                            bv[u][j] = load_b(Bv, rB, e.w, pb + 64 * j);
                            av[u][j] = a_at(e.x, j);
                        } else {
                            term(e, j, bv[u][j], av[u][j], ok[u][j]);
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < NU; ++u)
#pragma unroll
                    for (int j = 0; j < RR; ++j) { pin(bv[u][j]); pin(av[u][j]); }
#pragma unroll
                for (int u = 0; u < NU; ++u)
#pragma unroll
                    for (int j = 0; j < RR; ++j) {
                        if constexpr (kEvery)
                            acc[j] = mad(acc[j], av[u][j], bv[u][j]);
                        else
                            acc[j] = sel(ok[u][j], mad(acc[j], av[u][j], bv[u][j]), acc[j]);
                    }
            };
            // two entries' loads in flight, or one where two would hold more
            // than 8 dwords per lane per entry (within 64 VGPRs: two 16-wave
            // workgroups per CU); with Quad, four in the every-term form
            auto walk = [&](auto every) {
                int g = g0;
                if constexpr (Quad && decltype(every)::value && RR * kWords <= 4)
                    for (; g + 4 <= g1; g += 4) batch(std::integral_constant<int, 4>{}, every, g);
                if constexpr (RR * kWords <= 8)
                    for (; g + 2 <= g1; g += 2) batch(std::integral_constant<int, 2>{}, every, g);
                for (; g < g1; ++g) batch(std::integral_constant<int, 1>{}, every, g);
            };
            if (inner)
                walk(std::true_type{});
            else
                walk(std::false_type{});
            if constexpr (Epi) {
                if (dc == 0)
#pragma unroll
                    for (int j = 0; j < RR; ++j) acc[j] = add_(acc[j], sigma);
            }
            store_c<T, RR, Quad>(Cv + cst, pb, len, acc);
        }
    };
    if (tail5 && blk == blocks - 1)
        run(std::integral_constant<int, R + 1>{});
    else
        run(std::integral_constant<int, R>{});
}

// Workgroups of W waves of k_astat<T, *, R> that fit a CU by registers (its
// LDS aside), looked up once per instantiation and W: the 16-wave
// workgroups fit twice at up to 64 VGPRs, once above.
template <typename T, int R> int wgs_by_regs(int W)
{
    static std::atomic<int> cache[kWaves + 1];
    int v = cache[W].load(std::memory_order_relaxed);
    if (v) return v;
    int a = 0, b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, (const void*)k_astat<T, false, R>,
                                                    64 * W, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, (const void*)k_astat<T, true, R>,
                                                    64 * W, 0) != hipSuccess)
        v = 1;
    else
        v = std::max(1, std::min(a, b));
    cache[W].store(v, std::memory_order_relaxed);
    return v;
}

// Workgroup slots of k_astat<T, *, R> on the GPU for nA A diagonals: by
// registers and by the LDS the staged A rows take (160 KiB per CU).
template <typename T, int R> int64_t astat_slots(int32_t nA, int W = kWaves)
{
    const int64_t lds = (int64_t)nA * Astat<T, R>::kStage * (int64_t)sizeof(T);
    const int64_t by_lds = std::max<int64_t>(1, (160 * 1024) / lds);
    return std::min<int64_t>(wgs_by_regs<T, R>(W), by_lds) * (int64_t)cu_count();
}

// Waves per workgroup: kWaves, or one per C diagonal where there are fewer
// (a wave evaluates whole C diagonals, so the others would idle while
// holding the CU's registers): more, smaller workgroups share a CU.
// Measured (interleaved rounds, same bits): config 1's square (5 C
// diagonals) 14.6 -> 11.9 us; config 2's square (13) level.  Spreading
// more diagonals evenly over fewer waves (41 over 3 x 14 for gemm_diag at
// n = 4096) was 5 % slower, so from kWaves diagonals the workgroups keep
// kWaves waves.
inline int waves_for(int64_t c_ndiag)
{
    return c_ndiag < kWaves ? (int)std::max<int64_t>(1, c_ndiag) : kWaves;
}

// One launch of k_astat<T, *, R> (arguments checked by the caller).
template <typename T, int R>
int launch_rows(const char* fn, int32_t n, const int32_t* A_off, const int64_t* A_starts,
                int32_t nA, const T* A_vals, const T* B_vals, const int32_t* C_off,
                const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
                const int64_t* pair_ptr, const int32_t* records, int64_t n_pairs, T* C_vals,
                void* stream, bool epi, T alpha, T sigma)
{
    constexpr int kRB = Astat<T, R>::kRB, kLead = Astat<T, R>::kLead, kStage = Astat<T, R>::kStage;
    constexpr int kMax = Astat<T, R>::kMax;
    const size_t lds = (size_t)nA * kStage * sizeof(T);
    // Row blocks and their split: too few blocks to give every CU its
    // workgroups split each block's C diagonals over several workgroups (at
    // most one per wave's worth of diagonals).
    const int W = waves_for(c_ndiag);
    const int64_t slots = astat_slots<T, R>(nA, W);
    // fp32 launches of 4 rows per lane and fewer than 16 rounds of
    // workgroups also split each block, over G = 2 or 4 workgroups, towards
    // 16 rounds (while every wave keeps at least kPrefetchDiagsPerWave C
    // diagonals).  Measured on random 64..142 x 16..128 products over
    // +-512..+-8192 at n = 2^18..2^20 (forced, one buffer set): 4 -> 16
    // rounds 4-8% faster (config 5: 2.49 -> 2.34 ms under the bench's
    // rotation), 8 -> 16 rounds 3%, at 16 rounds no split gained more than
    // noise but one (128 x 16 at 2^20, 6%).  Lost with it: complex values
    // (config 5 complex, 8 rounds: 6.13 -> 6.28 ms at G = 2) and the 8 rows
    // per lane of the Taylor chain's products (numeric 1.96 -> 2.05 ms).
    int64_t G = 1;
    if constexpr (sizeof(T) == 4 && R == 4) {
        const int64_t r0 = ceil_div<int64_t>(ceil_div<int64_t>((int64_t)n + kLead, kRB), slots);
        while (G < 4 && r0 * G < 16 && c_ndiag >= 2 * G * kPrefetchDiagsPerWave * kWaves) G *= 2;
    }
    auto split = [&](int64_t blocks) {
        if (blocks >= slots) return G;
        return std::max<int64_t>(G, std::min<int64_t>(ceil_div<int64_t>(slots, blocks),
                                                      ceil_div<int64_t>(c_ndiag, W)));
    };
    // ceil((n + kLead) / kRB) blocks of R rows per lane, the last covering
    // the rows the line-aligned shift leaves (at most kLead - 1 per
    // diagonal); or ceil(n / kRB), the last block taking those rows as one
    // more per lane, where that saves one of at most 8 G rounds of
    // workgroups on the GPU (config 5 unsplit: 1025 blocks on 256 CUs take 5
    // rounds, 1024 take 4).  A workgroup's time is set by its waves' chains
    // of loads per diagonal, not by its rows, so the short block can cost a
    // full round; over more rounds the saving shrinks below the longer
    // block's own cost (the 7-point stencil's square, 4097 blocks in 9
    // rounds: 1 us slower).
    int64_t blocks = ceil_div<int64_t>((int64_t)n + kLead, kRB), groups = split(blocks);
    int32_t tail5 = 0;
    const int64_t b5 = ceil_div<int64_t>(n, kRB), g5 = split(b5);
    const int64_t rounds = ceil_div<int64_t>(blocks * groups, slots);
    if (b5 < blocks && ceil_div<int64_t>(b5 * g5, slots) < rounds && rounds <= 8 * G) {
        blocks = b5;
        groups = g5;
        tail5 = 1;
    }
    const int32_t per_xcd = (int32_t)ceil_div<int64_t>(blocks * groups, kNumXcd);
    // the metadata prefetch pays where waves walk many diagonals (config 5:
    // ~575 each) and costs where they walk one or two (the 7-point stencil's
    // square: 25 C diagonals over 16 waves, 31 -> 34 us)
    const bool prefetch = c_ndiag >= kPrefetchDiagsPerWave * groups * W;
    // Quad (fp32, 4 rows per lane): batches of four entries in the
    // every-term form, for plans of >= 3 entries per C diagonal on average
    // (make_banded(100000, 16) squared 27.9 -> 26.3 us, config 3's square
    // 7.45 -> 7.33 ms; config 5, 1.8 entries per C diagonal, lost 1 %)
    const bool quad = n_pairs >= 3 * c_ndiag;
    const dim3 grid((unsigned)(per_xcd * kNumXcd)), block(64 * W);
    const int4* rec = reinterpret_cast<const int4*>(records);
    const int32_t* aext = records + 4 * n_pairs + 2;
    auto go3 = [&](auto pf, auto qd, auto ep) {
        constexpr bool kPf = decltype(pf)::value, kQd = decltype(qd)::value;
        constexpr bool kEp = decltype(ep)::value;
        // more than 64 KiB of dynamic LDS must be allowed explicitly
        const int st = check_hip(
            hipFuncSetAttribute((const void*)k_astat<T, kPf, R, kQd, kEp>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                kStage * kMax * (int)sizeof(T)),
            fn);
        if (st) return st;
        hipLaunchKernelGGL((k_astat<T, kPf, R, kQd, kEp>), grid, block, lds, as_stream(stream), n,
                           A_off, A_starts, nA, A_vals, B_vals, C_off, C_len, C_starts,
                           (int32_t)c_ndiag, pair_ptr, rec, aext, C_vals, (int32_t)blocks,
                           (int32_t)groups, per_xcd, tail5, alpha, sigma);
        return check_launch(fn);
    };
    using yes = std::true_type;
    using no = std::false_type;
    auto go = [&](auto pf, auto qd) { return epi ? go3(pf, qd, yes{}) : go3(pf, qd, no{}); };
    if constexpr (sizeof(T) == 4 && R == 4) {
        if (quad) return prefetch ? go(yes{}, yes{}) : go(no{}, yes{});
    }
    return prefetch ? go(yes{}, no{}) : go(no{}, no{});
}

template <typename T>
int launch_astat(const char* fn, int32_t n, const int32_t* A_off, const int64_t* A_starts,
                 int32_t nA, const T* A_vals, const T* B_vals, const int32_t* C_off,
                 const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
                 const int64_t* pair_ptr, const int32_t* records, int64_t n_pairs, T* C_vals,
                 void* stream, bool epi = false, T alpha = T{}, T sigma = T{})
{
    constexpr int kMax = astat_cap<T>();
    // the kernel addresses metadata and records by 32-bit byte offsets
    if (n < 1 || n >= (1 << 30) || nA < 1 || c_ndiag < 0 || c_ndiag > 2 * (int64_t)n - 1 ||
        c_ndiag >= (1 << 29) || n_pairs < 0 || n_pairs >= (1 << 28))
        return fail(DIAGPU_ERR_ARG,
                    "%s: bad sizes (n=%d nA=%d c_ndiag=%lld n_pairs=%lld; n < 2^30, c_ndiag < "
                    "2^29 and n_pairs < 2^28 here)", fn, n, nA, (long long)c_ndiag,
                    (long long)n_pairs);
    if (nA > kMax)
        return fail(DIAGPU_ERR_CAPACITY, "%s: %d A diagonals, at most %d fit in LDS", fn, nA, kMax);
    if (c_ndiag == 0) return DIAGPU_OK;
    if (!A_off || !A_starts || !A_vals || !B_vals || !C_off || !C_len || !C_starts || !pair_ptr ||
        !records || !C_vals)
        return fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
#define DIAGPU_ASTAT_LAUNCH(RV)                                                                   \
    launch_rows<T, RV>(fn, n, A_off, A_starts, nA, A_vals, B_vals, C_off, C_len, C_starts, c_ndiag, \
                       pair_ptr, records, n_pairs, C_vals, stream, epi, alpha, sigma)
    // Rows per lane.  A wave's time per C diagonal is a chain of dependent
    // loads; longer blocks put more rows into each chain and need fewer
    // rounds of workgroups, where n gives at least 4 rounds of them.
    // Measured (fp32, us, R = 4 / 8 / 16): config 2's square (13 C
    // diagonals) 90 / 71 / 60; the 7-point stencil's square 35 / 33 / 28.5
    // and H H^2 (63 C diagonals) 86.5 / 82 / 75.5, H H^4 and H H^5 (231,
    // 377) 524 / 483 / 492 and 912 / 856 / 902; config 4 44 / 47 / 43.
    // Fewer blocks lose at small n (gemm_diag's band at n = 65536: 13.4 /
    // 18 / 21) and where the longer window costs a workgroup per CU (the
    // 64-diagonal band at n = 2^18: 379 / 405 / -).  Complex values, R = 8
    // (80 VGPRs: one workgroup per CU): config 2's square 223 -> 194,
    // config 4 78 -> 83.  Complex A with more diagonals than 4 rows per lane
    // hold takes 2 (config 5 with complex values: 6.15 ms against 7.06 on
    // the gather); fp32 stays at 4 and at most DIAGPU_ASTAT_MAX_A diagonals
    // (2 rows per lane over 142 fp32 A diagonals lost to the gather: 200 x 64
    // at n = 2^18 3.17 against 2.64 ms).
    auto rounds_ok = [&](int rows, int64_t slots) {
        return ceil_div<int64_t>(n, 64 * rows) >= 4 * slots;
    };
    if constexpr (sizeof(T) == 8)
        if (nA > Astat<T, 4>::kMax) return DIAGPU_ASTAT_LAUNCH(2);
    if constexpr (kForceR == 2) {
        if (nA <= Astat<T, 2>::kMax) return DIAGPU_ASTAT_LAUNCH(2);
    } else if constexpr (kForceR == 16 && sizeof(T) == 4) {
        if (nA <= Astat<T, 16>::kMax) return DIAGPU_ASTAT_LAUNCH(16);
    } else if constexpr (kForceR == 8) {
        if (nA <= Astat<T, 8>::kMax) return DIAGPU_ASTAT_LAUNCH(8);
    } else if constexpr (kForceR == 0 && sizeof(T) == 4) {
        // few, short C diagonals: 16 rows per lane
        if (c_ndiag <= 4 * kWaves && n_pairs <= 4 * c_ndiag && nA <= Astat<T, 16>::kMax &&
            rounds_ok(16, astat_slots<T, 16>(nA)))
            return DIAGPU_ASTAT_LAUNCH(16);
        // many C diagonals: 8, where two workgroups still fit a CU
        if (c_ndiag > 4 * kWaves && nA <= Astat<T, 8>::kMax2 && rounds_ok(8, astat_slots<T, 8>(nA)))
            return DIAGPU_ASTAT_LAUNCH(8);
    } else if constexpr (kForceR == 0) {
        // complex: 8 where every wave has at most one C diagonal
        if (c_ndiag <= kWaves && nA <= Astat<T, 8>::kMax && rounds_ok(8, astat_slots<T, 8>(nA)))
            return DIAGPU_ASTAT_LAUNCH(8);
    }
    return DIAGPU_ASTAT_LAUNCH(4);
#undef DIAGPU_ASTAT_LAUNCH
}

}  // namespace

int launch_astat_records(hipStream_t s, int32_t n, const int32_t* A_off,
                         const int64_t* A_starts, int32_t nA, const int32_t* B_off,
                         const int64_t* B_starts, int32_t nB, const int32_t* C_off,
                         const int64_t* pair_ptr, int64_t c_bound, int64_t c_capacity,
                         const diagpu_gpair* pairs, int64_t pair_capacity,
                         const int64_t* state_counts, int32_t* state_flags, int32_t* records)
{
    const int64_t c_grid = std::min(c_bound, c_capacity);
    hipLaunchKernelGGL(k_astat_records,
                       dim3((unsigned)std::max<int64_t>(1, ceil_div<int64_t>(c_grid, kPrepBlock))),
                       dim3(kPrepBlock), 0, s, n, A_off, A_starts, nA, B_off, B_starts, nB, C_off,
                       pair_ptr, c_capacity, pairs, pair_capacity, state_counts, state_flags,
                       records);
    return check_launch("diagpu_spgemm_symbolic_astat");
}

}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spgemm_astat_prepare(int32_t n, const int32_t* A_off,
                                           const int64_t* A_starts, int32_t nA,
                                           const int32_t* B_off, const int64_t* B_starts,
                                           int32_t nB, const int32_t* C_off,
                                           const int64_t* pair_ptr, int64_t c_ndiag,
                                           const diagpu_gpair* pairs, int64_t n_pairs,
                                           int32_t* records, void* stream)
{
    using namespace diagpu;
    const char* fn = "diagpu_spgemm_astat_prepare";
    if (n < 1 || nA < 1 || nB < 1 || n_pairs < 0 || n_pairs > INT_MAX || c_ndiag < 0 ||
        c_ndiag > 2 * (int64_t)n - 1)
        return fail(DIAGPU_ERR_ARG,
                    "%s: need n, nA, nB >= 1, 0 <= c_ndiag <= 2n - 1 and "
                    "0 <= n_pairs <= 2^31 - 1", fn);
    if (!A_off || !A_starts || !B_off || !B_starts || !records ||
        (n_pairs > 0 && (!pairs || !C_off || !pair_ptr)))
        return fail(DIAGPU_ERR_ARG, "%s: a pointer is NULL", fn);
    if (n_pairs > 0 && c_ndiag == 0)
        return fail(DIAGPU_ERR_ARG, "%s: plan entries without C diagonals", fn);
    hipStream_t s = as_stream(stream);
    int32_t* flag = records + 4 * n_pairs;   // the 4 ints after the records
    int32_t host[2] = {0, 0};
    hipLaunchKernelGGL(k_astat_init, dim3(1), dim3(64), 0, s, flag, A_off, nA);
    int st = check_launch(fn);
    if (!st && n_pairs > 0) {
        hipLaunchKernelGGL(k_astat_prepare,
                           dim3((unsigned)ceil_div<int64_t>(c_ndiag, kPrepBlock)),
                           dim3(kPrepBlock), 0, s, n, A_off, A_starts, nA, B_off, B_starts, nB,
                           C_off, pair_ptr, c_ndiag, pairs, n_pairs,
                           reinterpret_cast<int4*>(records), flag);
        st = check_launch(fn);
    }
    if (!st) st = check_hip(hipMemcpyWithStream(host, flag, sizeof(host), hipMemcpyDeviceToHost, s), fn);
    if (st) return st;
    if (host[0])
        return fail(DIAGPU_ERR_ARG,
                    "%s: a plan entry is not in the symbolic plan's form (starts, offsets, "
                    "shifts or lengths)", fn);
    if (host[1]) return fail(DIAGPU_ERR_CAPACITY, "%s: B indices beyond 2^30 - 1", fn);
    return DIAGPU_OK;
}

DIAGPU_API int diagpu_spgemm_numeric_astat_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    const float* B_vals, const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts,
    int64_t c_ndiag, const int64_t* pair_ptr, const int32_t* records, int64_t n_pairs,
    float* C_vals, void* stream)
{
    return diagpu::launch_astat<float>("diagpu_spgemm_numeric_astat_f32", n, A_off, A_starts, nA,
                                       A_vals, B_vals, C_off, C_len, C_starts, c_ndiag, pair_ptr,
                                       records, n_pairs, C_vals, stream);
}

DIAGPU_API int diagpu_spgemm_numeric_astat_c64(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA,
    const diagpu_complex64* A_vals, const diagpu_complex64* B_vals, const int32_t* C_off,
    const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag, const int64_t* pair_ptr,
    const int32_t* records, int64_t n_pairs, diagpu_complex64* C_vals, void* stream)
{
    using diagpu::cf32;
    return diagpu::launch_astat<cf32>("diagpu_spgemm_numeric_astat_c64", n, A_off, A_starts, nA,
                                      reinterpret_cast<const cf32*>(A_vals),
                                      reinterpret_cast<const cf32*>(B_vals), C_off, C_len,
                                      C_starts, c_ndiag, pair_ptr, records, n_pairs,
                                      reinterpret_cast<cf32*>(C_vals), stream);
}

DIAGPU_API int diagpu_spgemm_numeric_astat_scaled_f32(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA, const float* A_vals,
    float alpha, const float* B_vals, const int32_t* C_off, const int32_t* C_len,
    const int64_t* C_starts, int64_t c_ndiag, const int64_t* pair_ptr, const int32_t* records,
    int64_t n_pairs, float sigma, float* C_vals, void* stream)
{
    return diagpu::launch_astat<float>("diagpu_spgemm_numeric_astat_scaled_f32", n, A_off,
                                       A_starts, nA, A_vals, B_vals, C_off, C_len, C_starts,
                                       c_ndiag, pair_ptr, records, n_pairs, C_vals, stream, true,
                                       alpha, sigma);
}

DIAGPU_API int diagpu_spgemm_numeric_astat_scaled_c64(
    int32_t n, const int32_t* A_off, const int64_t* A_starts, int32_t nA,
    const diagpu_complex64* A_vals, diagpu_complex64 alpha, const diagpu_complex64* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const int32_t* records, int64_t n_pairs, diagpu_complex64 sigma,
    diagpu_complex64* C_vals, void* stream)
{
    using diagpu::cf32;
    return diagpu::launch_astat<cf32>(
        "diagpu_spgemm_numeric_astat_scaled_c64", n, A_off, A_starts, nA,
        reinterpret_cast<const cf32*>(A_vals), reinterpret_cast<const cf32*>(B_vals), C_off, C_len,
        C_starts, c_ndiag, pair_ptr, records, n_pairs, reinterpret_cast<cf32*>(C_vals), stream,
        true, cf32{alpha.re, alpha.im}, cf32{sigma.re, sigma.im});
}

}  // extern "C"
