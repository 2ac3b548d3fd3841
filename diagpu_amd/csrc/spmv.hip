// DIA SpMV on the column-indexed Recon layout, gfx950.
//
//   y[r] = sum_k [0 <= r + d_k < lim] Recon[k][r + d_k] * x[r + d_k],
//   lim = min(cols, x_size)
//
// (spmv/src/dia_reconstruct.cuh:22, bounds as in
// spmv/src/tc_spmv_regdirect_kernel.cu:85-104).  The reference lifts the band
// to a TF32 MMA and keeps 1/16 of the product; here the sum is what it is, an
// HBM stream: every useful value is read once and fused into its row's
// accumulator.
//
// Element types.  One kernel family serves real fp32 and fp64, complex64
// matrices with complex64 vectors, and real fp32 matrices with complex64
// vectors (a real Hamiltonian applied to a complex state: the matrix is read
// once for both parts of x).  A lane owns R rows, R times the wider of the
// two elements being 16 bytes: its x and y runs are 16 bytes, its value run
// 16 bytes (8 for a real matrix with complex vectors, where 32-byte x runs
// would leave every 16-byte x load half coalesced).
//
// Mapping.  A workgroup of 256 lanes owns a tile of 256 x R consecutive rows.
// For diagonal k the lane needs Recon[k][r+d_k ..] and x[r+d_k ..]: runs at
// the same column, loaded as 16-byte vectors (dword aligned: gfx950 serves
// unaligned global loads); the 64 lanes of a wave cover 1 KiB of each
// stream.  Value loads and the y store are non-temporal: each value is used
// once, while x stays in L2 for the tiles that re-read it.
//
// Memory-level parallelism.  What bounds this kernel is how many HBM bytes
// each CU keeps in flight, not the x re-reads or the misalignment (measured:
// a 64-stream read with the same offsets and no x runs at 80% of 8 TB/s, and
// adding the x loads costs 3 points).  So loads are never drained in chunks:
// the ring kernel keeps W diagonals' loads in flight per lane at all times --
// step j consumes slot j and refills it with the diagonal W ahead, and
// sched_barrier pins that order so the compiler emits a steady vmcnt window
// instead of hoisting or sinking the loads.  Offsets come through the scalar
// cache (the compiler batches them into s_load_dwordx4/x2), which does not
// queue behind the HBM stream, so one ring runs over all K diagonals with no
// drain anywhere (measured against 64 offsets per VGPR broadcast by
// readlane, with a refill of that VGPR every 64 diagonals: 1.7 points of
// 8 TB/s on config 3's 64 diagonals, about 1 point at 85 and 377).  For
// K <= 5 the short kernel issues all 2K loads straight-line.
//
// Edge tiles.  A tile whose rows or columns leave the matrix for some
// diagonal runs the same ring, still with 16-byte runs, each loaded at its
// start column clamped into [0, lim - R] (always a valid run), and masked
// accumulation: no branch around a load, so the loads pipeline like the
// interior ones.  A lane whose run straddles column 0 or lim finds its
// in-range elements inside the clamped run, shifted by (start - clamped
// start), and picks them out with selects; lanes wholly out of range all load
// the same clamped run (one cache line per wave) and mask every term.  This
// keeps an edge tile about as fast as an interior one, which matters when
// the offset spread is a sizeable part of n (a propagator with hundreds of
// diagonals spread over +-10^5 rows has a fifth of its tiles at the edges,
// all on the XCDs that own the first and last rows).  Only a matrix
// narrower than one run (lim < R) falls back to per-element loads at
// clamped columns.  An edge tile is also dispatched early (odd XCDs walk
// their row range from the end).
//
// XCD awareness: workgroup b runs on XCD b mod 8; tiles are remapped so each
// XCD owns one contiguous eighth of the rows.  x[c] is used by rows c - d_k
// of every diagonal, i.e. by this tile and by tiles up to max|d_k| rows away,
// which then sit on the same XCD and find x in its L2.
//
// Dot epilogue (Krylov drivers).  With DOT, each workgroup also forms
// sum_r Re(conj(x[r]) * y[r]) over its rows in fp64 and stores it as one
// partial; a one-workgroup kernel launched next adds the partials in tile
// order (a deterministic result).
#include <climits>

#include "common.hpp"
#include "elem.hpp"
#include "reduce.hpp"
#include "spmv_internal.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;
constexpr int kShortMax = 16;   // K <= kShortMax: straight-line kernel

// Per (matrix element, vector element) pair: rows per lane and ring depths,
// chosen so the kernels stay within 64 VGPRs (8 waves per SIMD).
template <typename TV, typename TX> struct Shape {
    // 16 bytes of the wider of the two elements: a real matrix applied to a
    // complex vector takes 2 rows per lane (8-byte value runs), so that every
    // x load and y store is a fully coalesced 16-byte run.
    static constexpr int R = (int)(16 / (sizeof(TV) > sizeof(TX) ? sizeof(TV) : sizeof(TX)));
    static constexpr int W = 6;    // interior ring
    static constexpr int WR = 4;   // edge ring
    static constexpr int TILE = kBlock * R;
};

// ---------------------------------------------------------------------------
// Shared pieces
// ---------------------------------------------------------------------------

// Tile index of workgroup b: XCD x = b mod 8 owns tiles [x*per_xcd,
// (x+1)*per_xcd); even XCDs walk their range upwards, odd ones downwards, so
// the last tile of the matrix (an edge tile) is among the first dispatched.
inline __device__ int tile_of_block(int per_xcd)
{
    const int x = (int)(blockIdx.x % kNumXcd);
    const int l = (int)(blockIdx.x / kNumXcd);
    return x * per_xcd + ((x & 1) ? per_xcd - 1 - l : l);
}

// min and max of a group of offsets held one per lane (lanes >= gn hold a
// copy of a valid offset), uniform across the wave.
inline __device__ void wave_minmax(int v, int& lo, int& hi)
{
    int a = v, b = v;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) {
        const int oa = __shfl_xor(a, s);
        const int ob = __shfl_xor(b, s);
        a = oa < a ? oa : a;
        b = ob > b ? ob : b;
    }
    lo = __builtin_amdgcn_readfirstlane(a);
    hi = __builtin_amdgcn_readfirstlane(b);
}

// How a group's loads treat columns outside [0, lim).
enum EdgeMode {
    kInterior = 0,   // the whole tile is in range: plain 16-byte runs
    kEdgeRun = 1,    // 16-byte runs at clamped starts, shifted and masked
};

// The gn diagonals with offsets `offs` (read with uniform indices: scalar
// loads) and values `vg` (Recon rows) accumulated into `acc` for the lane's R
// rows starting at row `r`.  W diagonals' loads in flight; every index is
// clamped to [0, gn) so all loads are valid, and the slots past the end are
// masked.  kEdgeRun needs lim >= R and masks every term whose column is
// outside [0, lim).
template <typename TV, typename TX, int W, int MODE>
__device__ __forceinline__ void ring_group(int64_t r, int64_t cols, int64_t lim, int gn,
                                           const int32_t* __restrict__ offs,
                                           const TV* __restrict__ vg, const TX* __restrict__ x,
                                           Run<TX, Shape<TV, TX>::R>& acc)
{
    constexpr int R = Shape<TV, TX>::R;
    Run<TV, R> a[W];
    Run<TX, R> b[W];
    // a run start clamped to a valid run, [0, lim - R] (kEdgeRun)
    auto clamp_run = [&](int64_t c) -> int64_t {
        const int64_t hi = lim - R;
        return c < 0 ? 0 : (c > hi ? hi : c);
    };
    auto issue = [&](int j, int k) {
        const int d = offs[k];
        const TV* vk = vg + (int64_t)k * cols;
        if constexpr (MODE == kInterior) {
            a[j] = load_run<TV, R, true>(vk + r + d);
            b[j] = load_run<TX, R, false>(x + r + d);
        } else {
            const uint32_t cc = (uint32_t)clamp_run(r + d);
            a[j] = load_run<TV, R, true>(vk + cc);
            b[j] = load_run<TX, R, false>(x + cc);
        }
    };
    // slot j holds diagonal k (k uniform); `on` = the slot is part of the group
    auto consume = [&](int j, int k, bool on) {
        if constexpr (MODE == kInterior) {
#pragma unroll
            for (int e = 0; e < R; ++e)
                acc.v[e] = sel(on, mad(acc.v[e], a[j].v[e], b[j].v[e]), acc.v[e]);
        } else {
            const int64_t c = r + offs[k];
            // element e of the run sits at index e + s of what was loaded
            const int s = (int)(c - clamp_run(c));
#pragma unroll
            for (int e = 0; e < R; ++e) {
                const bool ok = on && (uint64_t)(c + e) < (uint64_t)lim;
                TV av = a[j].v[0];
                TX bv = b[j].v[0];
#pragma unroll
                for (int i = 1; i < R; ++i) {
                    const bool m = e + s == i;
                    av = sel(m, a[j].v[i], av);
                    bv = sel(m, b[j].v[i], bv);
                }
                acc.v[e] = sel(ok, mad(acc.v[e], av, bv), acc.v[e]);
            }
        }
    };

#pragma unroll
    for (int j = 0; j < W; ++j) issue(j, j < gn ? j : gn - 1);
    __builtin_amdgcn_sched_barrier(0);
    int k0 = 0;
    while (k0 + 2 * W <= gn) {   // every refill of this round is in range
#pragma unroll
        for (int j = 0; j < W; ++j) {
            consume(j, k0 + j, true);
            __builtin_amdgcn_sched_barrier(0);
            issue(j, k0 + W + j);
            __builtin_amdgcn_sched_barrier(0);
        }
        k0 += W;
    }
    // Last two rounds: slots hold k0 .. k0+W-1 (those >= gn are clamped
    // copies); refills are clamped the same way.
#pragma unroll
    for (int j = 0; j < W; ++j) {
        const int kc = k0 + j;
        consume(j, kc < gn ? kc : gn - 1, kc < gn);
        __builtin_amdgcn_sched_barrier(0);
        const int kn = k0 + W + j;
        issue(j, kn < gn ? kn : gn - 1);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < W - 1; ++j) {
        const int kc = k0 + W + j;
        consume(j, kc < gn ? kc : gn - 1, kc < gn);
    }
}

// A non-interior tile (lim >= R: the host sends narrower matrices to
// spmv_narrow_kernel).
template <typename TV, typename TX>
__device__ __forceinline__ void edge_group(int64_t r, int64_t cols, int64_t lim, int gn,
                                           const int32_t* __restrict__ offs,
                                           const TV* __restrict__ vg, const TX* __restrict__ x,
                                           Run<TX, Shape<TV, TX>::R>& acc)
{
    ring_group<TV, TX, Shape<TV, TX>::WR, kEdgeRun>(r, cols, lim, gn, offs, vg, x, acc);
}

template <typename TX, int R>
__device__ __forceinline__ void store_rows(TX* __restrict__ y, int64_t r, int64_t rows,
                                           const Run<TX, R>& acc, bool full)
{
    if (full) {
        store_run_nt<TX, R>(y + r, acc);
    } else {
#pragma unroll
        for (int e = 0; e < R; ++e)
            if (r + e < rows) y[r + e] = acc.v[e];
    }
}

// DOT epilogue: see the file comment.  x must hold the lane's rows
// (x_size >= rows, checked by the host).
template <typename TX, int R>
__device__ __forceinline__ void dot_epilogue(const Run<TX, R>& acc, const TX* __restrict__ x,
                                             int64_t r, int64_t rows, bool full, int tile,
                                             int tiles, const DotArgs& da)
{
    double s = 0.0;
    if (full) {
        const Run<TX, R> u = load_run<TX, R, false>(x + r);
#pragma unroll
        for (int e = 0; e < R; ++e) s += dotpart(u.v[e], acc.v[e]);
    } else {
#pragma unroll
        for (int e = 0; e < R; ++e)
            if (r + e < rows) s += dotpart(x[r + e], acc.v[e]);
    }
    store_partial<kBlock>(s, tile, da.partials);
}

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------

// K > kShortMax: one ring over all K diagonals.
template <typename TV, typename TX, bool DOT>
__global__ __launch_bounds__(kBlock) void spmv_ring_kernel(
    int32_t rows, int32_t cols, int64_t lim, int32_t K, const int32_t* __restrict__ offs,
    const TV* __restrict__ vals, const TX* __restrict__ x, TX* __restrict__ y, int32_t tiles,
    int32_t per_xcd, DotArgs da)
{
    typedef Shape<TV, TX> S;
    constexpr int R = S::R;
    const int tile = tile_of_block(per_xcd);
    if (tile >= tiles) return;
    const int lane = (int)threadIdx.x & 63;
    const int64_t r0 = (int64_t)tile * S::TILE;
    const int64_t r = r0 + (int64_t)threadIdx.x * R;

    // offset range (one vector load per 64 offsets, reduced across the wave)
    int dmin = INT_MAX, dmax = INT_MIN;
    for (int g0 = 0; g0 < K; g0 += 64) {
        const int gn = (K - g0) < 64 ? (K - g0) : 64;
        int lo, hi;
        wave_minmax(offs[g0 + (lane < gn ? lane : gn - 1)], lo, hi);
        dmin = lo < dmin ? lo : dmin;
        dmax = hi > dmax ? hi : dmax;
    }
    const bool interior =
        r0 + S::TILE <= rows && r0 + dmin >= 0 && r0 + S::TILE + (int64_t)dmax <= lim;

    Run<TX, R> acc;
#pragma unroll
    for (int e = 0; e < R; ++e) acc.v[e] = zero_of<TX>();
    if (interior)
        ring_group<TV, TX, S::W, kInterior>(r, cols, lim, K, offs, vals, x, acc);
    else
        edge_group<TV, TX>(r, cols, lim, K, offs, vals, x, acc);
    store_rows<TX, R>(y, r, rows, acc, interior);
    if constexpr (DOT) dot_epilogue<TX, R>(acc, x, r, rows, interior, tile, tiles, da);
}

// K == KF <= kShortMax: offsets by scalar loads, all 2K loads straight-line.
template <typename TV, typename TX, int KF, bool DOT>
__global__ __launch_bounds__(kBlock) void spmv_short_kernel(
    int32_t rows, int32_t cols, int64_t lim, int32_t K, const int32_t* __restrict__ offs,
    const TV* __restrict__ vals, const TX* __restrict__ x, TX* __restrict__ y, int32_t tiles,
    int32_t per_xcd, DotArgs da)
{
    typedef Shape<TV, TX> S;
    constexpr int R = S::R;
    const int tile = tile_of_block(per_xcd);
    if (tile >= tiles) return;
    const int64_t r0 = (int64_t)tile * S::TILE;
    const int64_t r = r0 + (int64_t)threadIdx.x * R;
    (void)K;

    int d[KF > 0 ? KF : 1];
    int dmin = INT_MAX, dmax = INT_MIN;
#pragma unroll
    for (int k = 0; k < KF; ++k) {
        d[k] = offs[k];
        dmin = d[k] < dmin ? d[k] : dmin;
        dmax = d[k] > dmax ? d[k] : dmax;
    }
    const bool interior = r0 + S::TILE <= rows &&
                          (KF == 0 || (r0 + dmin >= 0 && r0 + S::TILE + (int64_t)dmax <= lim));

    Run<TX, R> acc;
#pragma unroll
    for (int e = 0; e < R; ++e) acc.v[e] = zero_of<TX>();
    if constexpr (KF > 0) {
        if (interior) {
            Run<TV, R> a[KF];
            Run<TX, R> b[KF];
#pragma unroll
            for (int k = 0; k < KF; ++k) {
                a[k] = load_run<TV, R, true>(vals + (int64_t)k * cols + r + d[k]);
                b[k] = load_run<TX, R, false>(x + r + d[k]);
            }
#pragma unroll
            for (int k = 0; k < KF; ++k)
#pragma unroll
                for (int e = 0; e < R; ++e) acc.v[e] = mad(acc.v[e], a[k].v[e], b[k].v[e]);
        } else {
            edge_group<TV, TX>(r, cols, lim, KF, offs, vals, x, acc);
        }
    }
    store_rows<TX, R>(y, r, rows, acc, interior);
    if constexpr (DOT) dot_epilogue<TX, R>(acc, x, r, rows, interior, tile, tiles, da);
}

// lim < R (fewer than R columns of x in range): no 16-byte run fits, so
// every term is a per-element load behind its bounds check.  Same tiles and
// epilogues as the other kernels.
template <typename TV, typename TX, bool DOT>
__global__ __launch_bounds__(kBlock) void spmv_narrow_kernel(
    int32_t rows, int32_t cols, int64_t lim, int32_t K, const int32_t* __restrict__ offs,
    const TV* __restrict__ vals, const TX* __restrict__ x, TX* __restrict__ y, int32_t tiles,
    int32_t per_xcd, DotArgs da)
{
    typedef Shape<TV, TX> S;
    constexpr int R = S::R;
    const int tile = tile_of_block(per_xcd);
    if (tile >= tiles) return;
    const int64_t r = (int64_t)tile * S::TILE + (int64_t)threadIdx.x * R;
    Run<TX, R> acc;
#pragma unroll
    for (int e = 0; e < R; ++e) acc.v[e] = zero_of<TX>();
    for (int k = 0; k < K; ++k) {
        const int64_t c = r + offs[k];
        const TV* vk = vals + (int64_t)k * cols;
#pragma unroll
        for (int e = 0; e < R; ++e)
            if ((uint64_t)(c + e) < (uint64_t)lim) acc.v[e] = mad(acc.v[e], vk[c + e], x[c + e]);
    }
    store_rows<TX, R>(y, r, rows, acc, false);
    if constexpr (DOT) dot_epilogue<TX, R>(acc, x, r, rows, false, tile, tiles, da);
}

template <typename TV, typename TX>
using SpmvKernel = void (*)(int32_t, int32_t, int64_t, int32_t, const int32_t*, const TV*,
                            const TX*, TX*, int32_t, int32_t, DotArgs);

template <typename TV, typename TX, bool DOT>
SpmvKernel<TV, TX> pick_kernel(int K, int64_t lim)
{
    if (K > 0 && lim < Shape<TV, TX>::R) return spmv_narrow_kernel<TV, TX, DOT>;
    switch (K) {
    case 0: return spmv_short_kernel<TV, TX, 0, DOT>;
    case 1: return spmv_short_kernel<TV, TX, 1, DOT>;
    case 2: return spmv_short_kernel<TV, TX, 2, DOT>;
    case 3: return spmv_short_kernel<TV, TX, 3, DOT>;
    case 4: return spmv_short_kernel<TV, TX, 4, DOT>;
    case 5: return spmv_short_kernel<TV, TX, 5, DOT>;
    case 6: return spmv_short_kernel<TV, TX, 6, DOT>;
    case 7: return spmv_short_kernel<TV, TX, 7, DOT>;
    case 8: return spmv_short_kernel<TV, TX, 8, DOT>;
    case 9: return spmv_short_kernel<TV, TX, 9, DOT>;
    case 10: return spmv_short_kernel<TV, TX, 10, DOT>;
    case 11: return spmv_short_kernel<TV, TX, 11, DOT>;
    case 12: return spmv_short_kernel<TV, TX, 12, DOT>;
    case 13: return spmv_short_kernel<TV, TX, 13, DOT>;
    case 14: return spmv_short_kernel<TV, TX, 14, DOT>;
    case 15: return spmv_short_kernel<TV, TX, 15, DOT>;
    case 16: return spmv_short_kernel<TV, TX, 16, DOT>;
    default: return spmv_ring_kernel<TV, TX, DOT>;
    }
}
static_assert(kShortMax == 16, "pick_kernel covers K = 0..16");

}  // namespace

template <typename TV, typename TX>
int32_t spmv_tiles(int32_t rows)
{
    return (int32_t)ceil_div<int64_t>(rows, Shape<TV, TX>::TILE);
}

template <typename TV, typename TX>
int spmv_run(int32_t rows, int32_t cols, int32_t num_diags, const int32_t* offs, const TV* vals,
             const TX* x, int64_t x_size, TX* y, const DotArgs* dot, void* stream,
             const char* name)
{
    if (rows < 0 || cols < 0 || num_diags < 0)
        return fail(DIAGPU_ERR_ARG, "%s: negative size (rows=%d cols=%d num_diags=%d)", name,
                    rows, cols, num_diags);
    if (x_size < 0) return fail(DIAGPU_ERR_ARG, "%s: negative x_size %lld", name, (long long)x_size);
    if (rows == 0) return DIAGPU_OK;
    if (!y) return fail(DIAGPU_ERR_ARG, "%s: y is NULL", name);
    const int64_t lim = x_size < cols ? x_size : (int64_t)cols;
    int K = num_diags;
    if (K > 0) {
        if (!offs) return fail(DIAGPU_ERR_ARG, "%s: diag_offsets is NULL", name);
        if (cols > 0 && !vals) return fail(DIAGPU_ERR_ARG, "%s: values is NULL", name);
        if (lim > 0 && !x) return fail(DIAGPU_ERR_ARG, "%s: x is NULL", name);
    }
    if (dot && (x_size < rows || !x || !dot->partials))
        return fail(DIAGPU_ERR_ARG, "%s: the dot epilogue needs x_size >= rows and its buffers",
                    name);
    if (lim == 0) K = 0;   // no column in range: y = 0 without touching values or x
    const int32_t tiles = spmv_tiles<TV, TX>(rows);
    const int32_t per_xcd = ceil_div<int32_t>(tiles, kNumXcd);
    const DotArgs da = dot ? *dot : DotArgs{nullptr, nullptr};
    hipLaunchKernelGGL((dot ? pick_kernel<TV, TX, true>(K, lim) : pick_kernel<TV, TX, false>(K, lim)),
                       dim3(per_xcd * kNumXcd), dim3(kBlock), 0, as_stream(stream), rows, cols,
                       lim, K, offs, vals, x, y, tiles, per_xcd, da);
    const int st = check_launch(name);
    if (st || !dot || !dot->out) return st;
    return sum_partials(dot->partials, tiles, dot->out, stream);
}

namespace {
constexpr int kSumBlock = 1024;
constexpr int kSumUnroll = 8;

struct SumJob {
    const double* partials;
    int32_t n;
    double* out;
};

// Workgroup b sums job b.  Lane l adds partials l, l + 1024, l + 2048, ... in
// that order (loads of a batch of 8 issued before their adds), then a fixed
// tree: deterministic, and up to 8192 partials cost one memory round trip.
__global__ __launch_bounds__(kSumBlock) void k_sum_partials(SumJob j0, SumJob j1)
{
    const SumJob job = blockIdx.x == 0 ? j0 : j1;
    const double* __restrict__ partials = job.partials;
    const int32_t n = job.n;
    double t = 0.0;
    int i = (int)threadIdx.x;
    for (; i + (kSumUnroll - 1) * kSumBlock < n; i += kSumUnroll * kSumBlock) {
        double v[kSumUnroll];
#pragma unroll
        for (int u = 0; u < kSumUnroll; ++u) v[u] = partials[i + u * kSumBlock];
#pragma unroll
        for (int u = 0; u < kSumUnroll; ++u) t += v[u];
    }
    for (; i < n; i += kSumBlock) t += partials[i];
    t = block_sum<kSumBlock>(t);
    if (threadIdx.x == 0) *job.out = t;
}
}  // namespace

int sum_partials(const double* partials, int32_t n, double* out, void* stream)
{
    const SumJob j0{partials, n, out};
    hipLaunchKernelGGL(k_sum_partials, dim3(1), dim3(kSumBlock), 0, as_stream(stream), j0, j0);
    return check_launch("sum_partials");
}

int sum_partials2(const double* p0, int32_t n0, double* out0, const double* p1, int32_t n1,
                  double* out1, void* stream)
{
    hipLaunchKernelGGL(k_sum_partials, dim3(2), dim3(kSumBlock), 0, as_stream(stream),
                       SumJob{p0, n0, out0}, SumJob{p1, n1, out1});
    return check_launch("sum_partials2");
}

#define DIAGPU_SPMV_INSTANCE(TV, TX)                                                          \
    template int32_t spmv_tiles<TV, TX>(int32_t);                                             \
    template int spmv_run<TV, TX>(int32_t, int32_t, int32_t, const int32_t*, const TV*,       \
                                  const TX*, int64_t, TX*, const DotArgs*, void*, const char*);
DIAGPU_SPMV_INSTANCE(float, float)
DIAGPU_SPMV_INSTANCE(double, double)
DIAGPU_SPMV_INSTANCE(cf32, cf32)
DIAGPU_SPMV_INSTANCE(float, cf32)
#undef DIAGPU_SPMV_INSTANCE

}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spmv_recon_f32(const diagpu_recon_view_f32* R, const float* x,
                                     int64_t x_size, float* y, void* stream)
{
    const char* fn = "diagpu_spmv_recon_f32";
    if (!R) return diagpu::fail(DIAGPU_ERR_ARG, "%s: R is NULL", fn);
    return diagpu::spmv_run<float, float>(R->rows, R->cols, R->num_diags, R->diag_offsets,
                                          R->values, x, x_size, y, nullptr, stream, fn);
}

DIAGPU_API int diagpu_spmv_recon_f64(const diagpu_recon_view_f64* R, const double* x,
                                     int64_t x_size, double* y, void* stream)
{
    const char* fn = "diagpu_spmv_recon_f64";
    if (!R) return diagpu::fail(DIAGPU_ERR_ARG, "%s: R is NULL", fn);
    return diagpu::spmv_run<double, double>(R->rows, R->cols, R->num_diags, R->diag_offsets,
                                            R->values, x, x_size, y, nullptr, stream, fn);
}

DIAGPU_API int diagpu_spmv_recon_c64(const diagpu_recon_view_c64* R, const diagpu_complex64* x,
                                     int64_t x_size, diagpu_complex64* y, void* stream)
{
    using diagpu::cf32;
    const char* fn = "diagpu_spmv_recon_c64";
    if (!R) return diagpu::fail(DIAGPU_ERR_ARG, "%s: R is NULL", fn);
    return diagpu::spmv_run<cf32, cf32>(R->rows, R->cols, R->num_diags, R->diag_offsets,
                                        reinterpret_cast<const cf32*>(R->values),
                                        reinterpret_cast<const cf32*>(x), x_size,
                                        reinterpret_cast<cf32*>(y), nullptr, stream, fn);
}

DIAGPU_API int diagpu_spmv_recon_f32_c64(const diagpu_recon_view_f32* R,
                                         const diagpu_complex64* x, int64_t x_size,
                                         diagpu_complex64* y, void* stream)
{
    using diagpu::cf32;
    const char* fn = "diagpu_spmv_recon_f32_c64";
    if (!R) return diagpu::fail(DIAGPU_ERR_ARG, "%s: R is NULL", fn);
    return diagpu::spmv_run<float, cf32>(R->rows, R->cols, R->num_diags, R->diag_offsets,
                                         R->values, reinterpret_cast<const cf32*>(x), x_size,
                                         reinterpret_cast<cf32*>(y), nullptr, stream, fn);
}

}  // extern "C"
