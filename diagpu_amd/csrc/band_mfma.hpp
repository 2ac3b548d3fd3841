// Geometry of the MFMA band kernel (spgemm_band_mfma.hip), shared with the
// band prepare step that reports it (spgemm_band.hip).
//
// The product is evaluated as dense 16 x 16 x 4 fp32 MFMA blocks over each
// 16-row tile of C.  For a tile at row t0 the blocks cover
//   rows    i = t0 + (0..15)
//   k       = t0 + a_min + 4 ks + (0..3)      ks < nks: k - i spans A's offsets
//   columns j = t0 + c_min + 16 ct + (0..15)  ct < nct: j - i spans C's offsets
// with A(i, k) = A's diagonal k - i (zero where A has none) and B(k, j)
// likewise, c_min = a_min + b_min.  A block (ct, ks) is issued only if, for
// some k of it, some row's A offset and some column's B offset fall inside
// A's and B's offset ranges; every other block is zero.  The issued blocks
// depend on the two offset spans only, and for each column tile they are a
// contiguous run of k steps [ks_lo, ks_hi].  The issued blocks per tile
// give the issued flops (2 * 16 * 16 * 4 per block), against which the
// plan's useful flops give the MFMA utilisation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace diagpu {

constexpr int kMfmaRows = 64;       // rows per wave slab (4 tiles of 16)
constexpr int kMfmaWaves = 4;       // waves per workgroup, each on its own slabs
constexpr int kMfmaThreads = 64 * kMfmaWaves;
constexpr int kMfmaMaxCt = 4;       // column tiles held in registers at once
constexpr int kMfmaMaxKs = 12;      // k steps of 4 per tile: A's range <= 32 wide
constexpr int kMfmaMaxC = 16 * kMfmaMaxCt - 15;   // C offsets per slab (c span <= 48)
constexpr int64_t kMfmaLdsBudget = 160 * 1024;
// LDS row strides in floats.  A lane (q, r) of an MFMA block reads A at row
// (q - r) + const, column r, B at row (r - q) + const, column q, and writes C
// at row (r - 4 q) + const, column 4 q.  These strides put the 64 lanes on 64
// different banks (and each half-wave on 32): A 80 (or 112), B any stride of
// residue 17 or 49 mod 64 (81, 113, 145, ...), C 69; the natural 64 / 128
// would put 4 / 16 lanes on one bank.
constexpr int kMfmaStrideA = 80;
constexpr int kMfmaStrideC = 69;
// Floats past a slab's C values where lanes outside C's offset range write
// theirs (read by nobody): lane l, tile u at l + 16 u.
constexpr int kMfmaDump = 64 + 48;
// Per workgroup, before the waves' buffers: the C start of every offset of
// C's range (int64), the lists of absent A and B offsets and their counts.
__host__ __device__ inline int64_t mfma_meta_bytes(int64_t aspan, int64_t bspan)
{
    const int64_t b = 8 * (aspan + bspan + 1) + 4 * (aspan + bspan + 4);
    return (b + 15) / 16 * 16;
}

struct MfmaGeom {
    int32_t a_min, a_max, b_min, b_max;
    int32_t nct, nks, nblk;
    int32_t wm;                       // B window rows in LDS: 48 + 4 nks
    int32_t sb;                       // B row stride (floats), >= wm
    int32_t b0;                       // first float of B's rows' region
    int32_t buf;                      // floats of one staging buffer:
                                      // [zero][A rows][zero] [zero][B rows][zero]
    int64_t lds_bytes;
    int32_t ok;                       // 1: fits the limits above
    int8_t ks_lo[kMfmaMaxCt];         // issued k steps of column tile ct:
    int8_t ks_hi[kMfmaMaxCt];         // [ks_lo, ks_hi], empty if ks_lo > ks_hi
};

inline MfmaGeom mfma_geom(int32_t a_min, int32_t a_max, int32_t b_min, int32_t b_max)
{
    MfmaGeom g{};
    g.a_min = a_min;
    g.a_max = a_max;
    g.b_min = b_min;
    g.b_max = b_max;
    const int64_t aspan = (int64_t)a_max - a_min, bspan = (int64_t)b_max - b_min;
    const int64_t cspan = aspan + bspan;
    if (aspan < 0 || bspan < 0 || aspan > 4 * kMfmaMaxKs || cspan > 16 * kMfmaMaxCt) return g;
    g.nct = (int32_t)((cspan + 16 + 15) / 16);
    g.nks = (int32_t)((aspan + 16 + 3) / 4);
    if (g.nct > kMfmaMaxCt || g.nks > kMfmaMaxKs || cspan + 1 > kMfmaMaxC) return g;
    int nb = 0;
    for (int ct = 0; ct < kMfmaMaxCt; ++ct) {
        g.ks_lo[ct] = 1;
        g.ks_hi[ct] = 0;
    }
    for (int ct = 0; ct < g.nct; ++ct) {
        int lo = -1, hi = -1;
        for (int ks = 0; ks < g.nks; ++ks) {
            // some k of the block (q) has an A element of some row i = r and
            // a B element of some column j = r inside the offset ranges
            bool any = false;
            for (int q = 0; q < 4 && !any; ++q) {
                bool a_in = false, b_in = false;
                for (int r = 0; r < 16; ++r) {
                    const int64_t da = 4 * ks + q - r;                  // minus a_min
                    const int64_t db = 16 * ct + r - 4 * ks - q;        // minus b_min
                    a_in = a_in || (da >= 0 && da <= aspan);
                    b_in = b_in || (db >= 0 && db <= bspan);
                }
                any = a_in && b_in;
            }
            if (!any) continue;
            if (hi >= 0 && hi != ks - 1) return g;   // not a contiguous run
            if (lo < 0) lo = ks;
            hi = ks;
            ++nb;
        }
        if (lo >= 0) {
            g.ks_lo[ct] = (int8_t)lo;
            g.ks_hi[ct] = (int8_t)hi;
        }
    }
    g.nblk = nb;
    g.wm = 48 + 4 * g.nks;
    // the smallest stride >= wm of residue 17 or 49 mod 64
    int sb = g.wm;
    while (sb % 64 != 17 && sb % 64 != 49) ++sb;
    g.sb = sb;
    // A's and B's rows each between two zero rows, so an operand row index
    // clamped into [-1, span + 1] reads zeros outside the offset range
    g.b0 = (int32_t)((aspan + 3) * kMfmaStrideA);
    const int64_t buf = g.b0 + (bspan + 3) * (int64_t)sb;
    // C (and the dump) are written over a consumed buffer
    if ((cspan + 1) * kMfmaStrideC + kMfmaDump > buf) return g;
    g.buf = (int32_t)buf;
    // per wave one staging buffer
    g.lds_bytes = mfma_meta_bytes(aspan, bspan) + 4 * (int64_t)kMfmaWaves * buf;
    g.ok = g.lds_bytes <= kMfmaLdsBudget ? 1 : 0;
    return g;
}

}  // namespace diagpu
