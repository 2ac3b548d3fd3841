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
// per tile give the issued flops (2 * 16 * 16 * 4 per block), against which
// the plan's useful flops give the MFMA utilisation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace diagpu {

constexpr int kMfmaRows = 64;       // rows per wave slab (4 tiles of 16)
constexpr int kMfmaWaves = 4;       // waves per workgroup, each on its own slabs
constexpr int kMfmaThreads = 64 * kMfmaWaves;
constexpr int kMfmaMaxBlocks = 64;  // issued (ct, ks) blocks per tile
constexpr int kMfmaMaxCt = 4;       // column tiles held in registers at once
constexpr int kMfmaMaxKs = 12;      // k steps of 4 per tile: A's range <= 32 wide
constexpr int64_t kMfmaLdsBudget = 80 * 1024;
// LDS row strides in floats.  A lane (q, r) of an MFMA block reads A at row
// (q - r) + const, column r, B at row (r - q) + const, column q, and writes C
// at row (r - 4 q) + const, column 4 q; these strides put the 64 lanes on 64
// different banks (and each half-wave on 32), where the natural 64 / 128
// would put 4 / 16 lanes on one bank.
constexpr int kMfmaStrideA = 80;
constexpr int kMfmaStrideB = 145;
constexpr int kMfmaStrideC = 69;

struct MfmaGeom {
    int32_t a_min, a_max, b_min, b_max;
    int32_t nct, nks, nblk;
    int32_t wm;                       // B window rows in LDS (2 kMfmaRows)
    int64_t lds_bytes;
    int32_t ok;                       // 1: fits the limits above
    uint8_t blk[kMfmaMaxBlocks];      // (ct << 5) | ks, ct ascending
};

// Floats of one wave's LDS: a zero row for A and one for B, then A's rows
// and B's window, over which the slab's C values are written once the
// matrix work is done.
__host__ __device__ inline int64_t mfma_wave_floats(int64_t aspan, int64_t bspan)
{
    const int64_t ab = (aspan + 1) * kMfmaStrideA + (bspan + 1) * kMfmaStrideB;
    const int64_t c = (aspan + bspan + 1) * kMfmaStrideC;
    return kMfmaStrideA + kMfmaStrideB + (ab > c ? ab : c);
}

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
    if (g.nct > kMfmaMaxCt || g.nks > kMfmaMaxKs) return g;
    const int64_t c_min = (int64_t)a_min + b_min;
    int nb = 0;
    for (int ct = 0; ct < g.nct; ++ct)
        for (int ks = 0; ks < g.nks; ++ks) {
            // some k of the block (q) has an A element of some row i and a B
            // element of some column j inside the offset ranges
            bool any = false;
            for (int q = 0; q < 4 && !any; ++q) {
                bool a_in = false, b_in = false;
                for (int r = 0; r < 16; ++r) {
                    const int64_t da = a_min + 4 * ks + q - r;            // row i = r
                    const int64_t db = c_min + 16 * ct + r - (a_min + 4 * ks + q);   // column j = r
                    a_in = a_in || (da >= a_min && da <= a_max);
                    b_in = b_in || (db >= b_min && db <= b_max);
                }
                any = a_in && b_in;
            }
            if (!any) continue;
            if (nb == kMfmaMaxBlocks) return g;
            g.blk[nb++] = (uint8_t)((ct << 5) | ks);
        }
    g.nblk = nb;
    g.wm = 2 * kMfmaRows;
    // per wave its rows; per workgroup the C starts by offset, the lists of
    // absent A and B offsets and their two counts
    g.lds_bytes = 4 * (int64_t)kMfmaWaves * mfma_wave_floats(aspan, bspan) + 8 * (cspan + 1) +
                  4 * (aspan + bspan + 4);
    g.ok = g.lds_bytes <= kMfmaLdsBudget ? 1 : 0;
    return g;
}

}  // namespace diagpu
