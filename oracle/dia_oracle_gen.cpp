/*
 * dia_oracle_gen.cpp -- the reference benches' own std::mt19937 inputs.
 *
 * TEST INFRASTRUCTURE ONLY (see dia_oracle.c for who may load it).
 *
 * The reference draws its SpGEMM and gemm_diag operands with std::mt19937 and
 * std::uniform_real_distribution<float>.  The engine is fixed by the C++
 * standard; the distribution's mapping is implementation-defined, and the
 * reference is built on Linux against libstdc++, which this file also uses
 * (g++ 11.4).  Values therefore match a libstdc++ build of the reference.
 */
#include <cstdint>
#include <cstdlib>
#include <random>

#define ORC_API extern "C" __attribute__((visibility("default")))

/* make_banded (spmspm/bench_spmspm.cu:89-106): offsets -w..w ascending
 * (diagonals with n - |d| <= 0 skipped), HM positions, values
 * U(-1, 1) from mt19937(seed), drawn diagonal by diagonal.  offsets/lengths
 * need 2w+1 entries, starts too, values sum(n - |d|).  Returns the diagonal
 * count. */
ORC_API int orc_make_banded(int n, int w, unsigned seed, int* offsets, int64_t* starts,
                            int* lengths, float* values)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    int nd = 0;
    int64_t off = 0;
    for (int d = -w; d <= w; ++d) {
        const int len = n - std::abs(d);
        if (len <= 0) continue;
        offsets[nd] = d; starts[nd] = off; lengths[nd] = len;
        for (int p = 0; p < len; ++p) values[off + p] = dist(rng);
        off += len;
        ++nd;
    }
    return nd;
}

/* pack_diag_matrix (gemm_diag/gemm_diag.cu:362-382): P x n row-packed array,
 * DA[ri * n + sr + p] = U(0.5, 1.5) from mt19937(seed) for p < n - |d|,
 * sr = max(-d, 0), zeros elsewhere. */
ORC_API void orc_pack_diag_matrix(int n, const int* offsets, int P, unsigned seed, float* DA)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(0.5f, 1.5f);
    for (int64_t i = 0; i < (int64_t)P * n; ++i) DA[i] = 0.0f;
    for (int ri = 0; ri < P; ++ri) {
        const int d = offsets[ri];
        const int sr = d >= 0 ? 0 : -d;
        const int len = n - std::abs(d);
        for (int p = 0; p < len; ++p) DA[(int64_t)ri * n + sr + p] = dist(rng);
    }
}
