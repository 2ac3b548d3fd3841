/*
 * ref_generators.cpp -- driver around the reference's own input generators.
 *
 * TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (target `ref`) where the
 * reference checkout exists, run only by tests/golden/make_generator_golden.py
 * to write the fixtures that pin the oracle's restatements of these
 * generators.  Nothing in the product or on the GPU box runs it.
 *
 * The generators themselves are not in this file: the Makefile cuts each one
 * out of its reference source by line range into a temporary directory and
 * this driver #includes it, so the program runs the reference's text as
 * written, with only standard headers around it:
 *   ref_hash.inc         hval, xval           spmv/bench/bench_cusparse.cu:70-82
 *   ref_lcg.inc          run_case's H and x   spmv/test/test_tc_spmv.cu:86-98
 *   ref_make_banded.inc  DiaMatrix, make_banded  spmspm/bench_spmspm.cu:79-106
 *   ref_pack.inc         pack_diag_matrix     gemm_diag/gemm_diag.cu:361-382
 *
 * Usage (raw little-endian arrays on stdout):
 *   xval N                   float32[N]           xval(0..N-1)
 *   hval N d...              float32[]            hval(r, d) for the band's entries
 *                                                 (0 <= r + d < N), offset by offset,
 *                                                 rows ascending
 *   lcg N d...               float32[N * N], float32[N]   H, x of run_case
 *   banded n w seed          int32 count, int32[count] offsets, int64[count]
 *                            starts, int32[count] lengths, float32[nnz] values
 *   pack n seed d...         float32[P * n]       DA of pack_diag_matrix
 */
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "ref_hash.inc"
#include "ref_make_banded.inc"
#include "ref_pack.inc"

static void ref_lcg_case(int N, const std::vector<int>& offsets, std::vector<float>& H_out,
                         std::vector<float>& x_out)
{
#include "ref_lcg.inc"
    H_out = H;
    x_out = x;
}

template <typename T>
static void put(const std::vector<T>& v)
{
    if (!v.empty()) std::fwrite(v.data(), sizeof(T), v.size(), stdout);
}

static std::vector<int> ints_from(int argc, char** argv, int first)
{
    std::vector<int> v;
    for (int i = first; i < argc; ++i) v.push_back(std::atoi(argv[i]));
    return v;
}

int main(int argc, char** argv)
{
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s xval|hval|lcg|banded|pack ...\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    const int N = std::atoi(argv[2]);
    if (mode == "xval") {
        std::vector<float> x(N);
        for (int i = 0; i < N; ++i) x[i] = xval(i);
        put(x);
    } else if (mode == "hval") {
        const std::vector<int> offs = ints_from(argc, argv, 3);
        std::vector<float> v;
        for (int d : offs)
            for (int r = 0; r < N; ++r)
                if (r + d >= 0 && r + d < N) v.push_back(hval(r, d));
        put(v);
    } else if (mode == "lcg") {
        const std::vector<int> offs = ints_from(argc, argv, 3);
        std::vector<float> H, x;
        ref_lcg_case(N, offs, H, x);
        put(H);
        put(x);
    } else if (mode == "banded" && argc == 5) {
        const DiaMatrix M = make_banded(N, std::atoi(argv[3]), (unsigned)std::strtoul(argv[4], nullptr, 10));
        const int32_t cnt = (int32_t)M.offsets.size();
        std::fwrite(&cnt, sizeof(cnt), 1, stdout);
        std::vector<int32_t> offs(M.offsets.begin(), M.offsets.end());
        std::vector<int64_t> starts(M.starts.begin(), M.starts.end());
        std::vector<int32_t> lens(M.lengths.begin(), M.lengths.end());
        put(offs);
        put(starts);
        put(lens);
        put(M.values);
    } else if (mode == "pack" && argc >= 4) {
        const unsigned seed = (unsigned)std::strtoul(argv[3], nullptr, 10);
        const std::vector<int> offs = ints_from(argc, argv, 4);
        std::vector<float> DA;
        std::vector<int> off_out;
        pack_diag_matrix(N, offs, seed, DA, off_out);
        put(DA);
    } else {
        std::fprintf(stderr, "bad arguments\n");
        return 2;
    }
    return std::fflush(stdout) == 0 ? 0 : 1;
}
