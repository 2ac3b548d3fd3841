// GPU test of the MatrixMarket path (include/diagpu/mtx.hpp): a file read
// with read_mtx_dia goes through the reference-named API onto the GPU,
//   DiaMatrix -> build_recon -> launch_tc_spmv_regdirect      (SpMV)
//   HM (the square file's diagonals) -> SpgemmPlan(H, H)     (SpGEMM)
// and the results are checked against the CPU oracle (oracle/liboracle.so,
// test infrastructure): the Recon layout, C structure and pair plan bit for
// bit, values within 1e-5 * sum |terms| of the fp64 sums.  This is the
// loading path gen_banded_mtx.cpp's files (spmv/tools/gen_banded_mtx.cpp:37-48)
// and Hamiltonians exported as MatrixMarket take.
//
//   test_mtx_gpu [--write-band PATH N] FILE...
// --write-band first writes the SpMV bench's 9-diagonal hash band of N rows
// (spmv/bench/bench_cusparse.cu:84-87) with write_mtx_band, then reads it
// back like the other files.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "diagpu/dia.hpp"
#include "diagpu/mtx.hpp"

extern "C" {
void orc_build_recon_f32(int rows, int cols, int K, const int* offsets, const int64_t* starts,
                         const int* lengths, const float* values, int* r_offsets, float* r_values);
void orc_spmv_recon_f32_ref64(int rows, int cols, int K, const int* offs, const float* vals,
                              const float* x, int64_t x_size, double* y, double* abs_sum);
int orc_c_structure(int n, const int* A_off, int nA, const int* B_off, int nB, int* C_off,
                    int* C_len, int64_t* C_starts, int64_t* nnz);
int64_t orc_pairs_only(int n, const int* A_off, int nA, const int* A_len, const int64_t* A_starts,
                       const int* B_off, int nB, const int* B_len, const int64_t* B_starts,
                       const int* C_off, int nC, int64_t* pair_ptr, void* pairs);
void orc_spgemm_pairs_f64(const float* A_vals, const float* B_vals, const int* C_len,
                          const int64_t* C_starts, const int64_t* pair_ptr, const void* pairs,
                          int kbeg, int kend, double* out, double* abs_out);
float orc_hval(int r, int d);
float orc_xval(int i);
}

static bool g_all = true;

static void report(const std::string& name, bool ok, const char* detail = "")
{
    std::printf("  %-44s %s %s\n", name.c_str(), ok ? "[OK]" : "[FAIL]", detail);
    std::fflush(stdout);
    g_all &= ok;
}

static void write_hash_band(const std::string& path, int N)
{
    diagpu::MtxBand B;
    B.rows = B.cols = N;
    int64_t s = 0;
    for (int d : {-9, -5, -2, -1, 0, 1, 2, 5, 9}) {
        B.offsets.push_back(d);
        B.starts.push_back(s);
        for (int r = std::max(0, -d); r < std::min(N, N - d); ++r, ++s) B.values.push_back(orc_hval(r, d));
    }
    diagpu::write_mtx_band(path, B);
}

static void spmv_case(const std::string& tag, const diagpu::MtxDia& M)
{
    DiaMatrix D;
    D.rows = M.rows;
    D.cols = M.cols;
    D.offsets = M.offsets;
    D.diag_lengths = M.lengths;
    D.values = M.values;
    for (int64_t s : M.starts) D.diag_starts.push_back(static_cast<int>(s));
    const ReconMatrix R = build_recon(D);
    const int K = R.num_diags;
    std::vector<int> o_off(K);
    std::vector<float> o_val(static_cast<size_t>(K) * M.cols);
    orc_build_recon_f32(M.rows, M.cols, K, M.offsets.data(), M.starts.data(), M.lengths.data(),
                        M.values.data(), o_off.data(), o_val.data());
    report(tag + ": build_recon == oracle", o_off == R.diag_offsets && o_val == R.values);

    std::vector<float> x(M.cols);
    for (int i = 0; i < M.cols; ++i) x[i] = orc_xval(i);
    diagpu::DeviceRecon dR(R);
    diagpu::DeviceArray<float> dx(x), dy(static_cast<size_t>(M.rows));
    launch_tc_spmv_regdirect(dR.view, dx.data(), M.cols, dy.data(), 0);
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const std::vector<float> y = dy.download();
    std::vector<double> y64(M.rows), ab(M.rows);
    orc_spmv_recon_f32_ref64(M.rows, M.cols, K, R.diag_offsets.data(), R.values.data(), x.data(),
                             M.cols, y64.data(), ab.data());
    bool ok = true;
    double worst = 0.0;
    for (int r = 0; r < M.rows; ++r) {
        const double err = std::fabs(y[r] - y64[r]);
        ok &= err <= 1e-5 * ab[r] + 1e-300;
        if (ab[r] > 0) worst = std::max(worst, err / ab[r]);
    }
    char buf[128];
    std::snprintf(buf, sizeof buf, "%dx%d, %d diagonals, worst err/sum|t| %.1e", M.rows, M.cols,
                  K, worst);
    report(tag + ": SpMV == oracle", ok, buf);
}

static void spgemm_case(const std::string& tag, const diagpu::MtxDia& M)
{
    const int n = M.rows, K = static_cast<int>(M.offsets.size());
    diagpu::DeviceArray<int> doff(M.offsets), dlen(M.lengths);
    diagpu::DeviceArray<int64_t> dst(M.starts);
    diagpu::DeviceArray<float> dv(M.values);
    diagpu::SpgemmPlan plan(n, doff.data(), dlen.data(), dst.data(), K, doff.data(), dlen.data(),
                            dst.data(), K);
    const diagpu_spgemm_info inf = plan.info();
    // plan against the oracle, bit for bit
    const int cap = std::min<int64_t>(int64_t(K) * K, 2 * int64_t(n) - 1);
    std::vector<int> c_off(cap), c_len(cap);
    std::vector<int64_t> c_st(cap);
    int64_t nnz = 0;
    const int nc = orc_c_structure(n, M.offsets.data(), K, M.offsets.data(), K, c_off.data(),
                                   c_len.data(), c_st.data(), &nnz);
    c_off.resize(nc);
    c_len.resize(nc);
    c_st.resize(nc);
    std::vector<int64_t> ptr(nc + 1);
    const int64_t np = orc_pairs_only(n, M.offsets.data(), K, M.lengths.data(), M.starts.data(),
                                      M.offsets.data(), K, M.lengths.data(), M.starts.data(),
                                      c_off.data(), nc, ptr.data(), nullptr);
    std::vector<diagpu_gpair> pairs(np);
    orc_pairs_only(n, M.offsets.data(), K, M.lengths.data(), M.starts.data(), M.offsets.data(), K,
                   M.lengths.data(), M.starts.data(), c_off.data(), nc, ptr.data(), pairs.data());
    auto down = [](const auto* p, int64_t cnt) {
        using T = std::remove_cv_t<std::remove_pointer_t<decltype(p)>>;
        std::vector<T> h(cnt);
        if (cnt) diagpu::check_hip(hipMemcpy(h.data(), p, cnt * sizeof(T), hipMemcpyDeviceToHost), "copy");
        return h;
    };
    const bool plan_ok = inf.c_ndiag == nc && inf.c_nnz == nnz && inf.n_pairs == np &&
                         down(plan.c_offsets(), nc) == c_off && down(plan.c_lengths(), nc) == c_len &&
                         down(plan.c_starts(), nc) == c_st && down(plan.pair_ptr(), nc + 1) == ptr &&
                         std::memcmp(down(plan.pairs(), np).data(), pairs.data(),
                                     np * sizeof(diagpu_gpair)) == 0;
    char buf[128];
    std::snprintf(buf, sizeof buf, "%d C diagonals, %lld entries", nc, (long long)np);
    report(tag + ": H*H plan == oracle", plan_ok, buf);
    diagpu::DeviceArray<float> dc(static_cast<size_t>(std::max<int64_t>(1, nnz)));
    plan.numeric(dv.data(), dv.data(), dc.data());
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const std::vector<float> c = dc.download();
    std::vector<double> want(nnz), ab(nnz);
    orc_spgemm_pairs_f64(M.values.data(), M.values.data(), c_len.data(), c_st.data(), ptr.data(),
                         pairs.data(), 0, nc, want.data(), ab.data());
    bool ok = true;
    for (int64_t i = 0; i < nnz; ++i) ok &= std::fabs(c[i] - want[i]) <= 1e-5 * ab[i] + 1e-300;
    report(tag + ": H*H values == oracle", ok);
}

int main(int argc, char** argv)
{
    std::vector<std::string> files;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--write-band") == 0 && i + 2 < argc) {
            const std::string path = argv[i + 1];
            write_hash_band(path, std::atoi(argv[i + 2]));
            files.push_back(path);
            i += 2;
        } else {
            files.push_back(argv[i]);
        }
    }
    if (files.empty()) {
        std::printf("usage: test_mtx_gpu [--write-band PATH N] FILE...\n");
        return 2;
    }
    std::printf("MatrixMarket files through the GPU path\n");
    for (const std::string& f : files) {
        const std::string tag = f.substr(f.find_last_of('/') + 1);
        std::printf("%s\n", f.c_str());
        std::fflush(stdout);
        const diagpu::MtxDia M = diagpu::read_mtx_dia(f);
        spmv_case(tag, M);
        if (M.rows == M.cols) spgemm_case(tag, M);
    }
    std::printf(g_all ? "ALL TESTS PASSED\n" : "SOME TESTS FAILED\n");
    return g_all ? 0 : 1;
}
