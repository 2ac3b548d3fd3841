// GPU test of the C++ drop-in headers (include/diagpu/*.hpp), written the way
// the reference's own tests are (spmv/test/test_tc_spmv.cu,
// spmv/test/test_reconstruct.cpp): build inputs on the host, run through the
// reference-named API, compare, print one line per case, exit status = pass.
//
// Integer outputs (Recon layout, C structure, lookup, pair plan) are compared
// bit for bit with the CPU oracle (oracle/liboracle.so, test infrastructure);
// values against an fp64 reference with |err| <= 1e-5 * sum |terms|.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <unistd.h>
#include <cstring>
#include <random>
#include <vector>

#include "diagpu/dia.hpp"

extern "C" {
void orc_build_recon_f32(int rows, int cols, int K, const int* offsets, const int64_t* starts,
                         const int* lengths, const float* values, int* r_offsets, float* r_values);
int orc_c_structure(int n, const int* A_off, int nA, const int* B_off, int nB, int* C_off,
                    int* C_len, int64_t* C_starts, int64_t* nnz);
void orc_c_lookup(int n, const int* C_off, int nC, int* lookup);
int64_t orc_pairs_only(int n, const int* A_off, int nA, const int* A_len, const int64_t* A_starts,
                       const int* B_off, int nB, const int* B_len, const int64_t* B_starts,
                       const int* C_off, int nC, int64_t* pair_ptr, void* pairs);
void orc_spgemm_pairs_f64(const float* A_vals, const float* B_vals, const int* C_len,
                          const int64_t* C_starts, const int64_t* pair_ptr, const void* pairs,
                          int kbeg, int kend, double* out, double* abs_out);
int orc_make_banded(int n, int w, unsigned seed, int* offsets, int64_t* starts, int* lengths,
                    float* values);
void orc_pack_diag_matrix(int n, const int* offsets, int P, unsigned seed, float* DA);
void orc_hash_band_recon(int N, const int* offsets, int K, int* r_offsets, float* r_values,
                         float* x);
void orc_gemm_diag_f64(int n, const float* DA, const int* off_A, int P, const float* DB,
                       const int* off_B, int Q, const int* C_lookup, const int64_t* C_starts,
                       double* out, double* abs_out);
}

static bool g_all = true;

static void report(const char* name, bool ok, const char* detail = "")
{
    std::printf("  %-40s %s %s\n", name, ok ? "[OK]" : "[FAIL]", detail);
    g_all &= ok;
}

static std::vector<float> gpu_spmv(const ReconMatrix& R, const std::vector<float>& x)
{
    diagpu::DeviceRecon dR(R);
    diagpu::DeviceArray<float> dx(x), dy(R.rows);
    launch_tc_spmv_regdirect(dR.view, dx.data(), (int)x.size(), dy.data(), 0);
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    return dy.download();
}

static void test_known_answer()
{
    // spmv/test/test_reconstruct.cpp:185-194
    const float H[25] = {1, 2, 3, 0, 0, 4, 5, 6, 7, 0, 8, 9, 8, 7, 6, 0, 5, 4, 3, 2, 0, 0, 1, 2, 3};
    const std::vector<float> x = {1, 2, 3, 4, 5};
    const DiaMatrix D = dense_to_dia(H, 5, 5);
    const ReconMatrix R = build_recon(D);
    const std::vector<int> want_off = {2, 1, 0, -1, -2};
    const std::vector<float> want_rows = {0, 0, 3, 7, 6, 0, 2, 6, 7, 2, 1, 5, 8, 3, 3,
                                          4, 9, 4, 2, 0, 8, 5, 1, 0, 0};
    report("5x5 build_recon", R.diag_offsets == want_off && R.values == want_rows);
    const auto y = gpu_spmv(R, x);
    report("5x5 launch_tc_spmv_regdirect", y == std::vector<float>({14, 60, 108, 44, 26}));
}

static void test_tc_case(const char* name, int N, const std::vector<int>& offsets)
{
    // inputs exactly as spmv/test/test_tc_spmv.cu:86-98
    std::vector<float> H((size_t)N * N, 0.0f);
    unsigned seed = 0x1234567u + (unsigned)N;
    auto rng = [&]() {
        seed = seed * 1664525u + 1013904223u;
        return (float)((seed >> 8) & 0xFFFF) / 65536.0f * 2.0f - 1.0f;
    };
    for (int r = 0; r < N; ++r)
        for (int d : offsets) {
            const int c = r + d;
            if (c >= 0 && c < N) H[(size_t)r * N + c] = rng();
        }
    std::vector<float> x(N);
    for (int i = 0; i < N; ++i) x[i] = rng();
    const DiaMatrix D = dense_to_dia(H.data(), N, N);
    const ReconMatrix R = build_recon(D);
    // Recon layout bit-exact with the oracle's build_recon
    std::vector<int64_t> st(D.diag_starts.begin(), D.diag_starts.end());
    std::vector<int> o_off(R.num_diags);
    std::vector<float> o_val((size_t)R.num_diags * N);
    orc_build_recon_f32(N, N, R.num_diags, D.offsets.data(), st.data(), D.diag_lengths.data(),
                        D.values.data(), o_off.data(), o_val.data());
    const bool layout_ok = o_off == R.diag_offsets && o_val == R.values;
    const auto y = gpu_spmv(R, x);
    const auto yh = spmv_from_recon(R, x);   // the header's host SpMV, same bound
    bool ok = yh.size() == (size_t)N;
    double worst = 0;
    for (int r = 0; r < N; ++r) {
        double s = 0, a = 0;
        for (int c = 0; c < N; ++c) {
            const double t = (double)H[(size_t)r * N + c] * x[c];
            s += t;
            a += std::fabs(t);
        }
        const double err = std::fabs(y[r] - s);
        worst = std::max(worst, err / (a + 1e-300));
        ok &= err <= 1e-5 * a + 1e-300;
        ok &= std::fabs(yh[r] - s) <= 1e-5 * a + 1e-300;
    }
    char buf[96];
    std::snprintf(buf, sizeof buf, "N=%d diags=%d worst err/sum|t|=%.1e", N, R.num_diags, worst);
    report(name, layout_ok && ok, buf);
}

static void test_spmv_f64()
{
    const int n = 4099;
    std::mt19937 g(3);
    std::vector<int> offs = {700, 3, 0, -1, -2000};
    std::vector<double> vals((size_t)offs.size() * n), x(n);
    for (auto& v : vals) v = (double)(g() % 20001) / 10000.0 - 1.0;
    for (auto& v : x) v = (double)(g() % 20001) / 10000.0 - 1.0;
    diagpu::DeviceArray<int> doff(offs);
    diagpu::DeviceArray<double> dv(vals), dx(x), dy(n);
    diagpu::launch_dia_spmv(diagpu::ReconViewF64{n, n, (int)offs.size(), doff.data(), dv.data()},
                            dx.data(), n, dy.data());
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto y = dy.download();
    bool ok = true;
    for (int r = 0; r < n; ++r) {
        long double s = 0, a = 0;
        for (size_t k = 0; k < offs.size(); ++k) {
            const long c = (long)r + offs[k];
            if (c >= 0 && c < n) {
                const long double t = (long double)vals[k * n + c] * x[c];
                s += t;
                a += std::fabs((double)t);
            }
        }
        ok &= std::fabs((double)(y[r] - s)) <= 1e-13 * (double)a + 1e-300;
    }
    report("fp64 launch_dia_spmv", ok);
}

static HMMatrix random_hm(int n, std::vector<int> offs, unsigned seed)
{
    std::mt19937 g(seed);
    std::vector<float> dense((size_t)n * n, 0.0f);
    for (int d : offs)
        for (int p = 0; p < n - std::abs(d); ++p) {
            const int r = d >= 0 ? p : p - d, c = d >= 0 ? p + d : p;
            dense[(size_t)r * n + c] = (float)(g() % 65536) / 32768.0f - 1.0f;
        }
    return dense_to_hm(dense.data(), n, offs);
}

static void test_spgemm(const char* name, int n, std::vector<int> oa, std::vector<int> ob)
{
    const HMMatrix A = random_hm(n, oa, 11), B = random_hm(n, ob, 12);
    const HMMatrix Cs = compute_c_hm_structure(A, B, n);
    const int cap = (int)std::min<int64_t>((int64_t)oa.size() * ob.size(), 2 * n - 1);
    std::vector<int> c_off(cap), c_len(cap);
    std::vector<int64_t> c_st(cap);
    int64_t nnz = 0;
    const int nc = orc_c_structure(n, oa.data(), (int)oa.size(), ob.data(), (int)ob.size(),
                                   c_off.data(), c_len.data(), c_st.data(), &nnz);
    c_off.resize(nc); c_len.resize(nc); c_st.resize(nc);
    report((std::string(name) + " compute_c_hm_structure").c_str(),
           Cs.diag_offsets == c_off && Cs.diag_lengths == c_len && Cs.diag_starts == c_st &&
               Cs.total_nz == nnz);
    std::vector<int> lk(2 * n - 1);
    orc_c_lookup(n, c_off.data(), nc, lk.data());
    report((std::string(name) + " build_c_diag_lookup").c_str(), build_c_diag_lookup(Cs, n) == lk);
    // pair plan, reference signature: Alookup built as the bench builds it
    std::vector<int> Alookup(2 * n - 1, -1);
    for (size_t i = 0; i < oa.size(); ++i) Alookup[oa[i] + (n - 1)] = (int)i;
    std::vector<size_t> as(A.diag_starts.begin(), A.diag_starts.end());
    std::vector<size_t> bs(B.diag_starts.begin(), B.diag_starts.end());
    const PairPlan pp = build_pairs_only(n, A.diag_lengths, as, B.diag_offsets, B.diag_lengths, bs,
                                         Alookup, c_off);
    std::vector<int64_t> o_ptr(nc + 1);
    const int64_t np = orc_pairs_only(n, oa.data(), (int)oa.size(), A.diag_lengths.data(),
                                      A.diag_starts.data(), ob.data(), (int)ob.size(),
                                      B.diag_lengths.data(), B.diag_starts.data(), c_off.data(), nc,
                                      o_ptr.data(), nullptr);
    std::vector<GPair> o_pairs(np);
    orc_pairs_only(n, oa.data(), (int)oa.size(), A.diag_lengths.data(), A.diag_starts.data(),
                   ob.data(), (int)ob.size(), B.diag_lengths.data(), B.diag_starts.data(),
                   c_off.data(), nc, o_ptr.data(), o_pairs.data());
    const bool plan_ok = pp.pairPtr == o_ptr && pp.pairs.size() == o_pairs.size() &&
                         std::memcmp(pp.pairs.data(), o_pairs.data(), np * sizeof(GPair)) == 0;
    report((std::string(name) + " build_pairs_only").c_str(), plan_ok);
    const FlatPlan fp = build_flat_plan(n, oa, A.diag_lengths, as, B.diag_offsets, B.diag_lengths,
                                        bs, Alookup, c_off, c_len, 512);
    int64_t tiles = 0;
    for (int k = 0; k < nc; ++k) tiles += (c_len[k] + 511) / 512;
    report((std::string(name) + " build_flat_plan").c_str(),
           fp.pairPtr == o_ptr && fp.nTiles == tiles);
    // values
    const HMMatrix C = spgemm_hm(A, B);
    std::vector<double> want(nnz), absum(nnz);
    orc_spgemm_pairs_f64(A.values.data(), B.values.data(), c_len.data(), c_st.data(), o_ptr.data(),
                         o_pairs.data(), 0, nc, want.data(), absum.data());
    bool ok = C.diag_offsets == c_off && (int64_t)C.values.size() == nnz;
    for (int64_t i = 0; ok && i < nnz; ++i)
        ok &= std::fabs(C.values[i] - want[i]) <= 1e-5 * absum[i] + 1e-300;
    report((std::string(name) + " spgemm_hm values").c_str(), ok);
}

// The two numeric kernels of one plan: NumericKernel::Band (operands staged
// in LDS) returns the gather's bits; Auto picks Band on the reference
// driver's band (offsets -10..10, gemm_diag/gemm_diag.cu:467-486) at
// n = 2^19 and the gather where the plan is too small; a plan whose staged
// window does not fit refuses Band with DIAGPU_ERR_CAPACITY.
static void test_band_kernel()
{
    std::mt19937 g(7);
    std::vector<int> offs;
    for (int d = -10; d <= 10; ++d) offs.push_back(d);
    const int n = 1 << 19, P = (int)offs.size();
    std::vector<float> D((size_t)P * n, 0.0f);
    for (int i = 0; i < P; ++i) {
        const int sr = offs[i] >= 0 ? 0 : -offs[i];
        for (int p = 0; p < n - std::abs(offs[i]); ++p)
            D[(size_t)i * n + sr + p] = 0.5f + (float)(g() % 65536) / 65536.0f;
    }
    diagpu::DeviceArray<int> doff(offs);
    diagpu::DeviceArray<float> dD(D);
    diagpu::GemmDiag gd(n, doff.data(), P, doff.data(), P);
    report("band: Auto picks Band at n = 2^19", gd.plan().uses_band());
    const size_t nnz = (size_t)gd.info().c_nnz;
    diagpu::DeviceArray<float> c_band(nnz), c_gather(nnz), c_auto(nnz);
    gd.run(dD.data(), dD.data(), c_gather.data(), 0, diagpu::NumericKernel::Gather);
    gd.run(dD.data(), dD.data(), c_band.data(), 0, diagpu::NumericKernel::Band);
    gd.run(dD.data(), dD.data(), c_auto.data());
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto cg = c_gather.download(), cb = c_band.download(), ca = c_auto.download();
    report("band: Band == Gather, bit for bit",
           std::memcmp(cg.data(), cb.data(), nnz * sizeof(float)) == 0);
    report("band: Auto == Band", std::memcmp(ca.data(), cb.data(), nnz * sizeof(float)) == 0);
    // and the values against fp64 (the gather's bound)
    const diagpu::CLayout L = diagpu::build_c_layout(n, offs, offs);
    std::vector<double> want(L.total_c), absum(L.total_c);
    orc_gemm_diag_f64(n, D.data(), offs.data(), P, D.data(), offs.data(), P, L.k_to_idx.data(),
                      L.C_offsets.data(), want.data(), absum.data());
    bool ok = (int64_t)nnz == L.total_c;
    for (int64_t i = 0; ok && i < L.total_c; ++i)
        ok &= std::fabs(cb[i] - want[i]) <= 1e-5 * absum[i] + 1e-300;
    report("band: values", ok);

    // a small plan: Auto takes the gather, Band forced still matches it
    const int ns = 512;
    std::vector<float> Ds((size_t)P * ns, 0.0f);
    for (int i = 0; i < P; ++i) {
        const int sr = offs[i] >= 0 ? 0 : -offs[i];
        for (int p = 0; p < ns - std::abs(offs[i]); ++p)
            Ds[(size_t)i * ns + sr + p] = 0.5f + (float)(g() % 65536) / 65536.0f;
    }
    diagpu::DeviceArray<float> dDs(Ds);
    diagpu::GemmDiag small(ns, doff.data(), P, doff.data(), P);
    report("band: Auto keeps the gather at n = 512", !small.plan().uses_band());
    const size_t snz = (size_t)small.info().c_nnz;
    diagpu::DeviceArray<float> s_band(snz), s_gather(snz);
    small.run(dDs.data(), dDs.data(), s_gather.data(), 0, diagpu::NumericKernel::Gather);
    small.run(dDs.data(), dDs.data(), s_band.data(), 0, diagpu::NumericKernel::Band);
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto sg = s_gather.download(), sb = s_band.download();
    report("band: forced Band == Gather at n = 512",
           std::memcmp(sg.data(), sb.data(), snz * sizeof(float)) == 0);

    // A span of 8000 rows: two B windows of 8256 floats exceed the LDS budget
    std::vector<int> wide = {-4000, 4000};
    const int nw = 5000;
    std::vector<float> Dw((size_t)2 * nw, 1.0f);
    diagpu::DeviceArray<int> dwo(wide);
    diagpu::DeviceArray<float> dDw(Dw);
    diagpu::GemmDiag gw(nw, dwo.data(), 2, dwo.data(), 2);
    diagpu::DeviceArray<float> cw((size_t)std::max<int64_t>(1, gw.info().c_nnz));
    int status = DIAGPU_OK;
    try {
        gw.run(dDw.data(), dDw.data(), cw.data(), 0, diagpu::NumericKernel::Band);
    } catch (const diagpu::Error& e) {
        status = e.status;
    }
    report("band: too wide a window -> DIAGPU_ERR_CAPACITY", status == DIAGPU_ERR_CAPACITY);
}

// The A-stationary kernel through diagpu::SpgemmPlan: the square of a
// 40-diagonal band spread over +-256 at n = 2^18 (1600 plan entries, 40 per
// A diagonal) takes it under Auto, and every kernel returns the gather's
// bits.
static void test_astat_kernel()
{
    const int n = 1 << 18;
    std::mt19937 g(11);
    std::vector<int> offs = {0};
    while (offs.size() < 40) {
        const int d = (int)(g() % 513) - 256;
        if (std::find(offs.begin(), offs.end(), d) == offs.end()) offs.push_back(d);
    }
    std::sort(offs.begin(), offs.end());
    const int K = (int)offs.size();
    std::vector<int> lens(K);
    std::vector<int64_t> starts(K);
    int64_t tot = 0;
    for (int k = 0; k < K; ++k) {
        lens[k] = n - std::abs(offs[k]);
        starts[k] = tot;
        tot += lens[k];
    }
    std::vector<float> vals((size_t)tot);
    for (auto& v : vals) v = -1.0f + 2.0f * (float)(g() % 65536) / 65536.0f;
    diagpu::DeviceArray<int> doff(offs), dlen(lens);
    diagpu::DeviceArray<int64_t> dst(starts);
    diagpu::DeviceArray<float> dv(vals);
    diagpu::SpgemmPlan plan(n, doff.data(), dlen.data(), dst.data(), K, doff.data(), dlen.data(),
                            dst.data(), K);
    report("astat: Auto picks the A-stationary kernel", plan.uses_astat() && !plan.uses_band());
    const size_t nnz = (size_t)plan.info().c_nnz;
    diagpu::DeviceArray<float> cg(nnz), ca(nnz), cf(nnz);
    plan.numeric(dv.data(), dv.data(), cg.data(), 0, diagpu::NumericKernel::Gather);
    plan.numeric(dv.data(), dv.data(), ca.data());
    plan.numeric(dv.data(), dv.data(), cf.data(), 0, diagpu::NumericKernel::AStationary);
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto hg = cg.download(), ha = ca.download(), hf = cf.download();
    report("astat: Auto == Gather, bit for bit", std::memcmp(hg.data(), ha.data(), nnz * 4) == 0);
    report("astat: AStationary == Gather", std::memcmp(hg.data(), hf.data(), nnz * 4) == 0);

    // complex values v + i v' on the same plan: Auto takes the complex
    // A-stationary kernel (40 A diagonals <= DIAGPU_ASTAT_MAX_A_C64)
    std::vector<diagpu_complex64> cv((size_t)tot);
    for (size_t p = 0; p < cv.size(); ++p) cv[p] = diagpu_complex64{vals[p], vals[(p + 7) % cv.size()]};
    diagpu::DeviceArray<diagpu_complex64> dcv(cv), zg(nnz), za(nnz);
    report("astat: Auto takes complex values too", plan.uses_astat_c64());
    plan.numeric(dcv.data(), dcv.data(), zg.data(), 0, diagpu::NumericKernel::Gather);
    plan.numeric(dcv.data(), dcv.data(), za.data());
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto hzg = zg.download(), hza = za.download();
    report("astat: complex Auto == Gather, bit for bit",
           std::memcmp(hzg.data(), hza.data(), nnz * sizeof(diagpu_complex64)) == 0);
    bool refused = false;
    try {
        plan.numeric(dcv.data(), dcv.data(), za.data(), 0, diagpu::NumericKernel::Band);
    } catch (const diagpu::Error& e) {
        refused = e.status == DIAGPU_ERR_ARG;
    }
    report("astat: complex Band refused", refused);
}

// The reference benchmarks' operand generators against the oracle's
// restatements: make_banded(100000, 16, 1234 / 5678)
// (spmspm/bench_spmspm.cu:465-466) and pack_diag_matrix(4096, -10..10, 42 /
// 137) (gemm_diag/gemm_diag.cu:485-486), value for value.
static void test_generators()
{
    bool ok = true;
    for (unsigned seed : {1234u, 5678u}) {
        const int n = 100000, w = 16;
        const HMMatrix M = diagpu::make_banded(n, w, seed);
        std::vector<int> off(2 * w + 1), len(2 * w + 1);
        std::vector<int64_t> st(2 * w + 1);
        std::vector<float> val((size_t)(2 * w + 1) * n);
        const int nd = orc_make_banded(n, w, seed, off.data(), st.data(), len.data(), val.data());
        off.resize(nd);
        len.resize(nd);
        st.resize(nd);
        ok &= M.num_diags == nd && M.diag_offsets == off && M.diag_lengths == len &&
              M.diag_starts == st && (int64_t)M.values.size() == M.total_nz &&
              std::memcmp(M.values.data(), val.data(), M.values.size() * sizeof(float)) == 0;
    }
    report("make_banded == oracle (seeds 1234, 5678)", ok);
    bool pk = true;
    std::vector<int> offs;
    for (int d = -10; d <= 10; ++d) offs.push_back(d);
    for (unsigned seed : {42u, 137u}) {
        std::vector<float> DA, want(offs.size() * 4096);
        std::vector<int> oo;
        diagpu::pack_diag_matrix(4096, offs, seed, DA, oo);
        orc_pack_diag_matrix(4096, offs.data(), (int)offs.size(), seed, want.data());
        pk &= DA == want && oo == offs;
    }
    report("pack_diag_matrix == oracle (seeds 42, 137)", pk);
    // The SpMV benchmark's band (bench_cusparse.cu:84-144), offsets given
    // unsorted, one of them reaching past the matrix.
    const int N = 1 << 16;
    const std::vector<int> bo = {0, -9, 5, 2, -1, 1, -2, 9, -5, N + 3};
    const ReconMatrix R = diagpu::make_hash_band(N, bo);
    const std::vector<float> hx = diagpu::make_hash_x(N);
    std::vector<int> ro(bo.size());
    std::vector<float> rv(bo.size() * (size_t)N), rx(N);
    orc_hash_band_recon(N, bo.data(), (int)bo.size(), ro.data(), rv.data(), rx.data());
    report("make_hash_band / make_hash_x == oracle",
           R.rows == N && R.cols == N && R.num_diags == (int)bo.size() && R.diag_offsets == ro &&
               R.values == rv && hx == rx);
}

// pack_diag_matrix (gemm_diag/gemm_diag.cu:362-382): zeros outside each
// diagonal's rows, U(0.5, 1.5) inside, in the draw order of one
// std::mt19937 stream; then the reference driver's product (seeds 42 and
// 137, gemm_diag.cu:485-486) through GemmDiag against the fp64 oracle.
static void test_pack_diag_matrix()
{
    const int n = 300;
    const std::vector<int> offs = {-7, -1, 0, 2, 299};
    std::vector<float> DA, DB;
    std::vector<int> oa, ob;
    diagpu::pack_diag_matrix(n, offs, 42, DA, oa);
    diagpu::pack_diag_matrix(n, offs, 137, DB, ob);
    std::mt19937 rng(42);
    std::uniform_real_distribution<float> dist(0.5f, 1.5f);
    bool ok = oa == offs && DA.size() == offs.size() * (size_t)n;
    for (size_t ri = 0; ok && ri < offs.size(); ++ri) {
        const int d = offs[ri], first = d >= 0 ? 0 : -d, len = n - std::abs(d);
        for (int t = 0; t < n; ++t) {
            const float v = DA[ri * n + t];
            ok &= (t >= first && t < first + len) ? v == dist(rng) : v == 0.0f;
        }
    }
    report("pack_diag_matrix layout and draws", ok);
    const diagpu::CLayout L = diagpu::build_c_layout(n, oa, ob);
    diagpu::DeviceArray<int> dof(oa);
    diagpu::DeviceArray<float> dA(DA), dB(DB);
    diagpu::GemmDiag gd(n, dof.data(), (int)oa.size(), dof.data(), (int)ob.size());
    diagpu::DeviceArray<float> dC((size_t)gd.info().c_nnz);
    gd.run(dA.data(), dB.data(), dC.data());
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto C = dC.download();
    std::vector<double> want(L.total_c), absum(L.total_c);
    orc_gemm_diag_f64(n, DA.data(), oa.data(), (int)oa.size(), DB.data(), ob.data(),
                      (int)ob.size(), L.k_to_idx.data(), L.C_offsets.data(), want.data(),
                      absum.data());
    bool vok = gd.info().c_nnz == L.total_c;
    for (int64_t i = 0; vok && i < L.total_c; ++i)
        vok &= std::fabs(C[i] - want[i]) <= 1e-5 * absum[i] + 1e-300;
    report("pack_diag_matrix operands through GemmDiag", vok);
}

static void test_gemm_diag(const char* name, int n, std::vector<int> oa, std::vector<int> ob)
{
    std::mt19937 g(42);
    auto pack = [&](const std::vector<int>& offs) {
        std::vector<float> D(offs.size() * (size_t)n, 0.0f);
        for (size_t i = 0; i < offs.size(); ++i) {
            const int sr = offs[i] >= 0 ? 0 : -offs[i];
            for (int p = 0; p < n - std::abs(offs[i]); ++p)
                D[i * n + sr + p] = 0.5f + (float)(g() % 65536) / 65536.0f;
        }
        return D;
    };
    const auto DA = pack(oa), DB = pack(ob);
    const diagpu::CLayout L = diagpu::build_c_layout(n, oa, ob);
    std::vector<int> lk(2 * n - 1);
    orc_c_lookup(n, L.k_list.data(), L.num_k, lk.data());
    report((std::string(name) + " build_c_layout").c_str(), L.k_to_idx == lk);
    diagpu::DeviceArray<int> doa(oa), dob(ob);
    diagpu::DeviceArray<float> dA(DA), dB(DB);
    diagpu::GemmDiag gd(n, doa.data(), (int)oa.size(), dob.data(), (int)ob.size());
    diagpu::DeviceArray<float> dC((size_t)gd.info().c_nnz);
    gd.run(dA.data(), dB.data(), dC.data());
    diagpu::check_hip(hipDeviceSynchronize(), "sync");
    const auto C = dC.download();
    std::vector<double> want(L.total_c, 0.0), absum(L.total_c, 0.0);
    orc_gemm_diag_f64(n, DA.data(), oa.data(), (int)oa.size(), DB.data(), ob.data(), (int)ob.size(),
                      lk.data(), L.C_offsets.data(), want.data(), absum.data());
    bool ok = gd.info().c_nnz == L.total_c;
    for (int64_t i = 0; ok && i < L.total_c; ++i)
        ok &= std::fabs(C[i] - want[i]) <= 1e-5 * absum[i] + 1e-300;
    report((std::string(name) + " GemmDiag values").c_str(), ok);
}

// The grouped pair schedule from a GPU-built plan (SpgemmPlan::schedule)
// equals build_schedule over the operands' offsets (schedule.hpp, checked
// against the oracle's restatement of spmspm/bench_spmspm.cu:137-243 on the
// CPU), member for member: the bench's make_banded(100000, 16) operands and
// BASELINE config 4's offsets.
static void test_schedule()
{
    auto same = [](const Schedule& x, const Schedule& y) {
        return x.a_halo == y.a_halo && x.b_halo == y.b_halo && x.num_groups == y.num_groups &&
               x.max_a == y.max_a && x.max_b == y.max_b && x.max_pairs == y.max_pairs &&
               x.num_blocks == y.num_blocks && x.a_count == y.a_count && x.b_count == y.b_count &&
               x.pair_count == y.pair_count && x.t_out == y.t_out && x.a_globals == y.a_globals &&
               x.b_globals == y.b_globals && x.c_globals == y.c_globals &&
               x.pairs.size() == y.pairs.size() &&
               std::memcmp(x.pairs.data(), y.pairs.data(), x.pairs.size() * sizeof(PairEntry)) == 0 &&
               x.block_group == y.block_group && x.block_tile == y.block_tile;
    };
    {
        const HMMatrix A = diagpu::make_banded(100000, 16, 1234u);
        const HMMatrix B = diagpu::make_banded(100000, 16, 5678u);
        const HMMatrix C = compute_c_hm_structure(A, B, 100000);
        const Schedule want = build_schedule(A, B, C, 100000);
        diagpu::DeviceArray<int> ao(A.diag_offsets), al(A.diag_lengths), bo(B.diag_offsets),
            bl(B.diag_lengths);
        diagpu::DeviceArray<int64_t> as(A.diag_starts), bs(B.diag_starts);
        diagpu::SpgemmPlan plan(100000, ao.data(), al.data(), as.data(), A.num_diags, bo.data(),
                                bl.data(), bs.data(), B.num_diags);
        char buf[96];
        std::snprintf(buf, sizeof buf, "groups=%d halos=(%d,%d) blocks=%d", want.num_groups,
                      want.a_halo, want.b_halo, want.num_blocks);
        report("schedule: make_banded(100000,16) plan", same(plan.schedule(), want) &&
               want.num_groups == 9 && want.max_pairs == 236, buf);
    }
    {
        const int n = 1 << 20;
        const std::vector<int> ao_h = {-4, -3, -2, -1, 0, 1, 2, 3, 4};
        const std::vector<int> bo_h = {-16384, -128, -1, 0, 1, 128, 16384};
        std::vector<int> al_h, bl_h;
        for (int d : ao_h) al_h.push_back(n - std::abs(d));
        for (int d : bo_h) bl_h.push_back(n - std::abs(d));
        diagpu::DeviceArray<int> ao(ao_h), al(al_h), bo(bo_h), bl(bl_h);
        diagpu::DeviceArray<int64_t> as(diagpu::hm_starts(n, ao_h)), bs(diagpu::hm_starts(n, bo_h));
        diagpu::SpgemmPlan plan(n, ao.data(), al.data(), as.data(), 9, bo.data(), bl.data(),
                                bs.data(), 7);
        std::vector<int> c_off(plan.info().c_ndiag);
        diagpu::check_hip(hipMemcpy(c_off.data(), plan.c_offsets(), c_off.size() * sizeof(int),
                                    hipMemcpyDeviceToHost), "copy");
        const Schedule want = diagpu::build_schedule(n, ao_h, bo_h, c_off);
        report("schedule: config 4 plan (a_halo 16384)",
               same(plan.schedule(), want) && want.a_halo == 16384 && want.num_groups == 6);
    }
}

int main()
{
    // Unbuffered, so every line is out before anything that follows it.
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    std::printf("C++ drop-in API on the GPU\n");
    try {
        test_known_answer();
        test_tc_case("tridiagonal", 48, {-1, 0, 1});
        test_tc_case("tridiag ragged", 37, {-1, 0, 1});
        test_tc_case("pentadiagonal", 64, {-2, -1, 0, 1, 2});
        test_tc_case("9-diag wide band", 80, {-9, -5, -2, -1, 0, 1, 2, 5, 9});
        test_tc_case("asymmetric band", 71, {-3, 0, 2, 4, 7});
        test_tc_case("main diagonal", 16, {0});
        test_tc_case("wide band 3000", 3000, {-1500, -7, 0, 9, 2048});
        test_spmv_f64();
        test_spgemm("band", 300, {-4, -3, -2, -1, 0, 1, 2, 3, 4}, {-16, -1, 0, 1, 16});
        test_spgemm("scattered", 2000, {-1900, -77, 0, 5, 640}, {-3, -2, 300, 1999, 1});
        test_gemm_diag("gemm_diag band", 512, {-3, -2, -1, 0, 1, 2, 3}, {-3, -2, -1, 0, 1, 2, 3});
        test_gemm_diag("gemm_diag scattered", 700, {-300, -9, 0, 33}, {-600, -1, 2, 5, 450});
        test_band_kernel();
        test_astat_kernel();
        test_pack_diag_matrix();
        test_generators();
        test_schedule();
    } catch (const std::exception& e) {
        std::printf("  exception: %s\n", e.what());
        g_all = false;
    }
    std::printf("\n%s\n", g_all ? "ALL TESTS PASSED" : "SOME TESTS FAILED");
    // Leave without running static destructors: the HIP runtime and the
    // libraries registered with it (libdiagpu.so's kernels) would otherwise
    // be torn down in an order this program does not control.
    std::fflush(stdout);
    _exit(g_all ? 0 : 1);
}
