// GPU test of include/diagpu/chain.hpp: matrix powers and the truncated
// Taylor series built by the device-planned SpGEMM chain, checked against
// dense float64 products on the host:
//   |P - P64| <= 1e-5 * k * (|H|^k)  elementwise (k products of fp32 sums),
// and the result's diagonal set equals the sumset of H's offsets.  The
// complex propagator U = exp(-i dt H) against a complex128 series on the
// host (|U - U64| <= 1e-5 * order * expm(dt |H|) + the truncation bound),
// U U^H = I, and U in the Recon layout (to_recon) applied by the complex
// SpMV against the dense product and against the Lanczos propagator.
#include <unistd.h>

#include <cmath>
#include <complex>
#include <cstdio>
#include <cstring>
#include <random>
#include <set>
#include <vector>

#include "diagpu/chain.hpp"
#include "diagpu/dia.hpp"

static bool g_all = true;

static void report(const char* name, bool ok, const char* detail = "")
{
    std::printf("  %-44s %s %s\n", name, ok ? "[OK]" : "[FAIL]", detail);
    g_all &= ok;
}

using Dense = std::vector<double>;   // n x n row-major

static HMMatrix random_hm(int n, const std::vector<int>& offs, unsigned seed)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> U(-1.0f, 1.0f);
    HMMatrix H;
    H.n = n;
    H.num_diags = static_cast<int>(offs.size());
    for (int d : offs) {
        H.diag_offsets.push_back(d);
        H.diag_starts.push_back(H.total_nz);
        H.diag_lengths.push_back(n - std::abs(d));
        for (int p = 0; p < n - std::abs(d); ++p) H.values.push_back(U(rng));
        H.total_nz += n - std::abs(d);
    }
    return H;
}

static Dense to_dense(const HMMatrix& H, bool absval = false)
{
    const int n = H.n;
    Dense D(static_cast<size_t>(n) * n, 0.0);
    for (int k = 0; k < H.num_diags; ++k) {
        const int d = H.diag_offsets[k];
        for (int p = 0; p < H.diag_lengths[k]; ++p) {
            const int r = p - std::min(d, 0);
            const double v = H.values[H.diag_starts[k] + p];
            D[static_cast<size_t>(r) * n + r + d] = absval ? std::fabs(v) : v;
        }
    }
    return D;
}

static Dense matmul(const Dense& A, const Dense& B, int n)
{
    Dense C(static_cast<size_t>(n) * n, 0.0);
    for (int i = 0; i < n; ++i)
        for (int k = 0; k < n; ++k) {
            const double a = A[static_cast<size_t>(i) * n + k];
            if (a == 0.0) continue;
            for (int j = 0; j < n; ++j) C[static_cast<size_t>(i) * n + j] += a * B[static_cast<size_t>(k) * n + j];
        }
    return C;
}

static std::vector<int> sumset(const std::vector<int>& a, const std::vector<int>& b, int n)
{
    std::set<int> s;
    for (int x : a)
        for (int y : b)
            if (std::abs(x + y) < n) s.insert(x + y);
    return {s.begin(), s.end()};
}

// got vs want with |err| <= rel * bound elementwise; the diagonal set must be `offs`.
static bool compare(const HMMatrix& got, const Dense& want, const Dense& bound, double rel,
                    const std::vector<int>& offs, char* detail, size_t dn)
{
    if (got.diag_offsets != offs) {
        std::snprintf(detail, dn, "diagonal set differs (%d vs %zu)", got.num_diags, offs.size());
        return false;
    }
    const Dense G = to_dense(got);
    double worst = 0.0;
    for (size_t i = 0; i < G.size(); ++i) {
        const double tol = rel * bound[i] + 1e-30;
        worst = std::max(worst, std::fabs(G[i] - want[i]) / tol);
    }
    std::snprintf(detail, dn, "max err/tol %.3f", worst);
    return worst <= 1.0;
}

static void test_power(const char* name, int n, const std::vector<int>& offs, int k)
{
    const HMMatrix H = random_hm(n, offs, 11u + n);
    const diagpu::DeviceHM dH = diagpu::DeviceHM::upload(H);
    const HMMatrix P = diagpu::power(dH, k).download();
    const Dense Hd = to_dense(H), Ha = to_dense(H, true);
    Dense W = Hd, Wa = Ha;
    std::vector<int> o = offs;
    for (int j = 1; j < k; ++j) {
        W = matmul(W, Hd, n);
        Wa = matmul(Wa, Ha, n);
        o = sumset(o, offs, n);
    }
    char det[96];
    const bool ok = compare(P, W, Wa, 1e-5 * k, o, det, sizeof det);
    report(name, ok, det);
}

static void test_taylor(const char* name, int n, const std::vector<int>& offs, float t, int order)
{
    const HMMatrix H = random_hm(n, offs, 29u + n);
    const diagpu::DeviceHM dH = diagpu::DeviceHM::upload(H);
    const HMMatrix S = diagpu::taylor_expm(dH, t, order).download();
    const Dense Hd = to_dense(H), Ha = to_dense(H, true);
    const size_t nn = static_cast<size_t>(n) * n;
    Dense W(nn, 0.0), Wa(nn, 0.0), T(nn, 0.0), Ta(nn, 0.0);
    for (int i = 0; i < n; ++i) W[static_cast<size_t>(i) * n + i] = Wa[static_cast<size_t>(i) * n + i] = 1.0;
    T = W;
    Ta = Wa;
    std::set<int> all = {0};
    std::vector<int> o = {0};
    for (int k = 1; k <= order; ++k) {
        W = matmul(W, Hd, n);
        Wa = matmul(Wa, Ha, n);
        const double c = std::pow(static_cast<double>(t), k) / std::tgamma(k + 1.0);
        for (size_t i = 0; i < nn; ++i) {
            T[i] += c * W[i];
            Ta[i] += std::fabs(c) * Wa[i];
        }
        o = sumset(o, offs, n);
        all.insert(o.begin(), o.end());
    }
    char det[96];
    const bool ok = compare(S, T, Ta, 1e-5 * order, std::vector<int>(all.begin(), all.end()), det, sizeof det);
    report(name, ok, det);
}

static void test_axpby()
{
    const int n = 500;
    const HMMatrix X = random_hm(n, {-7, 0, 3}, 5), Y = random_hm(n, {-7, 1, 3, 400}, 6);
    const diagpu::DeviceHM dX = diagpu::DeviceHM::upload(X), dY = diagpu::DeviceHM::upload(Y);
    const HMMatrix Z = diagpu::axpby(0.5f, dX, -2.0f, &dY).download();
    const Dense Xd = to_dense(X), Yd = to_dense(Y), Xa = to_dense(X, true), Ya = to_dense(Y, true);
    Dense W(Xd.size()), B(Xd.size());
    for (size_t i = 0; i < W.size(); ++i) {
        W[i] = 0.5 * Xd[i] - 2.0 * Yd[i];
        B[i] = 0.5 * Xa[i] + 2.0 * Ya[i];
    }
    char det[96];
    const bool ok = compare(Z, W, B, 1.2e-7, {-7, 0, 1, 3, 400}, det, sizeof det);
    report("axpby on the union of diagonals", ok, det);
}

// The fused Horner step I + (a H) S (diagpu_spgemm_numeric_astat_scaled_f32:
// H scaled in LDS, I added to the product's main diagonal) against the
// unfused one (axpby, product, add_identity): the same offsets and bits, at
// an n the A-stationary kernel takes; with and without a main diagonal in
// the product (then I is added on the union, as unfused).
static void test_horner_fused(const char* name, int n, const std::vector<int>& ho,
                              const std::vector<int>& so)
{
    const HMMatrix Hh = random_hm(n, ho, 11), Sh = random_hm(n, so, 12);
    const diagpu::DeviceHM H = diagpu::DeviceHM::upload(Hh), S = diagpu::DeviceHM::upload(Sh);
    const float a = 0.37f;
    const diagpu::SpgemmPlan plan(n, H.off.data(), H.len.data(), H.starts.data(), H.ndiag(),
                                  S.off.data(), S.len.data(), S.starts.data(), S.ndiag());
    const HMMatrix F = diagpu::horner_step<float>(H, a, S).download();
    const diagpu::DeviceHM Hj = diagpu::axpby<float>(a, H, 0.0f, nullptr);
    diagpu::DeviceHM P = diagpu::multiply(Hj, S);
    diagpu::add_identity<float>(P, 1.0f);
    const HMMatrix U = P.download();
    const bool same = F.diag_offsets == U.diag_offsets && F.values.size() == U.values.size() &&
                      std::memcmp(F.values.data(), U.values.data(),
                                  F.values.size() * sizeof(float)) == 0;
    char det[96];
    std::snprintf(det, sizeof det, "A-stationary plan %d, %d C diagonals, %zu values",
                  (int)plan.uses_astat(), (int)F.diag_offsets.size(), F.values.size());
    report(name, same && plan.uses_astat(), det);
}

// ---- complex propagator ----------------------------------------------------

using cd = std::complex<double>;
using DenseC = std::vector<cd>;

// Hermitian band: diagonal +d random, -d its conjugate at the same positions,
// main diagonal real.  Offsets ascending; values back to back.
static void hermitian_band(int n, const std::vector<int>& pos, bool cplx, unsigned seed,
                           std::vector<int>& offs, std::vector<diagpu_complex64>& vals, DenseC& D)
{
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> U(-1.0f, 1.0f);
    std::set<int> all;
    for (int d : pos) { all.insert(d); all.insert(-d); }
    offs.assign(all.begin(), all.end());
    std::vector<std::vector<diagpu_complex64>> diag(offs.size());
    for (size_t k = 0; k < offs.size(); ++k) diag[k].resize(static_cast<size_t>(n - std::abs(offs[k])));
    auto index = [&](int d) { return static_cast<size_t>(std::lower_bound(offs.begin(), offs.end(), d) - offs.begin()); };
    for (int d : pos) {
        auto& up = diag[index(d)];
        auto& lo = diag[index(-d)];
        for (auto& v : up) v = diagpu_complex64{U(rng), (cplx && d != 0) ? U(rng) : 0.0f};
        for (size_t p = 0; p < up.size(); ++p) lo[p] = diagpu_complex64{up[p].re, -up[p].im};
    }
    vals.clear();
    D.assign(static_cast<size_t>(n) * n, cd(0.0));
    for (size_t k = 0; k < offs.size(); ++k) {
        const int d = offs[k];
        for (size_t p = 0; p < diag[k].size(); ++p) {
            const int r = static_cast<int>(p) - std::min(d, 0);
            D[static_cast<size_t>(r) * n + r + d] = cd(diag[k][p].re, diag[k][p].im);
            vals.push_back(diag[k][p]);
        }
    }
}

static DenseC matmul_c(const DenseC& A, const DenseC& B, int n)
{
    DenseC C(static_cast<size_t>(n) * n, cd(0.0));
    for (int i = 0; i < n; ++i)
        for (int k = 0; k < n; ++k) {
            const cd a = A[static_cast<size_t>(i) * n + k];
            if (a == cd(0.0)) continue;
            for (int j = 0; j < n; ++j) C[static_cast<size_t>(i) * n + j] += a * B[static_cast<size_t>(k) * n + j];
        }
    return C;
}

// sum_{k<terms} (s M)^k / k! in complex128 (||s M|| small)
static DenseC series(const DenseC& M, cd s, int n, int terms)
{
    DenseC S(static_cast<size_t>(n) * n, cd(0.0)), P(S);
    for (int i = 0; i < n; ++i) S[static_cast<size_t>(i) * n + i] = P[static_cast<size_t>(i) * n + i] = cd(1.0);
    for (int k = 1; k < terms; ++k) {
        P = matmul_c(P, M, n);
        for (auto& v : P) v *= s / static_cast<double>(k);
        for (size_t i = 0; i < S.size(); ++i) S[i] += P[i];
    }
    return S;
}

static DenseC hm_to_dense_c(const diagpu::DeviceHMC& M)
{
    const int n = M.n;
    const std::vector<diagpu_complex64> v = M.download_values();
    DenseC D(static_cast<size_t>(n) * n, cd(0.0));
    size_t q = 0;
    for (int d : M.offsets)
        for (int p = 0; p < n - std::abs(d); ++p, ++q) {
            const int r = p - std::min(d, 0);
            D[static_cast<size_t>(r) * n + r + d] = cd(v[q].re, v[q].im);
        }
    return D;
}

static void test_propagator(const char* name, int n, const std::vector<int>& pos, bool cplx,
                            float dt, int order)
{
    std::vector<int> offs;
    std::vector<diagpu_complex64> vals;
    DenseC Hd;
    hermitian_band(n, pos, cplx, 77u + n, offs, vals, Hd);
    diagpu::DeviceHMC U;
    if (cplx) {
        U = diagpu::propagator(diagpu::DeviceHMC::upload(n, offs, vals), dt, order);
    } else {   // a real H: promoted on the device
        std::vector<float> rv(vals.size());
        for (size_t i = 0; i < vals.size(); ++i) rv[i] = vals[i].re;
        U = diagpu::propagator(diagpu::DeviceHM::upload(n, offs, rv), dt, order);
    }
    const DenseC Ud = hm_to_dense_c(U);
    const DenseC want = series(Hd, cd(0.0, -dt), n, 40);
    DenseC Ha(Hd.size());
    double nrm = 0.0;   // ||dt H||_inf
    for (int i = 0; i < n; ++i) {
        double row = 0.0;
        for (int j = 0; j < n; ++j) {
            Ha[static_cast<size_t>(i) * n + j] = cd(std::abs(Hd[static_cast<size_t>(i) * n + j]));
            row += std::abs(Hd[static_cast<size_t>(i) * n + j]);
        }
        nrm = std::max(nrm, row * dt);
    }
    const DenseC bound = series(Ha, cd(dt, 0.0), n, 40);   // expm(dt |H|)
    double fact = 1.0;
    for (int k = 2; k <= order + 1; ++k) fact *= k;
    const double trunc = std::pow(nrm, order + 1) / fact * std::exp(nrm);
    double worst = 0.0;
    for (size_t i = 0; i < Ud.size(); ++i)
        worst = std::max(worst, std::abs(Ud[i] - want[i]) / (1e-5 * order * bound[i].real() + trunc + 1e-30));
    // unitarity
    double uni = 0.0;
    for (int i = 0; i < n; ++i)
        for (int j = 0; j < n; ++j) {
            cd s(0.0);
            for (int k = 0; k < n; ++k)
                s += Ud[static_cast<size_t>(i) * n + k] * std::conj(Ud[static_cast<size_t>(j) * n + k]);
            uni = std::max(uni, std::abs(s - cd(i == j ? 1.0 : 0.0)));
        }
    char det[96];
    std::snprintf(det, sizeof det, "max err/tol %.3f, |UU^H - I| %.1e", worst, uni);
    report(name, worst <= 1.0 && uni <= 1e-5, det);
}

// U in the Recon layout applied by the complex SpMV: against the dense
// product, and against the Lanczos propagator of the same H.
static void test_propagator_applied()
{
    const int n = 3000;   // H only as HM (no dense copy at this size)
    const float dt = 0.05f;
    const std::vector<int> pos = {0, 1, 2, 57};
    std::vector<int> offs;
    std::vector<diagpu_complex64> vals;
    {
        std::set<int> all;
        for (int d : pos) { all.insert(d); all.insert(-d); }
        offs.assign(all.begin(), all.end());
        std::mt19937 rng(11);
        std::uniform_real_distribution<float> U(-1.0f, 1.0f);
        std::vector<std::vector<diagpu_complex64>> diag(offs.size());
        for (size_t k = 0; k < offs.size(); ++k) diag[k].resize(static_cast<size_t>(n - std::abs(offs[k])));
        auto index = [&](int d) { return static_cast<size_t>(std::lower_bound(offs.begin(), offs.end(), d) - offs.begin()); };
        for (int d : pos) {
            auto& up = diag[index(d)];
            auto& lo = diag[index(-d)];
            for (auto& v : up) v = diagpu_complex64{U(rng), d ? U(rng) : 0.0f};
            for (size_t p = 0; p < up.size(); ++p) lo[p] = diagpu_complex64{up[p].re, -up[p].im};
        }
        for (auto& d : diag) vals.insert(vals.end(), d.begin(), d.end());
    }
    const diagpu::DeviceHMC H = diagpu::DeviceHMC::upload(n, offs, vals);
    const diagpu::DeviceHMC U = diagpu::propagator(H, dt, 8);
    const auto UR = diagpu::to_recon(U);
    const auto HR = diagpu::to_recon(H);
    // Recon layout: offsets descending, Recon[k][c] = U[c - d][c], zero padding
    const std::vector<int> ro = UR.offsets.download();
    const std::vector<diagpu_complex64> rv = UR.values.download();
    const std::vector<diagpu_complex64> uv = U.download_values();
    bool layout_ok = static_cast<int>(ro.size()) == U.ndiag();
    size_t q = 0;
    std::vector<size_t> start(U.offsets.size());
    for (size_t k = 0; k < U.offsets.size(); ++k) { start[k] = q; q += static_cast<size_t>(n - std::abs(U.offsets[k])); }
    for (int k = 0; layout_ok && k < U.ndiag(); ++k) {
        const int ks = U.ndiag() - 1 - k;
        const int d = U.offsets[ks];
        layout_ok = ro[k] == d;
        for (int c = 0; layout_ok && c < n; ++c) {
            const diagpu_complex64 g = rv[static_cast<size_t>(k) * n + c];
            const int r = c - d;
            diagpu_complex64 w{0.0f, 0.0f};
            if (r >= 0 && r < n) w = uv[start[ks] + static_cast<size_t>(std::min(r, c))];
            layout_ok = g.re == w.re && g.im == w.im;
        }
    }
    report("to_recon(U): build_recon layout, exact", layout_ok);

    std::mt19937 rng(3);
    std::normal_distribution<float> N(0.0f, 1.0f);
    std::vector<std::complex<float>> psi(static_cast<size_t>(n));
    for (auto& v : psi) v = {N(rng), N(rng)};
    diagpu::DeviceArray<std::complex<float>> dpsi(psi), dy(static_cast<size_t>(n)), dk(static_cast<size_t>(n));
    const diagpu_recon_view_c64 uview = diagpu::view(UR);
    diagpu::check(diagpu_spmv_recon_c64(&uview, reinterpret_cast<const diagpu_complex64*>(dpsi.data()), n,
                                        reinterpret_cast<diagpu_complex64*>(dy.data()), nullptr));
    diagpu::KrylovPropagator prop(n, 20);
    const diagpu::KrylovResult kr = prop.run(diagpu::view(HR), dpsi.data(), dt, dk.data());
    const std::vector<std::complex<float>> y = dy.download(), yk = dk.download();
    // U psi on the host from U's own values (fp64)
    std::vector<cd> yh(static_cast<size_t>(n), cd(0.0));
    for (size_t k = 0; k < U.offsets.size(); ++k) {
        const int d = U.offsets[k];
        for (int p = 0; p < n - std::abs(d); ++p) {
            const int r = p - std::min(d, 0);
            const diagpu_complex64 u = uv[start[k] + static_cast<size_t>(p)];
            yh[static_cast<size_t>(r)] += cd(u.re, u.im) * cd(psi[static_cast<size_t>(r + d)]);
        }
    }
    double e1 = 0.0, e2 = 0.0, np = 0.0, ny = 0.0;
    for (int i = 0; i < n; ++i) {
        e1 += std::norm(cd(y[i]) - yh[i]);
        e2 += std::norm(cd(y[i]) - cd(yk[i]));
        np += std::norm(cd(psi[i]));
        ny += std::norm(cd(y[i]));
    }
    e1 = std::sqrt(e1 / np);
    e2 = std::sqrt(e2 / np);
    const double unit = std::fabs(std::sqrt(ny / np) - 1.0);
    char det[128];
    std::snprintf(det, sizeof det, "vs U psi (fp64) %.1e, vs Lanczos %.1e, | ||U psi||/||psi|| - 1 | %.1e",
                  e1, e2, unit);
    report("U psi by the complex SpMV", e1 <= 1e-6 && e2 <= 2e-5 && unit <= 2e-5 && kr.steps > 0, det);
}

int main()
{
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    std::printf("Matrix-power chain and Taylor series on the GPU\n");
    try {
        test_axpby();
        test_power("H^5, band with main diagonal", 257, {-3, -1, 0, 1, 4}, 5);
        test_power("H^4, offsets {-2, 1} (no main diagonal)", 300, {-2, 1}, 4);
        test_power("H^3, wide offsets near n", 200, {-150, -2, 0, 7, 120}, 3);
        test_taylor("exp(0.2 H), order 10", 240, {-3, -1, 0, 1, 4}, 0.2f, 10);
        test_taylor("exp(0.5 H), order 8, no main diagonal", 180, {-2, 1}, 0.5f, 8);
        test_taylor("order 0 is the identity", 64, {-1, 1}, 1.0f, 0);
        test_propagator("exp(-i 0.05 H), complex Hermitian, order 10", 120, {0, 1, 3, 17}, true, 0.05f, 10);
        test_propagator("exp(-i 0.1 H), real H promoted, order 12", 96, {0, 2, 5}, false, 0.1f, 12);
        test_propagator_applied();
        test_horner_fused("fused Horner step, fp32 bits", 8192, {-3, -1, 0, 1, 4},
                          {-40, -2, 0, 5, 9, 33});
        test_horner_fused("fused Horner step, no main diagonal", 6000, {-2, 1}, {-5, 3});
    } catch (const std::exception& e) {
        std::printf("  exception: %s\n", e.what());
        g_all = false;
    }
    std::printf("\n%s\n", g_all ? "ALL TESTS PASSED" : "SOME TESTS FAILED");
    std::fflush(stdout);
    _exit(g_all ? 0 : 1);
}
