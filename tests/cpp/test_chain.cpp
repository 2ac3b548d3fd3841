// GPU test of include/diagpu/chain.hpp: matrix powers and the truncated
// Taylor series built by the device-planned SpGEMM chain, checked against
// dense float64 products on the host:
//   |P - P64| <= 1e-5 * k * (|H|^k)  elementwise (k products of fp32 sums),
// and the result's diagonal set equals the sumset of H's offsets.
#include <unistd.h>

#include <cmath>
#include <cstdio>
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
    } catch (const std::exception& e) {
        std::printf("  exception: %s\n", e.what());
        g_all = false;
    }
    std::printf("\n%s\n", g_all ? "ALL TESTS PASSED" : "SOME TESTS FAILED");
    std::fflush(stdout);
    _exit(g_all ? 0 : 1);
}
