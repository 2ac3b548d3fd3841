// GPU test of include/diagpu/krylov.hpp: exp(-i t H) psi_0 by the device
// Lanczos propagator, for a complex Hermitian band (complex64 Recon) and for
// a real symmetric band built with the drop-in DiaMatrix / build_recon /
// ReconView API, checked against a host complex128 Taylor series of the same
// dense matrix (an independent algorithm: sum_k (-i t H)^k psi_0 / k!, 80
// terms, so its truncation is far below fp32 rounding):
//   ||psi - psi_ref|| <= 1e-4 ||psi_0||.
#include <cmath>
#include <complex>
#include <cstdio>
#include <random>
#include <vector>

#include "diagpu/dia.hpp"
#include "diagpu/krylov.hpp"

using cd = std::complex<double>;
using cf = std::complex<float>;

static bool g_all = true;

static void report(const char* name, bool ok, const char* detail = "")
{
    std::printf("  %-48s %s %s\n", name, ok ? "[OK]" : "[FAIL]", detail);
    g_all &= ok;
}

// psi(t) = sum_k (-i t H)^k psi0 / k! with dense complex128 H (n x n)
static std::vector<cd> taylor_ref(int n, const std::vector<cd>& H, const std::vector<cd>& psi0,
                                  double t)
{
    std::vector<cd> term = psi0, out = psi0, next(n);
    for (int k = 1; k <= 80; ++k) {
        for (int r = 0; r < n; ++r) {
            cd s = 0.0;
            for (int c = 0; c < n; ++c) s += H[(size_t)r * n + c] * term[c];
            next[r] = s * cd(0.0, -t) / double(k);
        }
        term.swap(next);
        for (int r = 0; r < n; ++r) out[r] += term[r];
    }
    return out;
}

static double rel_err(const std::vector<cf>& got, const std::vector<cd>& want, const std::vector<cf>& psi0)
{
    double e = 0.0, nn = 0.0;
    for (size_t i = 0; i < got.size(); ++i) {
        e += std::norm(cd(got[i]) - want[i]);
        nn += std::norm(cd(psi0[i]));
    }
    return std::sqrt(e / nn);
}

int main()
{
    const int n = 300;
    const double t = 0.6;
    std::mt19937 rng(11);
    std::uniform_real_distribution<double> U(-1.0, 1.0);
    std::vector<cf> psi0(n);
    for (auto& v : psi0) v = cf((float)U(rng), (float)U(rng));
    std::vector<cd> psi0d(psi0.begin(), psi0.end());
    diagpu::DeviceArray<cf> d_psi0(psi0), d_out(n);
    diagpu::KrylovPropagator prop(n, 40);

    // complex Hermitian band, offsets +-{0, 1, 4, 29}; Recon[k][c] = H[c - d, c]
    {
        const std::vector<int> offs = {29, 4, 1, 0, -1, -4, -29};
        std::vector<cd> H((size_t)n * n, 0.0);
        for (int d : {0, 1, 4, 29})
            for (int r = 0; r + d < n; ++r) {
                const cf h = d == 0 ? cf((float)(2 * U(rng)), 0.f) : cf((float)U(rng), (float)U(rng));
                H[(size_t)r * n + r + d] = cd(h);
                H[(size_t)(r + d) * n + r] = std::conj(cd(h));
            }
        std::vector<cf> vals(offs.size() * (size_t)n, cf(0.f, 0.f));
        for (size_t k = 0; k < offs.size(); ++k)
            for (int c = 0; c < n; ++c) {
                const int r = c - offs[k];
                if (r >= 0 && r < n) vals[k * n + c] = cf(H[(size_t)r * n + c]);
            }
        diagpu::DeviceArray<int> d_off(offs);
        diagpu::DeviceArray<cf> d_vals(vals);
        diagpu_recon_view_c64 view{n, n, (int)offs.size(), d_off.data(),
                                   reinterpret_cast<const diagpu_complex64*>(d_vals.data())};
        diagpu::KrylovResult r = prop.run(view, d_psi0.data(), t, d_out.data());
        diagpu::check_hip(hipDeviceSynchronize(), "sync");
        const double e = rel_err(d_out.download(), taylor_ref(n, H, psi0d, t), psi0);
        char buf[128];
        std::snprintf(buf, sizeof buf, "(rel err %.2e, %d steps, est %.1e)", e, r.steps, r.err_estimate);
        report("complex Hermitian band vs Taylor series", e <= 1e-4 && r.steps == 40, buf);
    }

    // real symmetric band through the drop-in API: DiaMatrix -> build_recon -> ReconView
    {
        DiaMatrix D;
        D.rows = D.cols = n;
        std::vector<cd> H((size_t)n * n, 0.0);
        for (int d : {-7, -2, 0, 2, 7}) {
            D.offsets.push_back(d);
            D.diag_starts.push_back(0);
            D.diag_lengths.push_back(n - std::abs(d));
        }
        // symmetric values: H[r, r + d] = H[r + d, r]
        for (int d : {0, 2, 7})
            for (int r = 0; r + d < n; ++r) {
                const double h = d == 0 ? 2 * U(rng) : U(rng);
                H[(size_t)r * n + r + d] = H[(size_t)(r + d) * n + r] = (double)(float)h;
            }
        for (size_t k = 0; k < D.offsets.size(); ++k) {
            const int d = D.offsets[k];
            D.diag_starts[k] = (int)D.values.size();
            const int sr = d < 0 ? -d : 0, sc = d > 0 ? d : 0;
            for (int j = 0; j < D.diag_lengths[k]; ++j)
                D.values.push_back((float)H[(size_t)(sr + j) * n + sc + j].real());
        }
        ReconMatrix R = build_recon(D);
        diagpu::DeviceRecon dR(R);
        diagpu::KrylovResult r = prop.run(dR.view, d_psi0.data(), t, d_out.data(), nullptr, 25);
        diagpu::check_hip(hipDeviceSynchronize(), "sync");
        const double e = rel_err(d_out.download(), taylor_ref(n, H, psi0d, t), psi0);
        char buf[128];
        std::snprintf(buf, sizeof buf, "(rel err %.2e, %d steps)", e, r.steps);
        report("real symmetric band (ReconView) vs Taylor series", e <= 1e-4 && r.steps == 25, buf);
        bool threw = false;
        try {
            prop.run(dR.view, d_psi0.data(), t, d_out.data(), nullptr, 41);
        } catch (const diagpu::Error& ex) {
            threw = ex.status == DIAGPU_ERR_ARG;
        }
        report("more steps than the workspace throws", threw);
    }

    std::printf(g_all ? "ALL TESTS PASSED\n" : "SOME TESTS FAILED\n");
    std::fflush(stdout);
    std::_Exit(g_all ? 0 : 1);
}
