// exp(-i t H) psi_0 by Lanczos on the GPU, for Hermitian H in the Recon
// layout (spmv/src/dia_reconstruct.cuh:9-17): the matrix-free SpMV caller of
// slides/transcript.md:10-18, which the reference does not ship.
//
//   diagpu::KrylovPropagator prop(n, 30);              // workspace for m <= 30
//   diagpu::KrylovResult r = prop.run(H, d_psi0, t, d_psi_t, stream);
//
// H is a diagpu_recon_view_c64 (complex values) or a ReconView /
// diagpu_recon_view_f32 (real symmetric values applied to the complex
// state).  d_psi0 and d_psi_t are device arrays of n std::complex<float>.
// run() synchronises `stream` once (after the Lanczos steps) and returns with
// the final combine kernel queued on it.
#pragma once

#include <complex>
#include <memory>
#include <vector>

#include "common.hpp"

namespace diagpu {

struct KrylovResult {
    int steps = 0;               // Lanczos steps used
    bool breakdown = false;      // invariant subspace reached: result exact
    double psi0_norm = 0.0;
    double err_estimate = 0.0;   // ||psi_0|| beta_m |[exp(-i t T_m)]_{m,1}|
    std::vector<double> alpha;   // T_m diagonal
    std::vector<double> beta;    // T_m off-diagonal
};

class KrylovPropagator {
public:
    KrylovPropagator(int32_t n, int32_t max_steps) : n_(n), m_(max_steps)
    {
        size_t bytes = 0;
        check(diagpu_expm_krylov_workspace(n, max_steps, &bytes));
        ws_.resize(bytes);
        double* h = nullptr;   // pinned: T_m's entries come back without a staged copy
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&h), (2 * static_cast<size_t>(max_steps) + 1) * sizeof(double)),
                  "hipHostMalloc");
        host_.reset(h);
    }

    int32_t n() const { return n_; }
    int32_t max_steps() const { return m_; }

    KrylovResult run(const diagpu_recon_view_c64& H, const std::complex<float>* d_psi0, double t,
                     std::complex<float>* d_psi_t, hipStream_t stream = nullptr, int32_t m = 0)
    {
        return finish(m, [&](int32_t mm, double* a, double* b, diagpu_krylov_info* info) {
            return diagpu_expm_krylov_c64(&H, as_c(d_psi0), t, mm, as_c(d_psi_t), ws_.data(),
                                          ws_.size(), host_.get(), a, b, info, stream);
        });
    }

    template <typename View>   // diagpu_recon_view_f32 or the drop-in ReconView
    KrylovResult run(const View& H, const std::complex<float>* d_psi0, double t,
                     std::complex<float>* d_psi_t, hipStream_t stream = nullptr, int32_t m = 0)
    {
        static_assert(sizeof(View) == sizeof(diagpu_recon_view_f32),
                      "a real Recon view has the members of diagpu_recon_view_f32");
        return finish(m, [&](int32_t mm, double* a, double* b, diagpu_krylov_info* info) {
            return diagpu_expm_krylov_f32(reinterpret_cast<const diagpu_recon_view_f32*>(&H),
                                          as_c(d_psi0), t, mm, as_c(d_psi_t), ws_.data(),
                                          ws_.size(), host_.get(), a, b, info, stream);
        });
    }

private:
    static const diagpu_complex64* as_c(const std::complex<float>* p)
    {
        return reinterpret_cast<const diagpu_complex64*>(p);
    }
    static diagpu_complex64* as_c(std::complex<float>* p)
    {
        return reinterpret_cast<diagpu_complex64*>(p);
    }

    template <typename Call>
    KrylovResult finish(int32_t m, Call call)
    {
        const int32_t mm = m > 0 ? m : m_;
        if (mm > m_) throw Error(DIAGPU_ERR_ARG, "KrylovPropagator: more steps than the workspace holds");
        KrylovResult r;
        r.alpha.assign(mm, 0.0);
        r.beta.assign(mm, 0.0);
        diagpu_krylov_info info{};
        check(call(mm, r.alpha.data(), r.beta.data(), &info));
        r.steps = info.steps;
        r.breakdown = info.breakdown != 0;
        r.psi0_norm = info.psi0_norm;
        r.err_estimate = info.err_estimate;
        r.alpha.resize(info.steps);
        r.beta.resize(info.steps);
        return r;
    }

    struct PinnedFree {
        void operator()(double* p) const { (void)hipHostFree(p); }
    };

    int32_t n_, m_;
    DeviceArray<unsigned char> ws_;
    std::unique_ptr<double, PinnedFree> host_;
};

}  // namespace diagpu
