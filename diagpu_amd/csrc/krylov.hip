// Krylov propagator psi(t) = exp(-i t H) psi_0 for a Hermitian H in the Recon
// layout (Lanczos), on the SpMV kernels of spmv.hip.
//
// This is the matrix-free caller the reference's SpMV exists for
// (slides/transcript.md:10-18: "apply H to the state vector, then apply H
// again ... exactly what Krylov-subspace methods do"); the reference ships no
// driver for it.
//
// Lanczos with unnormalised basis vectors.  v_j = u_j / s_j with s_1 =
// ||psi_0|| (u_1 = psi_0 itself, never copied) and s_{j+1} = beta_j.  Step j:
//   z  = H u_j                            SpMV with the fused dot epilogue:
//   d_j = Re <u_j, z>                     alpha_j = d_j / s_j^2
//   u_{j+1} = (z - alpha_j u_j) / s_j - (s_j / s_{j-1}) u_{j-1}
//   q_j = ||u_{j+1}||^2                   beta_j = s_{j+1} = sqrt(q_j)
// i.e. the three-term recurrence H v_j = beta_{j-1} v_{j-1} + alpha_j v_j +
// beta_j v_{j+1} without a separate normalisation pass: two kernels per step
// (SpMV+dot, update+norm), z is written into u_{j+1}'s slot and updated in
// place, and every scalar stays on the device.  Each reduction is one fp64
// partial per workgroup plus a one-workgroup fixed-order sum (reduce.hpp,
// sum_partials): deterministic, and free of device-scope fences.  q_j is
// not needed before step j+1's update, so its sum shares one launch with
// step j+1's d sum (sum_partials2): three launches per step.
//
// After m steps the host reads alpha and beta (the only synchronisation, one
// copy), forms T_m = tridiag(beta, alpha, beta) and evaluates
// c = exp(-i t T_m) e_1 in fp64 (expm_tridiag_e1: scaled Taylor steps on the
// tridiagonal, scaling and squaring for large t, no eigendecomposition).  One combine kernel then writes
// psi(t) = ||psi_0|| sum_j c_j v_j.  A beta_j that vanishes relative to
// |alpha_j| + beta_{j-1} marks an invariant subspace: the expansion stops
// there and is exact (up to rounding).  The a posteriori error estimate
// ||psi_0|| beta_m |c_m| is returned.
#include <cmath>
#include <complex>
#include <vector>

#include "common.hpp"
#include "expm_tridiag.hpp"
#include "reduce.hpp"
#include "spmv_internal.hpp"

namespace diagpu {
namespace {

constexpr int kVB = 256;          // lanes per workgroup of the vector kernels
constexpr int kVR = 2;            // complex elements per lane (16 bytes)
constexpr int kVTile = kVB * kVR;
constexpr int kMaxSteps = 64;

typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

inline __device__ int vec_tile(int per_xcd)
{
    const int x = (int)(blockIdx.x % kNumXcd);
    const int l = (int)(blockIdx.x / kNumXcd);
    return x * per_xcd + ((x & 1) ? per_xcd - 1 - l : l);
}

inline __device__ void ld2(const cf32* p, int64_t i, int64_t n, cf32 (&v)[kVR])
{
    if (i + kVR <= n) {
        const f4u q = *reinterpret_cast<const f4u*>(p + i);
        v[0] = cf32{q.x, q.y};
        v[1] = cf32{q.z, q.w};
    } else {
#pragma unroll
        for (int e = 0; e < kVR; ++e) v[e] = i + e < n ? p[i + e] : cf32{0.f, 0.f};
    }
}

inline __device__ void st2(cf32* p, int64_t i, int64_t n, const cf32 (&v)[kVR])
{
    if (i + kVR <= n) {
        const f4u q = {v[0].re, v[0].im, v[1].re, v[1].im};
        *reinterpret_cast<f4u*>(p + i) = q;
    } else {
#pragma unroll
        for (int e = 0; e < kVR; ++e)
            if (i + e < n) p[i + e] = v[e];
    }
}

// partials[tile] = this workgroup's part of ||x||^2
__global__ __launch_bounds__(kVB) void k_norm2(const cf32* __restrict__ x, int64_t n, int tiles,
                                              int per_xcd, double* partials)
{
    const int tile = vec_tile(per_xcd);
    if (tile >= tiles) return;
    const int64_t i = (int64_t)tile * kVTile + (int64_t)threadIdx.x * kVR;
    cf32 v[kVR];
    ld2(x, i, n, v);
    double s = 0.0;
#pragma unroll
    for (int e = 0; e < kVR; ++e) s += (double)v[e].re * v[e].re + (double)v[e].im * v[e].im;
    store_partial<kVB>(s, tile, partials);
}

// Step j (1-based) update in place over zw (holding z = H u_j):
//   zw = (z - alpha_j u_j) / s_j - (s_j / s_{j-1}) u_{j-1}
// and this workgroup's part of q[j] = ||zw||^2 into partials[tile].
// alpha_j = d[j-1] / q[j-1], s_j = sqrt(q[j-1]), s_{j-1} = sqrt(q[j-2]).
// A zero s_j (breakdown before this step) writes zeros.
__global__ __launch_bounds__(kVB) void k_lanczos_update(cf32* __restrict__ zw,
                                                       const cf32* __restrict__ uj,
                                                       const cf32* __restrict__ ujm1, int64_t n,
                                                       int j, const double* __restrict__ d,
                                                       const double* q, int tiles, int per_xcd,
                                                       double* partials)
{
    const int tile = vec_tile(per_xcd);
    if (tile >= tiles) return;
    const double qj = q[j - 1];
    const double sj = sqrt(qj);
    const float inv_s = qj > 0.0 ? (float)(1.0 / sj) : 0.f;
    const float alpha = qj > 0.0 ? (float)(d[j - 1] / qj) : 0.f;
    float ratio = 0.f;   // s_j / s_{j-1} = beta_{j-1} / s_{j-1}
    if (j >= 2) {
        const double qm = q[j - 2];
        ratio = qm > 0.0 ? (float)(sj / sqrt(qm)) : 0.f;
    }
    const int64_t i = (int64_t)tile * kVTile + (int64_t)threadIdx.x * kVR;
    cf32 z[kVR], u[kVR], w[kVR];
    ld2(zw, i, n, z);
    ld2(uj, i, n, u);
    if (j >= 2) ld2(ujm1, i, n, w);
    double s = 0.0;
#pragma unroll
    for (int e = 0; e < kVR; ++e) {
        float re = __builtin_fmaf(-alpha, u[e].re, z[e].re) * inv_s;
        float im = __builtin_fmaf(-alpha, u[e].im, z[e].im) * inv_s;
        if (j >= 2) {
            re = __builtin_fmaf(-ratio, w[e].re, re);
            im = __builtin_fmaf(-ratio, w[e].im, im);
        }
        z[e] = cf32{re, im};
        s += (double)re * re + (double)im * im;
    }
    st2(zw, i, n, z);
    store_partial<kVB>(s, tile, partials);
}

struct Coefs {
    cf32 g[kMaxSteps];
};

// out = sum_{j < m} g_j u_j, u_0 = first, u_j = rest + (j - 1) n
__global__ __launch_bounds__(kVB) void k_combine(const cf32* __restrict__ first,
                                                const cf32* __restrict__ rest, int64_t n, int m,
                                                Coefs c, cf32* __restrict__ out, int tiles,
                                                int per_xcd)
{
    const int tile = vec_tile(per_xcd);
    if (tile >= tiles) return;
    const int64_t i = (int64_t)tile * kVTile + (int64_t)threadIdx.x * kVR;
    cf32 acc[kVR] = {cf32{0.f, 0.f}, cf32{0.f, 0.f}};
    for (int j = 0; j < m; ++j) {
        cf32 u[kVR];
        ld2(j == 0 ? first : rest + (int64_t)(j - 1) * n, i, n, u);
        const cf32 g = c.g[j];
#pragma unroll
        for (int e = 0; e < kVR; ++e) {
            acc[e].re = __builtin_fmaf(-g.im, u[e].im, __builtin_fmaf(g.re, u[e].re, acc[e].re));
            acc[e].im = __builtin_fmaf(g.im, u[e].re, __builtin_fmaf(g.re, u[e].im, acc[e].im));
        }
    }
    st2(out, i, n, acc);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct Layout {
    size_t vecs, pd, pq, d, q, total;   // pd: SpMV dot partials, pq: norm partials
};

Layout layout(int64_t n, int m)
{
    Layout L;
    // one partial per workgroup of the largest launch: either SpMV (real or
    // complex matrix) or the vector kernels
    int64_t tiles = spmv_tiles<float, cf32>((int32_t)n);
    const int64_t tc = spmv_tiles<cf32, cf32>((int32_t)n);
    const int64_t tv = (n + kVTile - 1) / kVTile;
    tiles = tc > tiles ? tc : tiles;
    tiles = tv > tiles ? tv : tiles;
    size_t off = 0;
    L.vecs = off;
    off += align256((size_t)m * (size_t)n * sizeof(cf32));
    L.pd = off;
    off += align256((size_t)tiles * sizeof(double));
    L.pq = off;
    off += align256((size_t)tiles * sizeof(double));
    L.d = off;   // d[m] and q[m+1] back to back: one copy to the host
    L.q = off + (size_t)m * sizeof(double);
    off += align256((size_t)(2 * m + 1) * sizeof(double));
    L.total = off;
    return L;
}

template <typename TV>
int expm_krylov(int32_t rows, int32_t cols, int32_t K, const int32_t* offs, const TV* vals,
                const cf32* psi0, double t, int32_t m, cf32* psi_t, void* workspace,
                size_t ws_bytes, double* host_scratch, double* alpha_out, double* beta_out,
                diagpu_krylov_info* info,
                void* stream, const char* fn)
{
    if (rows != cols || rows < 1)
        return fail(DIAGPU_ERR_ARG, "%s: H must be square with n >= 1 (rows=%d cols=%d)", fn,
                    rows, cols);
    if (m < 1 || m > kMaxSteps)
        return fail(DIAGPU_ERR_ARG, "%s: m=%d outside [1, %d]", fn, m, kMaxSteps);
    if (!psi0 || !psi_t || !workspace)
        return fail(DIAGPU_ERR_ARG, "%s: psi0, psi_t or workspace is NULL", fn);
    if (!std::isfinite(t)) return fail(DIAGPU_ERR_ARG, "%s: t is not finite", fn);
    const int64_t n = rows;
    const Layout L = layout(n, m);
    if (ws_bytes < L.total)
        return fail(DIAGPU_ERR_CAPACITY, "%s: workspace %zu bytes, needs %zu", fn, ws_bytes,
                    L.total);
    char* ws = static_cast<char*>(workspace);
    cf32* vecs = reinterpret_cast<cf32*>(ws + L.vecs);
    double* pd = reinterpret_cast<double*>(ws + L.pd);
    double* pq = reinterpret_cast<double*>(ws + L.pq);
    double* d = reinterpret_cast<double*>(ws + L.d);
    double* q = reinterpret_cast<double*>(ws + L.q);
    hipStream_t s = as_stream(stream);
    auto slot = [&](int j) { return vecs + (int64_t)(j - 2) * n; };   // u_j, j >= 2

    const int vtiles = (int)((n + kVTile - 1) / kVTile);
    const int vper = (vtiles + kNumXcd - 1) / kNumXcd;
    const dim3 vgrid((unsigned)(vper * kNumXcd));

    const int stiles = spmv_tiles<TV, cf32>(rows);

    // pq holds the partials of q[j-1] when step j starts (||psi_0||^2 for j = 1)
    hipLaunchKernelGGL(k_norm2, vgrid, dim3(kVB), 0, s, psi0, n, vtiles, vper, pq);
    int st = check_launch(fn);
    if (st) return st;
    for (int j = 1; j <= m; ++j) {
        const cf32* uj = j == 1 ? psi0 : slot(j);
        const cf32* ujm1 = j == 1 ? nullptr : (j == 2 ? psi0 : slot(j - 1));
        DotArgs da{pd, nullptr};
        st = spmv_run<TV, cf32>(rows, cols, K, offs, vals, uj, n, slot(j + 1), &da, stream, fn);
        if (!st) st = sum_partials2(pd, stiles, d + (j - 1), pq, vtiles, q + (j - 1), stream);
        if (st) return st;
        hipLaunchKernelGGL(k_lanczos_update, vgrid, dim3(kVB), 0, s, slot(j + 1), uj, ujm1, n, j,
                           d, q, vtiles, vper, pq);
        st = check_launch(fn);
        if (st) return st;
    }
    st = sum_partials(pq, vtiles, q + m, stream);
    if (st) return st;
    // d and q to the host: into the caller's pinned buffer when given (the
    // copy is queued like a kernel), else through a pageable vector (the HIP
    // runtime stages that copy; it measured 80+ us of GPU idle time)
    std::vector<double> pageable;
    double* hdq = host_scratch;
    if (!hdq) {
        pageable.resize(2 * (size_t)m + 1);
        hdq = pageable.data();
    }
    st = check_hip(hipMemcpyAsync(hdq, d, sizeof(double) * (2 * (size_t)m + 1),
                                  hipMemcpyDeviceToHost, s), fn);
    if (!st) st = check_hip(hipStreamSynchronize(s), fn);
    if (st) return st;
    const double* hd = hdq;
    const double* hq = hdq + m;

    // T_m and the number of usable steps
    const double nrm0 = std::sqrt(hq[0]);
    std::vector<double> al(m), be(m);
    int meff = 0;
    bool breakdown = false;
    if (hq[0] > 0.0) {
        for (int j = 1; j <= m; ++j) {
            al[j - 1] = hd[j - 1] / hq[j - 1];
            be[j - 1] = std::sqrt(hq[j]);
            meff = j;
            const double scale = std::fabs(al[j - 1]) + (j >= 2 ? be[j - 2] : 0.0);
            if (!(be[j - 1] > 1e-6 * scale)) {   // also catches NaN
                breakdown = j < m || !(be[j - 1] > 0.0);
                break;
            }
        }
    }
    Coefs cf{};
    double err = 0.0;
    if (meff > 0) {
        std::vector<std::complex<double>> c;
        if (!expm_tridiag_e1(meff, al, be, t, c))
            return fail(DIAGPU_ERR_ARG, "%s: t T_m is not finite (|t| = %g)", fn, std::fabs(t));
        for (int j = 1; j <= meff; ++j) {
            // psi(t) = ||psi0|| sum c_j v_j, v_j = u_j / s_j, s_j = sqrt(q[j-1])
            const std::complex<double> g = nrm0 * c[j - 1] / std::sqrt(hq[j - 1]);
            cf.g[j - 1] = cf32{(float)g.real(), (float)g.imag()};
        }
        if (!breakdown) err = nrm0 * be[meff - 1] * std::abs(c[meff - 1]);
    }
    hipLaunchKernelGGL(k_combine, vgrid, dim3(kVB), 0, s, psi0, vecs, n, meff, cf, psi_t, vtiles,
                       vper);
    st = check_launch(fn);
    if (st) return st;
    if (alpha_out)
        for (int j = 0; j < m; ++j) alpha_out[j] = j < meff ? al[j] : 0.0;
    if (beta_out)
        for (int j = 0; j < m; ++j) beta_out[j] = j < meff ? be[j] : 0.0;
    if (info) {
        info->steps = meff;
        info->breakdown = breakdown ? 1 : 0;
        info->psi0_norm = nrm0;
        info->err_estimate = err;
    }
    return DIAGPU_OK;
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_expm_krylov_workspace(int32_t n, int32_t m, size_t* bytes)
{
    const char* fn = "diagpu_expm_krylov_workspace";
    if (!bytes) return diagpu::fail(DIAGPU_ERR_ARG, "%s: bytes is NULL", fn);
    if (n < 1 || m < 1 || m > diagpu::kMaxSteps)
        return diagpu::fail(DIAGPU_ERR_ARG, "%s: n=%d m=%d (need n >= 1, 1 <= m <= %d)", fn, n, m,
                            diagpu::kMaxSteps);
    *bytes = diagpu::layout(n, m).total;
    return DIAGPU_OK;
}

DIAGPU_API int diagpu_expm_krylov_c64(const diagpu_recon_view_c64* H,
                                      const diagpu_complex64* psi0, double t, int32_t m,
                                      diagpu_complex64* psi_t, void* workspace,
                                      size_t workspace_bytes, double* host_scratch, double* alpha,
                                      double* beta, diagpu_krylov_info* info, void* stream)
{
    using diagpu::cf32;
    const char* fn = "diagpu_expm_krylov_c64";
    if (!H) return diagpu::fail(DIAGPU_ERR_ARG, "%s: H is NULL", fn);
    return diagpu::expm_krylov<cf32>(H->rows, H->cols, H->num_diags, H->diag_offsets,
                                     reinterpret_cast<const cf32*>(H->values),
                                     reinterpret_cast<const cf32*>(psi0), t, m,
                                     reinterpret_cast<cf32*>(psi_t), workspace, workspace_bytes,
                                     host_scratch, alpha, beta, info, stream, fn);
}

DIAGPU_API int diagpu_expm_krylov_f32(const diagpu_recon_view_f32* H,
                                      const diagpu_complex64* psi0, double t, int32_t m,
                                      diagpu_complex64* psi_t, void* workspace,
                                      size_t workspace_bytes, double* host_scratch, double* alpha,
                                      double* beta, diagpu_krylov_info* info, void* stream)
{
    using diagpu::cf32;
    const char* fn = "diagpu_expm_krylov_f32";
    if (!H) return diagpu::fail(DIAGPU_ERR_ARG, "%s: H is NULL", fn);
    return diagpu::expm_krylov<float>(H->rows, H->cols, H->num_diags, H->diag_offsets, H->values,
                                      reinterpret_cast<const cf32*>(psi0), t, m,
                                      reinterpret_cast<cf32*>(psi_t), workspace, workspace_bytes,
                                      host_scratch, alpha, beta, info, stream, fn);
}

}  // extern "C"
