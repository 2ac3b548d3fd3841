// Matrix-power chain and truncated Taylor series for HM (compact diagonal)
// matrices on the GPU: the caller of the SpGEMM hot path that the reference
// describes but does not ship (spmspm/gather_flat.cuh:13-14, 110-117: a chain
// P_{k+1} = P_k * H whose plan is rebuilt on the device every step).
// power() is that chain; taylor_expm() runs the same kind of chain in Horner
// form, so that no step needs a full pass to add the powers together.
//
// Values are fp32 (DeviceHM) or complex64 (DeviceHMC: complex Hamiltonians,
// which the reference's real kernels do not cover).  propagator() builds
// U = exp(-i dt H) as an explicit complex matrix, and to_recon() hands any
// of these matrices to the SpMV kernels (build_recon on the device), so that
// U is built once and applied to many states.
//
// Each product builds its C structure and pair plan with the device symbolic
// phase (one stream sync returns the counts), then runs the numeric phase.
// Sums and scalings run diagpu_dia_axpby_f32 / _c64 over the union of the
// operands' diagonals; the union is a merge of two short sorted offset lists
// on the host, which holds a copy of every matrix's offsets.
#pragma once

#include <algorithm>
#include <complex>
#include <cstdlib>
#include <iterator>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "spgemm.hpp"

namespace diagpu {

// Per value type: the scalar type of factors and the entry points.
template <typename T> struct HMValue;

template <> struct HMValue<float> {
    using scalar = float;
    static float to_c(scalar s) { return s; }
    static int axpby(int n, const int* xo, const int64_t* xs, int nx, const float* xv, scalar a,
                     const int* yo, const int64_t* ys, int ny, const float* yv, scalar b,
                     const int* zo, const int64_t* zs, int nz, float* zv, hipStream_t st)
    {
        return diagpu_dia_axpby_f32(n, xo, xs, nx, xv, a, yo, ys, ny, yv, b, zo, zs, nz, zv, st);
    }
    static int to_recon(int n, const int* o, const int64_t* s, int k, const float* v, int* ro,
                        float* rv, hipStream_t st)
    {
        return diagpu_hm_to_recon_f32(n, o, s, k, v, ro, rv, st);
    }
};

template <> struct HMValue<diagpu_complex64> {
    using scalar = std::complex<float>;
    static diagpu_complex64 to_c(scalar s) { return diagpu_complex64{s.real(), s.imag()}; }
    static int axpby(int n, const int* xo, const int64_t* xs, int nx, const diagpu_complex64* xv,
                     scalar a, const int* yo, const int64_t* ys, int ny,
                     const diagpu_complex64* yv, scalar b, const int* zo, const int64_t* zs,
                     int nz, diagpu_complex64* zv, hipStream_t st)
    {
        return diagpu_dia_axpby_c64(n, xo, xs, nx, xv, to_c(a), yo, ys, ny, yv, to_c(b), zo, zs,
                                    nz, zv, st);
    }
    static int to_recon(int n, const int* o, const int64_t* s, int k, const diagpu_complex64* v,
                        int* ro, diagpu_complex64* rv, hipStream_t st)
    {
        return diagpu_hm_to_recon_c64(n, o, s, k, v, ro, rv, st);
    }
};

template <typename T> using HMScalar = typename HMValue<T>::scalar;

// Device-resident square HM matrix; `offsets` is the host copy (ascending).
template <typename T>
struct DeviceHMT {
    int n = 0;
    std::vector<int> offsets;
    int64_t nnz = 0;
    DeviceArray<int> off, len;
    DeviceArray<int64_t> starts;
    DeviceArray<T> vals;

    int ndiag() const { return static_cast<int>(offsets.size()); }

    // Structure for the given offsets (ascending, distinct, |d| < n); values
    // allocated, not initialised.
    static DeviceHMT with_offsets(int n, const std::vector<int>& offs)
    {
        DeviceHMT M;
        M.n = n;
        M.offsets = offs;
        std::vector<int> lens(offs.size());
        std::vector<int64_t> st(offs.size());
        for (size_t i = 0; i < offs.size(); ++i) {
            if ((i && offs[i] <= offs[i - 1]) || offs[i] <= -n || offs[i] >= n)
                throw Error(DIAGPU_ERR_OFFSET, "DeviceHM: offsets must be ascending, distinct, |d| < n");
            lens[i] = n - std::abs(offs[i]);
            st[i] = M.nnz;
            M.nnz += lens[i];
        }
        M.off.upload(offs);
        M.len.upload(lens);
        M.starts.upload(st);
        M.vals.resize(static_cast<size_t>(M.nnz));
        return M;
    }

    // Offsets (ascending) and their values back to back, n - |d| per diagonal.
    static DeviceHMT upload(int n, const std::vector<int>& offs, const std::vector<T>& values)
    {
        DeviceHMT M = with_offsets(n, offs);
        if (values.size() < static_cast<size_t>(M.nnz))
            throw Error(DIAGPU_ERR_ARG, "DeviceHM::upload: too few values");
        M.vals.upload(std::vector<T>(values.begin(), values.begin() + M.nnz));
        return M;
    }

    // The reference's host HM matrix (fp32 only).
    static DeviceHMT upload(const HMMatrix& H)
    {
        static_assert(std::is_same<T, float>::value, "HMMatrix holds fp32 values");
        int64_t s = 0;
        for (int i = 0; i < H.num_diags; ++i) {
            if (H.diag_starts[i] != s)
                throw Error(DIAGPU_ERR_ARG, "DeviceHM::upload: starts must be the prefix sum of lengths");
            s += H.n - std::abs(H.diag_offsets[i]);
        }
        return upload(H.n, H.diag_offsets, H.values);
    }

    HMMatrix download() const
    {
        static_assert(std::is_same<T, float>::value, "HMMatrix holds fp32 values");
        check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
        HMMatrix H;
        H.n = n;
        H.num_diags = ndiag();
        H.diag_offsets = offsets;
        H.diag_lengths = len.download(offsets.size());
        H.diag_starts = starts.download(offsets.size());
        H.values = vals.download(static_cast<size_t>(nnz));
        H.total_nz = nnz;
        return H;
    }

    // The values, diagonal after diagonal in offset order.
    std::vector<T> download_values() const
    {
        check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
        return vals.download(static_cast<size_t>(nnz));
    }
};

using DeviceHM = DeviceHMT<float>;
using DeviceHMC = DeviceHMT<diagpu_complex64>;

// Keeps a parameter out of template argument deduction.
template <typename U> struct NoDeduce { using type = U; };

template <typename T = float>
inline DeviceHMT<T> identity_hm(int n)
{
    DeviceHMT<T> I = DeviceHMT<T>::with_offsets(n, {0});
    I.vals.upload(std::vector<T>(static_cast<size_t>(n), HMValue<T>::to_c(HMScalar<T>(1))));
    return I;
}

// The same matrix with complex64 values (imaginary parts zero).
inline DeviceHMC to_complex(const DeviceHM& M, hipStream_t stream = 0)
{
    DeviceHMC C = DeviceHMC::with_offsets(M.n, M.offsets);
    check(diagpu_promote_f32_c64(M.nnz, M.vals.data(), C.vals.data(), stream));
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return C;
}

// Z = alpha * X + beta * Y on the union of the diagonal sets (Y may be null).
template <typename T>
inline DeviceHMT<T> axpby(typename NoDeduce<HMScalar<T>>::type alpha, const DeviceHMT<T>& X,
                          typename NoDeduce<HMScalar<T>>::type beta,
                          const typename NoDeduce<DeviceHMT<T>>::type* Y, hipStream_t stream = 0)
{
    if (Y && Y->n != X.n) throw Error(DIAGPU_ERR_ARG, "axpby: X and Y differ in dimension");
    std::vector<int> u;
    const std::vector<int> none;
    const std::vector<int>& oy = Y ? Y->offsets : none;
    std::set_union(X.offsets.begin(), X.offsets.end(), oy.begin(), oy.end(), std::back_inserter(u));
    DeviceHMT<T> Z = DeviceHMT<T>::with_offsets(X.n, u);
    const int ny = Y ? Y->ndiag() : 0;
    check(HMValue<T>::axpby(X.n, X.off.data(), X.starts.data(), X.ndiag(), X.vals.data(), alpha,
                            ny ? Y->off.data() : nullptr, ny ? Y->starts.data() : nullptr, ny,
                            ny ? Y->vals.data() : nullptr, beta, Z.off.data(), Z.starts.data(),
                            Z.ndiag(), Z.vals.data(), stream));
    return Z;
}

// The product's structure from a built plan (values allocated, not
// initialised; the host offsets arrive once `stream` has run the copies).
template <typename T>
inline DeviceHMT<T> product_structure(int n, const SpgemmPlan& plan, hipStream_t stream)
{
    const auto& inf = plan.info();
    DeviceHMT<T> C;
    C.n = n;
    C.nnz = inf.c_nnz;
    const size_t nc = static_cast<size_t>(inf.c_ndiag);
    C.offsets.resize(nc);
    C.off.resize(nc);
    C.len.resize(nc);
    C.starts.resize(nc);
    C.vals.resize(static_cast<size_t>(inf.c_nnz));
    if (nc) {
        check_hip(hipMemcpyAsync(C.off.data(), plan.c_offsets(), nc * sizeof(int), hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
        check_hip(hipMemcpyAsync(C.len.data(), plan.c_lengths(), nc * sizeof(int), hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
        check_hip(hipMemcpyAsync(C.starts.data(), plan.c_starts(), nc * sizeof(int64_t), hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
        check_hip(hipMemcpyAsync(C.offsets.data(), plan.c_offsets(), nc * sizeof(int), hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    }
    return C;
}

// C = A * B; the plan is built on the device for this product.
template <typename T>
inline DeviceHMT<T> multiply(const DeviceHMT<T>& A, const DeviceHMT<T>& B, hipStream_t stream = 0)
{
    SpgemmPlan plan(A.n, A.off.data(), A.len.data(), A.starts.data(), A.ndiag(), B.off.data(),
                    B.len.data(), B.starts.data(), B.ndiag(), false, stream);
    DeviceHMT<T> C = product_structure<T>(A.n, plan, stream);
    if (C.offsets.size()) plan.numeric(A.vals.data(), B.vals.data(), C.vals.data(), stream);
    // the plan's buffers are released when it goes out of scope
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return C;
}

// Whether a chain step multiplies the narrow factor X from the left: it is
// then the A operand, whose few diagonals the A-stationary kernel holds in
// LDS (the 7-point stencil's order-6 Taylor chain: fp32 products 2.12 ms
// against 2.58 with the wide factor first; complex propagator 4.46 ms against
// 5.89).  Always for fp32; for complex values where X fits the complex
// kernel (DIAGPU_ASTAT_MAX_A_C64 diagonals), else the gather takes the
// product, which is faster with the wide factor first.
template <typename T> inline bool narrow_first(const DeviceHMT<T>& X)
{
    return std::is_same<T, float>::value || X.ndiag() <= DIAGPU_ASTAT_MAX_A_C64;
}

// H^k (k >= 1) by the chain P_j = H * P_{j-1} (P_{j-1} * H for complex
// values when H is too wide for the complex A-stationary kernel; the factors
// commute).
template <typename T>
inline DeviceHMT<T> power(const DeviceHMT<T>& H, int k, hipStream_t stream = 0)
{
    if (k < 1) throw Error(DIAGPU_ERR_ARG, "power: k must be >= 1");
    DeviceHMT<T> P = axpby<T>(HMScalar<T>(1), H, HMScalar<T>(0), nullptr, stream);
    for (int j = 1; j < k; ++j)    // multiply syncs before P is freed
        P = narrow_first(H) ? multiply(H, P, stream) : multiply(P, H, stream);
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return P;
}

// S + sigma I: in place when S holds the main diagonal (axpby over that one
// diagonal with Z = X), else a new matrix on the union of the diagonal sets.
template <typename T>
inline void add_identity(DeviceHMT<T>& S, typename NoDeduce<HMScalar<T>>::type sigma,
                         hipStream_t stream = 0)
{
    const DeviceHMT<T> I = identity_hm<T>(S.n);
    const auto it = std::lower_bound(S.offsets.begin(), S.offsets.end(), 0);
    if (it == S.offsets.end() || *it != 0) {
        DeviceHMT<T> U = axpby<T>(HMScalar<T>(1), S, sigma, &I, stream);
        check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");   // before S is freed
        S = std::move(U);
        return;
    }
    const size_t i = static_cast<size_t>(it - S.offsets.begin());
    const int* o = S.off.data() + i;
    const int64_t* st = S.starts.data() + i;
    check(HMValue<T>::axpby(S.n, o, st, 1, S.vals.data(), HMScalar<T>(1), I.off.data(),
                            I.starts.data(), 1, I.vals.data(), sigma, o, st, 1, S.vals.data(),
                            stream));
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");       // before I is freed
}

// One Horner step I + (alpha H) S.  Where H goes first (narrow_first) and
// the A-stationary kernel takes the plan, one fused product:
// diagpu_spgemm_numeric_astat_scaled_* scales H in LDS and adds I to the
// product's main diagonal (fp32: the bits of the unfused step on finite
// values whose scaled elements are normal or zero).  Otherwise (alpha H)
// is formed by axpby, multiplied, and I added in place.  Synchronises
// before returning, so S may be freed.
template <typename T>
inline DeviceHMT<T> horner_step(const DeviceHMT<T>& H, typename NoDeduce<HMScalar<T>>::type alpha,
                                const DeviceHMT<T>& S, hipStream_t stream = 0)
{
    using S_t = HMScalar<T>;
    if (narrow_first(H)) {
        SpgemmPlan plan(H.n, H.off.data(), H.len.data(), H.starts.data(), H.ndiag(), S.off.data(),
                        S.len.data(), S.starts.data(), S.ndiag(), false, stream);
        const bool fused = std::is_same<T, float>::value ? plan.uses_astat() : plan.uses_astat_c64();
        if (fused) {
            DeviceHMT<T> C = product_structure<T>(H.n, plan, stream);
            // C has a main diagonal where some offset of H has its negation in S
            bool has0 = false;
            for (int h : H.offsets)
                has0 = has0 || std::binary_search(S.offsets.begin(), S.offsets.end(), -h);
            if (C.offsets.size())
                plan.numeric_scaled(H.vals.data(), HMValue<T>::to_c(alpha), S.vals.data(),
                                    HMValue<T>::to_c(S_t(has0 ? 1 : 0)), C.vals.data(), stream);
            check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");   // C's host offsets
            if (!has0) add_identity<T>(C, S_t(1), stream);                      // (synchronises)
            return C;
        }
    }
    const DeviceHMT<T> Hj = axpby<T>(alpha, H, S_t(0), nullptr, stream);
    // multiply syncs before its operands may be freed
    DeviceHMT<T> C = narrow_first(Hj) ? multiply(Hj, S, stream) : multiply(S, Hj, stream);
    add_identity<T>(C, S_t(1), stream);
    return C;
}

// S = sum_{k=0..order} (t H)^k / k! in Horner form:
//   S_order = I + (t/order) H,  S_j = I + S_{j+1} * ((t/j) H),  S = S_1,
// one device-planned SpGEMM per step of the wide S_{j+1} and the narrow
// (t/j) H (S_{j+1} is a polynomial in H, so they commute; the narrow factor
// goes first where the A-stationary kernel holds it: narrow_first).  t is real
// for DeviceHM, complex for DeviceHMC.
template <typename T>
inline DeviceHMT<T> taylor_expm(const DeviceHMT<T>& H, typename NoDeduce<HMScalar<T>>::type t,
                                int order, hipStream_t stream = 0)
{
    using S_t = HMScalar<T>;
    if (order < 0) throw Error(DIAGPU_ERR_ARG, "taylor_expm: order must be >= 0");
    if (order == 0) return identity_hm<T>(H.n);
    const DeviceHMT<T> I = identity_hm<T>(H.n);
    DeviceHMT<T> S = axpby<T>(t / static_cast<float>(order), H, S_t(1), &I, stream);
    for (int j = order - 1; j >= 1; --j)
        S = horner_step<T>(H, t / static_cast<float>(j), S, stream);
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return S;
}

// U = sum_{k=0..order} (-i dt H)^k / k!, the truncated Taylor propagator
// exp(-i dt H) as an explicit complex matrix (slides/transcript.md:10-18:
// build U once, apply it to many states).
inline DeviceHMC propagator(const DeviceHMC& H, float dt, int order, hipStream_t stream = 0)
{
    return taylor_expm<diagpu_complex64>(H, std::complex<float>(0.f, -dt), order, stream);
}

inline DeviceHMC propagator(const DeviceHM& H, float dt, int order, hipStream_t stream = 0)
{
    return propagator(to_complex(H, stream), dt, order, stream);
}

// A square HM matrix in the Recon layout the SpMV kernels read
// (build_recon on the device): offsets descending, ndiag x n values.
template <typename T>
struct DeviceReconT {
    int n = 0, ndiag = 0;
    DeviceArray<int> offsets;
    DeviceArray<T> values;
};

template <typename T>
inline DeviceReconT<T> to_recon(const DeviceHMT<T>& M, hipStream_t stream = 0)
{
    DeviceReconT<T> R;
    R.n = M.n;
    R.ndiag = M.ndiag();
    R.offsets.resize(static_cast<size_t>(R.ndiag));
    R.values.resize(static_cast<size_t>(R.ndiag) * static_cast<size_t>(M.n));
    check(HMValue<T>::to_recon(M.n, M.off.data(), M.starts.data(), R.ndiag, M.vals.data(),
                               R.offsets.data(), R.values.data(), stream));
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return R;
}

// The non-owning views the SpMV entry points and KrylovPropagator take.
inline diagpu_recon_view_f32 view(const DeviceReconT<float>& R)
{
    return diagpu_recon_view_f32{R.n, R.n, R.ndiag, R.offsets.data(), R.values.data()};
}

inline diagpu_recon_view_c64 view(const DeviceReconT<diagpu_complex64>& R)
{
    return diagpu_recon_view_c64{R.n, R.n, R.ndiag, R.offsets.data(), R.values.data()};
}

}  // namespace diagpu
