// Matrix-power chain and truncated Taylor series for HM (compact diagonal)
// matrices on the GPU: the caller of the SpGEMM hot path that the reference
// describes but does not ship (spmspm/gather_flat.cuh:13-14, 110-117: a chain
// P_{k+1} = P_k * H whose plan is rebuilt on the device every step).
// power() is that chain; taylor_expm() runs the same kind of chain in Horner
// form, so that no step needs a full pass to add the powers together.
//
// Each product builds its C structure and pair plan with the device symbolic
// phase (one stream sync returns the counts), then runs the numeric phase.
// Sums and scalings run diagpu_dia_axpby_f32 over the union of the operands'
// diagonals; the union is a merge of two short sorted offset lists on the
// host, which holds a copy of every matrix's offsets.
#pragma once

#include <algorithm>
#include <cstdlib>
#include <iterator>
#include <vector>

#include "common.hpp"
#include "spgemm.hpp"

namespace diagpu {

// Device-resident square HM matrix; `offsets` is the host copy (ascending).
struct DeviceHM {
    int n = 0;
    std::vector<int> offsets;
    int64_t nnz = 0;
    DeviceArray<int> off, len;
    DeviceArray<int64_t> starts;
    DeviceArray<float> vals;

    int ndiag() const { return static_cast<int>(offsets.size()); }

    // Structure for the given offsets (ascending, distinct, |d| < n); values
    // allocated, not initialised.
    static DeviceHM with_offsets(int n, const std::vector<int>& offs)
    {
        DeviceHM M;
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

    static DeviceHM upload(const HMMatrix& H)
    {
        int64_t s = 0;
        for (int i = 0; i < H.num_diags; ++i) {
            if (H.diag_starts[i] != s)
                throw Error(DIAGPU_ERR_ARG, "DeviceHM::upload: starts must be the prefix sum of lengths");
            s += H.n - std::abs(H.diag_offsets[i]);
        }
        DeviceHM M = with_offsets(H.n, H.diag_offsets);
        if (H.values.size() < static_cast<size_t>(M.nnz))
            throw Error(DIAGPU_ERR_ARG, "DeviceHM::upload: too few values");
        M.vals.upload(std::vector<float>(H.values.begin(), H.values.begin() + M.nnz));
        return M;
    }

    HMMatrix download() const
    {
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
};

inline DeviceHM identity_hm(int n)
{
    DeviceHM I = DeviceHM::with_offsets(n, {0});
    I.vals.upload(std::vector<float>(static_cast<size_t>(n), 1.0f));
    return I;
}

// Z = alpha * X + beta * Y on the union of the diagonal sets (Y may be null).
inline DeviceHM axpby(float alpha, const DeviceHM& X, float beta, const DeviceHM* Y,
                      hipStream_t stream = 0)
{
    if (Y && Y->n != X.n) throw Error(DIAGPU_ERR_ARG, "axpby: X and Y differ in dimension");
    std::vector<int> u;
    const std::vector<int> none;
    const std::vector<int>& oy = Y ? Y->offsets : none;
    std::set_union(X.offsets.begin(), X.offsets.end(), oy.begin(), oy.end(), std::back_inserter(u));
    DeviceHM Z = DeviceHM::with_offsets(X.n, u);
    const int ny = Y ? Y->ndiag() : 0;
    check(diagpu_dia_axpby_f32(X.n, X.off.data(), X.starts.data(), X.ndiag(), X.vals.data(), alpha,
                               ny ? Y->off.data() : nullptr, ny ? Y->starts.data() : nullptr, ny,
                               ny ? Y->vals.data() : nullptr, beta, Z.off.data(), Z.starts.data(),
                               Z.ndiag(), Z.vals.data(), stream));
    return Z;
}

// C = A * B; the plan is built on the device for this product.
inline DeviceHM multiply(const DeviceHM& A, const DeviceHM& B, hipStream_t stream = 0)
{
    SpgemmPlan plan(A.n, A.off.data(), A.len.data(), A.starts.data(), A.ndiag(), B.off.data(),
                    B.len.data(), B.starts.data(), B.ndiag(), false, stream);
    const auto& inf = plan.info();
    DeviceHM C;
    C.n = A.n;
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
        plan.numeric(A.vals.data(), B.vals.data(), C.vals.data(), stream);
    }
    // the plan's buffers are released when it goes out of scope
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return C;
}

// H^k (k >= 1) by the chain P_j = P_{j-1} * H.
inline DeviceHM power(const DeviceHM& H, int k, hipStream_t stream = 0)
{
    if (k < 1) throw Error(DIAGPU_ERR_ARG, "power: k must be >= 1");
    DeviceHM P = axpby(1.0f, H, 0.0f, nullptr, stream);
    for (int j = 1; j < k; ++j) P = multiply(P, H, stream);    // multiply syncs before P is freed
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return P;
}

// S + sigma I: in place when S holds the main diagonal (axpby over that one
// diagonal with Z = X), else a new matrix on the union of the diagonal sets.
inline void add_identity(DeviceHM& S, float sigma, hipStream_t stream = 0)
{
    const DeviceHM I = identity_hm(S.n);
    const auto it = std::lower_bound(S.offsets.begin(), S.offsets.end(), 0);
    if (it == S.offsets.end() || *it != 0) {
        DeviceHM U = axpby(1.0f, S, sigma, &I, stream);
        check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");   // before S is freed
        S = std::move(U);
        return;
    }
    const size_t i = static_cast<size_t>(it - S.offsets.begin());
    const int* o = S.off.data() + i;
    const int64_t* st = S.starts.data() + i;
    check(diagpu_dia_axpby_f32(S.n, o, st, 1, S.vals.data(), 1.0f, I.off.data(), I.starts.data(), 1,
                               I.vals.data(), sigma, o, st, 1, S.vals.data(), stream));
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");       // before I is freed
}

// S = sum_{k=0..order} (t H)^k / k! in Horner form:
//   S_order = I + (t/order) H,  S_j = I + S_{j+1} * ((t/j) H),  S = S_1,
// one device-planned SpGEMM per step, the wide S_{j+1} times the narrow
// (t/j) H (S_{j+1} is a polynomial in H, so they commute; this order is the
// faster one for the numeric kernel).
inline DeviceHM taylor_expm(const DeviceHM& H, float t, int order, hipStream_t stream = 0)
{
    if (order < 0) throw Error(DIAGPU_ERR_ARG, "taylor_expm: order must be >= 0");
    if (order == 0) return identity_hm(H.n);
    const DeviceHM I = identity_hm(H.n);
    DeviceHM S = axpby(t / static_cast<float>(order), H, 1.0f, &I, stream);
    for (int j = order - 1; j >= 1; --j) {
        const DeviceHM Hj = axpby(t / static_cast<float>(j), H, 0.0f, nullptr, stream);
        S = multiply(S, Hj, stream);          // multiply syncs before the old S is freed
        add_identity(S, 1.0f, stream);
    }
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return S;
}

}  // namespace diagpu
