// gemm_diag (gemm_diag/gemm_diag.cu) over libdiagpu: row-packed operands,
// compact C.
//
//   C[k][t] = sum_{i + j = k} DA[i][t] * DB[j][t + d_i]        (:9-15)
//
// DA / DB are P x n / Q x n row-packed arrays (DA[i][t] = A[t, t + d_i], zero
// elsewhere; pack_diag_matrix, :362-382).  C uses the compact layout of
// build_c_layout (:388-423), with int64 offsets.  The product is exact for
// any offset sets (the reference kernel's 7-entry k-map per 4x4 tile drops
// terms for non-contiguous offsets); C is overwritten, so no memset first.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <random>
#include <vector>

#include "common.hpp"
#include "spgemm.hpp"

namespace diagpu {

// pack_diag_matrix (gemm_diag.cu:362-382): the P x n row-packed operand of
// the reference driver.  Row ri holds diagonal d = offsets[ri]: its n - |d|
// elements at columns [max(-d, 0), max(-d, 0) + n - |d|), drawn in that
// order, diagonal after diagonal, from U(0.5, 1.5) with std::mt19937(seed);
// zeros elsewhere.  The draws are the reference's; the values equal its
// wherever the standard library's uniform_real_distribution is the same.
inline void pack_diag_matrix(int n, const std::vector<int>& offsets, unsigned seed,
                             std::vector<float>& DA_out, std::vector<int>& off_out)
{
    const int P = static_cast<int>(offsets.size());
    DA_out.assign(static_cast<size_t>(P) * n, 0.0f);
    off_out = offsets;
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(0.5f, 1.5f);
    for (int ri = 0; ri < P; ++ri) {
        const int d = offsets[ri];
        const int first = d >= 0 ? 0 : -d;
        const int len = n - std::abs(d);
        for (int p = 0; p < len; ++p) DA_out[static_cast<size_t>(ri) * n + first + p] = dist(rng);
    }
}

// build_c_layout (gemm_diag.cu:388-423) with 64-bit C offsets.
struct CLayout {
    std::vector<int64_t> C_offsets;   // start of each C diagonal
    std::vector<int> C_lens;
    std::vector<int> k_to_idx;        // 2n - 1 entries
    std::vector<int> k_list;          // C diagonal offsets, ascending
    int64_t total_c = 0;
    int num_k = 0;
};

inline CLayout build_c_layout(int n, const std::vector<int>& off_A, const std::vector<int>& off_B)
{
    std::vector<int> la, lb;
    for (int d : off_A) la.push_back(n - std::abs(d));
    for (int d : off_B) lb.push_back(n - std::abs(d));
    const auto r = run_symbolic(n, off_A, la, hm_starts(n, off_A), off_B, lb, hm_starts(n, off_B), true);
    CLayout L;
    L.C_offsets = r.C_starts;
    L.C_lens = r.C_len;
    L.k_to_idx = r.lookup;
    L.k_list = r.C_off;
    L.total_c = r.info.c_nnz;
    L.num_k = static_cast<int>(r.info.c_ndiag);
    return L;
}

// Device gemm_diag: row-packed DA (P x n) and DB (Q x n) with device offsets.
// Builds the HM addressing of both operands and the plan at construction;
// run() computes C (info().c_nnz values) on `stream`.
class GemmDiag {
public:
    GemmDiag(int n, const int* d_off_A, int P, const int* d_off_B, int Q, hipStream_t stream = 0)
        : n_(n), sa_(P), la_(P), sb_(Q), lb_(Q)
    {
        check(diagpu_rowpacked_as_hm(n, d_off_A, P, sa_.data(), la_.data(), stream));
        check(diagpu_rowpacked_as_hm(n, d_off_B, Q, sb_.data(), lb_.data(), stream));
        plan_ = new SpgemmPlan(n, d_off_A, la_.data(), sa_.data(), P, d_off_B, lb_.data(), sb_.data(),
                               Q, true, stream);
    }
    GemmDiag(const GemmDiag&) = delete;
    GemmDiag& operator=(const GemmDiag&) = delete;
    ~GemmDiag() { delete plan_; }

    void run(const float* d_DA, const float* d_DB, float* d_C, hipStream_t stream = 0,
             NumericKernel kernel = NumericKernel::Auto) const
    {
        plan_->numeric(d_DA, d_DB, d_C, stream, kernel);
    }
    const SpgemmPlan& plan() const { return *plan_; }
    const diagpu_spgemm_info& info() const { return plan_->info(); }

private:
    int n_;
    DeviceArray<int64_t> sa_;
    DeviceArray<int> la_;
    DeviceArray<int64_t> sb_;
    DeviceArray<int> lb_;
    SpgemmPlan* plan_ = nullptr;
};

}  // namespace diagpu
