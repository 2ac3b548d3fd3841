// SpMV host API of spmv/src/dia_reconstruct.cuh, over libdiagpu.
//
// Same type names, members and semantics as the reference header, so code
// written against it compiles unchanged with hipcc after swapping the
// include: DiaMatrix, ReconMatrix, build_recon, ReconView and
// launch_tc_spmv_regdirect.  The launcher runs the gfx950 FP32 kernel
// (diagpu_spmv_recon_f32) instead of the TF32 MMA; results are the exact-FP32
// sum, i.e. at least as accurate.  Failures throw diagpu::Error (the
// reference returned void and left errors to cudaGetLastError).
#pragma once

#include <algorithm>
#include <cstdint>
#include <functional>
#include <type_traits>
#include <vector>

#include "common.hpp"

// Host-side compact DIA matrix (spmv/src/dia_reconstruct.cuh:52-59).
struct DiaMatrix {
    int                rows;
    int                cols;
    std::vector<int>   offsets;
    std::vector<int>   diag_starts;
    std::vector<int>   diag_lengths;
    std::vector<float> values;
};

// Host-side K x cols Recon matrix (:64-70): row k holds diagonal
// diag_offsets[k] at columns [max(d,0), max(d,0) + len), offsets descending.
struct ReconMatrix {
    int                rows;
    int                cols;
    int                num_diags;
    std::vector<int>   diag_offsets;
    std::vector<float> values;
};

// dense_to_dia of the reference's SpMV tests (spmv/test/test_tc_spmv.cu:39-62,
// spmv/test/test_reconstruct.cpp): every diagonal of the row-major
// rows x cols matrix H that holds a nonzero, offsets ascending from
// -(rows - 1), each stored whole (zeros included).
inline DiaMatrix dense_to_dia(const float* H, int rows, int cols)
{
    DiaMatrix D;
    D.rows = rows;
    D.cols = cols;
    for (int d = -(rows - 1); d <= cols - 1; ++d) {
        const int sr = d >= 0 ? 0 : -d, sc = d >= 0 ? d : 0;
        const int len = std::min(rows - sr, cols - sc);
        if (len <= 0) continue;
        bool any = false;
        for (int j = 0; j < len && !any; ++j) any = H[size_t(sr + j) * cols + (sc + j)] != 0.0f;
        if (!any) continue;
        D.offsets.push_back(d);
        D.diag_starts.push_back(static_cast<int>(D.values.size()));
        D.diag_lengths.push_back(len);
        for (int j = 0; j < len; ++j) D.values.push_back(H[size_t(sr + j) * cols + (sc + j)]);
    }
    return D;
}

// build_recon (:77-107): offsets sorted descending; row k receives the values
// of the first input diagonal whose offset equals d_k.
inline ReconMatrix build_recon(const DiaMatrix& H)
{
    ReconMatrix R;
    R.rows = H.rows;
    R.cols = H.cols;
    R.num_diags = static_cast<int>(H.offsets.size());
    R.diag_offsets = H.offsets;
    std::sort(R.diag_offsets.begin(), R.diag_offsets.end(), std::greater<int>());
    R.values.assign(static_cast<size_t>(R.num_diags) * static_cast<size_t>(R.cols), 0.0f);
    for (int k = 0; k < R.num_diags; ++k) {
        const int d = R.diag_offsets[k];
        const auto it = std::find(H.offsets.begin(), H.offsets.end(), d);
        const size_t di = static_cast<size_t>(it - H.offsets.begin());
        const int first_col = d > 0 ? d : 0;
        const int len = H.diag_lengths[di];
        const float* src = H.values.data() + H.diag_starts[di];
        std::copy(src, src + len,
                  R.values.begin() + static_cast<std::ptrdiff_t>(k) * R.cols + first_col);
    }
    return R;
}

// Non-owning device view (:112-118).  Layout-identical to the C ABI's
// diagpu_recon_view_f32.
struct ReconView {
    int          rows;
    int          cols;
    int          num_diags;
    const int*   diag_offsets;   // device [num_diags]
    const float* values;         // device [num_diags * cols]
};
static_assert(sizeof(ReconView) == sizeof(diagpu_recon_view_f32) &&
                  offsetof(ReconView, diag_offsets) == offsetof(diagpu_recon_view_f32, diag_offsets) &&
                  offsetof(ReconView, values) == offsetof(diagpu_recon_view_f32, values),
              "ReconView must match diagpu_recon_view_f32");

// spmv_from_recon of the reference's SpMV tests (test_tc_spmv.cu:64-79,
// test_reconstruct.cpp:122-138): y = R x on the host in fp32, one row at a
// time, terms in Recon row order (offsets descending).
inline std::vector<float> spmv_from_recon(const ReconMatrix& R, const std::vector<float>& x)
{
    std::vector<float> y(static_cast<size_t>(R.rows), 0.0f);
    for (int r = 0; r < R.rows; ++r) {
        float sum = 0.0f;
        for (int k = 0; k < R.num_diags; ++k) {
            const int c = r + R.diag_offsets[k];
            if (c >= 0 && c < R.cols) sum += R.values[size_t(k) * R.cols + c] * x[c];
        }
        y[r] = sum;
    }
    return y;
}

// y = H x on `stream` (:139-144; tc_spmv_regdirect_kernel.cu:135-147): y is
// overwritten, rows == 0 is a no-op, asynchronous, allocates nothing.
inline void launch_tc_spmv_regdirect(ReconView R, const float* d_x, int x_size, float* d_y,
                                     hipStream_t stream = 0)
{
    diagpu::check(diagpu_spmv_recon_f32(reinterpret_cast<const diagpu_recon_view_f32*>(&R), d_x,
                                        x_size, d_y, stream));
}

namespace diagpu {

// The same SpMV under its own name, and the fp64 variant.
inline void launch_dia_spmv(ReconView R, const float* d_x, int64_t x_size, float* d_y,
                            hipStream_t stream = 0)
{
    check(diagpu_spmv_recon_f32(reinterpret_cast<const diagpu_recon_view_f32*>(&R), d_x, x_size,
                                d_y, stream));
}

struct ReconViewF64 {
    int           rows;
    int           cols;
    int           num_diags;
    const int*    diag_offsets;
    const double* values;
};

inline void launch_dia_spmv(ReconViewF64 R, const double* d_x, int64_t x_size, double* d_y,
                            hipStream_t stream = 0)
{
    check(diagpu_spmv_recon_f64(reinterpret_cast<const diagpu_recon_view_f64*>(&R), d_x, x_size,
                                d_y, stream));
}

// Band values of the reference SpMV benchmark (spmv/bench/bench_cusparse.cu:
// 70-82; the same hval is in spmv/tools/gen_banded_mtx.cpp:18-23): an integer
// hash of (row, offset), resp. of the index, whose low 16 bits map onto
// [-1, 1) in steps of 2^-15.  hval(r, d) is H[r, r + d]; xval(i) is x[i].
inline float hval(int r, int d)
{
    uint32_t h = static_cast<uint32_t>(r) * 2654435761u;
    h ^= static_cast<uint32_t>(d + 1024) * 40503u;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    return static_cast<float>(h & 0xFFFFu) * (2.0f / 65536.0f) - 1.0f;
}

inline float xval(int i)
{
    uint32_t h = static_cast<uint32_t>(i) * 2246822519u;
    h ^= h >> 13;
    h *= 0x85ebca6bu;
    h ^= h >> 16;
    return static_cast<float>(h & 0xFFFFu) * (2.0f / 65536.0f) - 1.0f;
}

// The benchmark's N x N Recon matrix for the given offsets (:84-89 default
// {-9, -5, -2, -1, 0, 1, 2, 5, 9}; fill :131-144): offsets sorted descending,
// R[k][c] = hval(c - d_k, d_k) where that row exists, zero elsewhere.
inline ReconMatrix make_hash_band(int N, std::vector<int> offsets)
{
    std::sort(offsets.begin(), offsets.end(), std::greater<int>());
    ReconMatrix R;
    R.rows = N;
    R.cols = N;
    R.num_diags = static_cast<int>(offsets.size());
    R.diag_offsets = offsets;
    R.values.assign(static_cast<size_t>(R.num_diags) * static_cast<size_t>(N), 0.0f);
    for (int k = 0; k < R.num_diags; ++k) {
        const int d = offsets[k];
        const int c0 = std::max(d, 0), c1 = std::min(N, N + d);
        float* row = R.values.data() + static_cast<size_t>(k) * N;
        for (int c = c0; c < c1; ++c) row[c] = hval(c - d, d);
    }
    return R;
}

// x of the same benchmark (:97-98).
inline std::vector<float> make_hash_x(int N)
{
    std::vector<float> x(static_cast<size_t>(N));
    for (int i = 0; i < N; ++i) x[static_cast<size_t>(i)] = xval(i);
    return x;
}

// Owning device copy of a ReconMatrix with its view.
struct DeviceRecon {
    DeviceArray<int> offsets;
    DeviceArray<float> values;
    ReconView view{};

    explicit DeviceRecon(const ReconMatrix& R)
        : offsets(R.diag_offsets), values(R.values)
    {
        view = ReconView{R.rows, R.cols, R.num_diags, offsets.data(), values.data()};
    }
};

}  // namespace diagpu
