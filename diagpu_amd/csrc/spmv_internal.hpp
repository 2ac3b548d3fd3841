// Library-internal SpMV interface shared by the C ABI (spmv.hip) and the
// Krylov drivers (krylov.hip).
#pragma once

#include <cstdint>

namespace diagpu {

// Complex fp32 element: the layout of diagpu_complex64 and std::complex<float>.
struct cf32 {
    float re, im;
};

// Fused dot epilogue of an SpMV launch: every workgroup stores one fp64
// partial of sum_r Re(conj(x[r]) * y[r]) into partials[tile], and a
// one-workgroup kernel on the same stream adds them in tile order into *out
// (deterministic).  `partials` holds spmv_tiles<TV, TX>(rows) doubles.
struct DotArgs {
    double* partials;   // one per row tile (spmv_tiles)
    double* out;        // the sum, or NULL: the caller adds the partials itself
};

// *out = sum of partials[0 .. n) in index order (one workgroup, async).
int sum_partials(const double* partials, int32_t n, double* out, void* stream);

// Two such sums in one launch (one workgroup each), each in index order.
int sum_partials2(const double* p0, int32_t n0, double* out0, const double* p1, int32_t n1,
                  double* out1, void* stream);

// Number of row tiles (= workgroups doing work) of an SpMV launch.
template <typename TV, typename TX>
int32_t spmv_tiles(int32_t rows);

// y = Recon x for TV matrix elements and TX vector elements; instantiated for
// (float, float), (double, double), (cf32, cf32) and (float, cf32).  With
// `dot`, also the fused epilogue above (needs x_size >= rows).  Asynchronous.
template <typename TV, typename TX>
int spmv_run(int32_t rows, int32_t cols, int32_t num_diags, const int32_t* offs, const TV* vals,
             const TX* x, int64_t x_size, TX* y, const DotArgs* dot, void* stream,
             const char* name);

}  // namespace diagpu
