// c = exp(-i t T) e_1 for an m x m real symmetric tridiagonal T (diagonal
// al[0..m-1], off-diagonal be[0..m-2]) in complex128: the small dense step of
// the Lanczos propagator (krylov.hip).  Host code only, no HIP: the CPU test
// tests/cpp/test_expm_tridiag_cpu.cpp compiles it with g++.
//
// With r = ||t T|| (Gershgorin bound):
//   r <= 2 kMaxSubsteps   t is split into s = ceil(r / 2) sub-steps, each
//                         applying exp(-i (t/s) T) to the vector as a Taylor
//                         series of tridiagonal products, stopped when a term
//                         falls below 1e-17 of the sum (at most 50 terms:
//                         2^50 / 50! ~ 1e-50).  With each sub-step's norm at
//                         most 2 no term exceeds 2 times the sum's scale, so
//                         nothing cancels; the cost is O(s m), tens of
//                         microseconds for m <= 64 (a cyclic Jacobi
//                         eigendecomposition of T took 276 us at m = 30).
//   larger r              scaling and squaring: E = exp(-i (t / 2^q) T) as a
//                         dense Taylor series with r / 2^q <= 1/2, squared q
//                         times, c = E e_1.  The cost grows with log2 r
//                         (O(q m^3)), so no t makes the host loop for long.
// Returns false (c untouched) if T or t is not finite.
#pragma once

#include <cmath>
#include <complex>
#include <vector>

namespace diagpu {

constexpr int kMaxSubsteps = 256;

inline bool expm_tridiag_e1(int m, const std::vector<double>& al, const std::vector<double>& be,
                            double t, std::vector<std::complex<double>>& c)
{
    typedef std::complex<double> cd;
    double gersh = 0.0;
    for (int i = 0; i < m; ++i) {
        const double r = std::fabs(al[i]) + (i > 0 ? std::fabs(be[i - 1]) : 0.0) +
                         (i + 1 < m ? std::fabs(be[i]) : 0.0);
        gersh = r > gersh ? r : gersh;
    }
    const double nrm = gersh * std::fabs(t);
    if (!std::isfinite(nrm)) return false;
    c.assign(m, cd(0.0));
    if (m <= 0) return true;
    // (T v) for a vector v
    auto tmul = [&](const std::vector<cd>& v, std::vector<cd>& out) {
        for (int i = 0; i < m; ++i) {
            cd x = al[i] * v[i];
            if (i > 0) x += be[i - 1] * v[i - 1];
            if (i + 1 < m) x += be[i] * v[i + 1];
            out[i] = x;
        }
    };
    if (nrm <= 2.0 * kMaxSubsteps) {
        const int steps = nrm > 2.0 ? (int)std::ceil(nrm / 2.0) : 1;
        const cd h(0.0, -t / steps);
        std::vector<cd> term(m), next(m);
        c[0] = 1.0;
        for (int st = 0; st < steps; ++st) {
            term = c;
            for (int k = 1; k <= 50; ++k) {
                tmul(term, next);
                double tn = 0.0, cn = 0.0;
                for (int i = 0; i < m; ++i) {
                    term[i] = next[i] * (h / (double)k);
                    c[i] += term[i];
                    tn = std::max(tn, std::fabs(term[i].real()) + std::fabs(term[i].imag()));
                    cn = std::max(cn, std::fabs(c[i].real()) + std::fabs(c[i].imag()));
                }
                if (tn <= 1e-17 * cn) break;
            }
        }
        return true;
    }
    // scaling and squaring on the dense m x m exponential (column-major E)
    const int q = (int)std::ceil(std::log2(nrm / 0.5));
    const cd h(0.0, -std::ldexp(t, -q));
    std::vector<cd> E((size_t)m * m, cd(0.0)), term((size_t)m * m, cd(0.0)), col(m), tmp(m);
    for (int i = 0; i < m; ++i) E[(size_t)i * m + i] = term[(size_t)i * m + i] = 1.0;
    for (int k = 1; k <= 40; ++k) {     // ||h T|| <= 1/2: 2^-40 / 40! is far below rounding
        double tn = 0.0;
        for (int j = 0; j < m; ++j) {   // term = term (h T) / k, column by column
            for (int i = 0; i < m; ++i) col[i] = term[(size_t)j * m + i];
            tmul(col, tmp);             // T symmetric: (term T) = (T term^T)^T, and term
            for (int i = 0; i < m; ++i) {   // is a polynomial in T, so it commutes with T
                const cd v = tmp[i] * (h / (double)k);
                term[(size_t)j * m + i] = v;
                E[(size_t)j * m + i] += v;
                tn = std::max(tn, std::abs(v));
            }
        }
        if (tn <= 1e-18) break;
    }
    std::vector<cd> S((size_t)m * m);
    for (int s = 0; s < q; ++s) {       // E = E E
        for (int j = 0; j < m; ++j)
            for (int i = 0; i < m; ++i) {
                cd acc = 0.0;
                for (int l = 0; l < m; ++l) acc += E[(size_t)l * m + i] * E[(size_t)j * m + l];
                S[(size_t)j * m + i] = acc;
            }
        E.swap(S);
    }
    for (int i = 0; i < m; ++i) c[i] = E[i];   // first column
    return true;
}

}  // namespace diagpu
