// CPU driver of expm_tridiag_e1 (diagpu_amd/csrc/expm_tridiag.hpp), the
// host step of the Lanczos propagator: reads "m t", m diagonal entries and
// m - 1 off-diagonal entries from stdin, prints c = exp(-i t T) e_1 as m
// lines "re im" (or "NOT FINITE").  tests/test_krylov_cpu.py checks it
// against dense exponentials.
#include <cstdio>
#include <vector>

#include "expm_tridiag.hpp"

int main()
{
    int m = 0;
    double t = 0.0;
    if (std::scanf("%d %lf", &m, &t) != 2 || m < 1) return 2;
    std::vector<double> al(m), be(m > 1 ? m - 1 : 0);
    for (int i = 0; i < m; ++i)
        if (std::scanf("%lf", &al[i]) != 1) return 2;
    for (int i = 0; i + 1 < m; ++i)
        if (std::scanf("%lf", &be[i]) != 1) return 2;
    std::vector<std::complex<double>> c;
    if (!diagpu::expm_tridiag_e1(m, al, be, t, c)) {
        std::printf("NOT FINITE\n");
        return 0;
    }
    for (int i = 0; i < m; ++i) std::printf("%.17g %.17g\n", c[i].real(), c[i].imag());
    return 0;
}
