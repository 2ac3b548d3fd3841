// DIA x DIA SpGEMM, numeric phase on the GPU (HM layout, fp32).
//
//   C[k][p] = sum over the plan entries g of C diagonal k of
//             Av[g.ab + p + g.ash] * Bv[g.bb + p + g.bsh]
//   for 0 <= p < C_len[k], terms with p + ash outside [0, al) or p + bsh
//   outside [0, bl) dropped -- the shifted multiply-accumulate of
//   hm_structured_sparse_matmul_kernel (spmspm/paper_hm_kernel.cu:31-93) and
//   of gather_flat_kernel (spmspm/gather_flat.cuh:47-62), evaluated in plan
//   order with fp32 accumulation.  Every C value is written exactly once: no
//   atomics, no pre-zeroing, deterministic.
//
// Work decomposition.  An item is (row block rb, C diagonal k): the 1024
// positions of diagonal k whose matrix rows fall in block rb (shifted by at
// most 3 so the item's first C element is 16-byte aligned).  Each lane owns 4
// consecutive positions: one aligned 128-bit store of C and, per plan entry,
// one 128-bit load each of A and B (dword aligned).
//
// Row-space locality.  In row coordinates the entry (da, db) of C row i
// reads A(i, i + da) and B(i + da, i + dc): every A diagonal at rows i, every
// B diagonal at rows i + da.  Items are ordered row block first, so the
// workgroups active on one XCD all work inside one row block and share an L2
// working set of |A| x 1024 A values and |B| x (1024 + spread of da) B
// values.  The launch is persistent: XCD x (workgroups b with b mod 8 == x)
// owns the row blocks [x * nbx, (x + 1) * nbx) and its workgroups stride
// through that range's items in order, so each XCD's L2 streams one
// contiguous band of rows.  Each workgroup's item loop ends at a fixed count.
#include "common.hpp"

namespace diagpu {
namespace {

constexpr int kBlock = 256;
constexpr int kTB = kBlock * 4;   // positions per item
constexpr int kPairChunk = 4;     // plan entries whose loads are issued together

typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));
typedef float f4a __attribute__((ext_vector_type(4), aligned(16)));

__device__ __forceinline__ f4u ld4(const float* p) { return *reinterpret_cast<const f4u*>(p); }

struct PairVals {
    f4u a, b;
    uint32_t valid;   // bit e: position e of the quad has both operands in range
};

__global__ __launch_bounds__(kBlock) void k_gather(
    int32_t n, const float* __restrict__ Av, const float* __restrict__ Bv,
    const int32_t* __restrict__ C_off, const int32_t* __restrict__ C_len,
    const int64_t* __restrict__ C_starts, int32_t nC, const int64_t* __restrict__ pair_ptr,
    const diagpu_gpair* __restrict__ pairs, float* __restrict__ Cv, int32_t NB,
    int32_t nb_per_xcd, int32_t wg_per_xcd)
{
    (void)n;
    const int xcd = (int)(blockIdx.x % kNumXcd);
    const int l = (int)(blockIdx.x / kNumXcd);
    const int rb0 = xcd * nb_per_xcd;
    const int rb_end = (rb0 + nb_per_xcd) < NB ? (rb0 + nb_per_xcd) : NB;
    if (rb0 >= rb_end || nC <= 0) return;

    // Item (rb, k) for j = l, l + L, l + 2L, ...: k advances by L mod nC.
    int rb = rb0 + l / nC;
    int k = l % nC;
    const int lane4 = (int)threadIdx.x * 4;

    while (rb < rb_end) {
        const int dc = C_off[k];
        const int lenC = C_len[k];
        const int64_t cst = C_starts[k];
        const int mc = dc < 0 ? dc : 0;
        const int delta = (int)((cst + mc) & 3);
        const int64_t P0 = (int64_t)rb * kTB + mc - delta;

        if (P0 < lenC && P0 + kTB > 0) {
            const int64_t g0 = pair_ptr[k], g1 = pair_ptr[k + 1];
            const bool item_full = P0 >= 0 && P0 + kTB <= lenC;
            const int64_t p = P0 + lane4;
            float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;

            for (int64_t g = g0; g < g1; g += kPairChunk) {
                diagpu_gpair gp[kPairChunk];
#pragma unroll
                for (int c = 0; c < kPairChunk; ++c)
                    if (g + c < g1) gp[c] = pairs[g + c];
                PairVals pv[kPairChunk];
#pragma unroll
                for (int c = 0; c < kPairChunk; ++c) {
                    if (g + c >= g1) continue;
                    const int ash = gp[c].ash, bsh = gp[c].bsh, al = gp[c].al, bl = gp[c].bl;
                    const float* __restrict__ ap = Av + gp[c].ab + ash;
                    const float* __restrict__ bp = Bv + gp[c].bb + bsh;
                    const bool full = item_full && P0 + ash >= 0 && P0 + kTB + ash <= al &&
                                      P0 + bsh >= 0 && P0 + kTB + bsh <= bl;
                    if (full) {
                        pv[c].a = ld4(ap + p);
                        pv[c].b = ld4(bp + p);
                        pv[c].valid = 0xF;
                    } else {
                        float a[4], b[4];
                        uint32_t v = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int64_t q = p + e;
                            const bool ok = q >= 0 && q < lenC && q + ash >= 0 && q + ash < al &&
                                            q + bsh >= 0 && q + bsh < bl;
                            a[e] = ok ? ap[q] : 0.f;
                            b[e] = ok ? bp[q] : 0.f;
                            v |= ok ? (1u << e) : 0u;
                        }
                        pv[c].a = f4u{a[0], a[1], a[2], a[3]};
                        pv[c].b = f4u{b[0], b[1], b[2], b[3]};
                        pv[c].valid = v;
                    }
                }
#pragma unroll
                for (int c = 0; c < kPairChunk; ++c) {
                    if (g + c >= g1) continue;
                    const uint32_t v = pv[c].valid;
                    acc0 = (v & 1) ? __builtin_fmaf(pv[c].a.x, pv[c].b.x, acc0) : acc0;
                    acc1 = (v & 2) ? __builtin_fmaf(pv[c].a.y, pv[c].b.y, acc1) : acc1;
                    acc2 = (v & 4) ? __builtin_fmaf(pv[c].a.z, pv[c].b.z, acc2) : acc2;
                    acc3 = (v & 8) ? __builtin_fmaf(pv[c].a.w, pv[c].b.w, acc3) : acc3;
                }
            }

            float* __restrict__ cp = Cv + cst;
            if (item_full) {
                *reinterpret_cast<f4a*>(cp + p) = f4a{acc0, acc1, acc2, acc3};
            } else {
                const float r[4] = {acc0, acc1, acc2, acc3};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (p + e >= 0 && p + e < lenC) cp[p + e] = r[e];
            }
        }

        k += wg_per_xcd;
        while (k >= nC) {
            k -= nC;
            ++rb;
        }
    }
}

}  // namespace
}  // namespace diagpu

extern "C" {

DIAGPU_API int diagpu_spgemm_numeric_f32(
    int32_t n, const float* A_vals, const float* B_vals,
    const int32_t* C_off, const int32_t* C_len, const int64_t* C_starts, int64_t c_ndiag,
    const int64_t* pair_ptr, const diagpu_gpair* pairs, int64_t max_pairs,
    float* C_vals, void* stream)
{
    using namespace diagpu;
    const char* fn = "diagpu_spgemm_numeric_f32";
    if (n < 1 || n > (1 << 30)) return fail(DIAGPU_ERR_ARG, "%s: n=%d outside [1, 2^30]", fn, n);
    if (c_ndiag < 0 || c_ndiag > 2 * (int64_t)n - 1)
        return fail(DIAGPU_ERR_ARG, "%s: c_ndiag=%lld outside [0, 2n-1]", fn, (long long)c_ndiag);
    if (max_pairs < 0) return fail(DIAGPU_ERR_ARG, "%s: negative max_pairs", fn);
    if (c_ndiag == 0) return DIAGPU_OK;
    if (!C_off || !C_len || !C_starts || !pair_ptr || !C_vals)
        return fail(DIAGPU_ERR_ARG, "%s: C structure, pair_ptr or C_vals is NULL", fn);
    if (max_pairs > 0 && (!pairs || !A_vals || !B_vals))
        return fail(DIAGPU_ERR_ARG, "%s: pairs or operand values are NULL", fn);

    const int32_t NB = (int32_t)ceil_div<int64_t>((int64_t)n + 3, kTB);
    const int32_t nb_per_xcd = ceil_div<int32_t>(NB, kNumXcd);
    const int64_t items_per_xcd = (int64_t)nb_per_xcd * c_ndiag;
    int64_t wg = (int64_t)(cu_count() / kNumXcd) * 4;       // 4 workgroups per CU
    if (wg > items_per_xcd) wg = items_per_xcd;
    if (wg < 1) wg = 1;
    hipLaunchKernelGGL(k_gather, dim3((unsigned)(wg * kNumXcd)), dim3(kBlock), 0,
                       as_stream(stream), n, A_vals, B_vals, C_off, C_len, C_starts,
                       (int32_t)c_ndiag, pair_ptr, pairs, C_vals, NB, nb_per_xcd, (int32_t)wg);
    return check_launch(fn);
}

}  // extern "C"
