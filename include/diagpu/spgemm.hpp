// DIA x DIA SpGEMM host API of spmspm/paper_hm.cuh and spmspm/gather_flat.cuh,
// over libdiagpu.
//
// HMMatrix, dense_to_hm, hm_to_dense, compute_c_hm_structure,
// build_c_diag_lookup, GPair, PairPlan, build_pairs_only, FlatPlan and
// build_flat_plan keep the reference names and meanings.  Two deliberate
// differences: element starts and totals are int64 (the reference's int
// overflows once C exceeds 2^31 values), and the integer planners run as the
// GPU symbolic phase (diagpu_spgemm_symbolic), whose output is bit-identical
// to the reference's host loops.  diagpu::SpgemmPlan keeps the plan on the
// device for the numeric phase; spgemm_hm() is a one-call host convenience.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

#include "common.hpp"
#include "schedule.hpp"

// HM (Hossain-Mahmud) diagonal storage (spmspm/paper_hm.cuh:18-37): diagonal d
// has length n - |d|; element (i, j) sits at position min(i, j).
struct HMMatrix {
    int                  n = 0;
    int                  num_diags = 0;
    std::vector<int>     diag_offsets;
    std::vector<int64_t> diag_starts;
    std::vector<int>     diag_lengths;
    std::vector<float>   values;
    int64_t              total_nz = 0;
};

// dense_to_hm (:41-65): the given offsets, in the given order.
inline HMMatrix dense_to_hm(const float* dense, int n, const std::vector<int>& offsets)
{
    HMMatrix hm;
    hm.n = n;
    hm.num_diags = static_cast<int>(offsets.size());
    hm.diag_offsets = offsets;
    int64_t off = 0;
    for (int d : offsets) {
        const int len = n - std::abs(d);
        const int sr = d >= 0 ? 0 : -d, sc = d >= 0 ? d : 0;
        hm.diag_starts.push_back(off);
        hm.diag_lengths.push_back(len);
        for (int p = 0; p < len; ++p)
            hm.values.push_back(dense[static_cast<size_t>(sr + p) * n + (sc + p)]);
        off += len;
    }
    hm.total_nz = off;
    return hm;
}

// hm_to_dense (:68-83).
inline void hm_to_dense(const HMMatrix& hm, float* dense)
{
    const int n = hm.n;
    std::memset(dense, 0, sizeof(float) * static_cast<size_t>(n) * n);
    for (int i = 0; i < hm.num_diags; ++i) {
        const int d = hm.diag_offsets[i];
        const int sr = d >= 0 ? 0 : -d, sc = d >= 0 ? d : 0;
        for (int p = 0; p < hm.diag_lengths[i]; ++p)
            dense[static_cast<size_t>(sr + p) * n + (sc + p)] = hm.values[hm.diag_starts[i] + p];
    }
}

// One pair-plan entry (spmspm/gather_flat.cuh:21); layout of diagpu_gpair.
struct GPair {
    size_t ab, bb;
    int ash, bsh, al, bl;
};
static_assert(sizeof(GPair) == sizeof(diagpu_gpair), "GPair must match diagpu_gpair");

// Pair plan (gather_flat.cuh:231): pairPtr has one entry per C diagonal + 1.
struct PairPlan {
    std::vector<int64_t> pairPtr;
    std::vector<GPair> pairs;
};

// Pair plan plus the flat tile list of gather_flat (:264): tiles (k, ts)
// every POS positions of each C diagonal.
struct FlatPlan {
    std::vector<int64_t> pairPtr;
    std::vector<GPair> pairs;
    std::vector<int2> tiles;
    int64_t nTiles = 0;
};

namespace diagpu {

// Everything the GPU symbolic phase produces, on the host.
struct SymbolicResult {
    std::vector<int> C_off, C_len;
    std::vector<int64_t> C_starts, pair_ptr;
    std::vector<GPair> pairs;
    std::vector<int> lookup;
    diagpu_spgemm_info info{};
};

// Run diagpu_spgemm_symbolic on host operand descriptions and bring every
// output back to the host (one stream sync).
inline SymbolicResult run_symbolic(int n, const std::vector<int>& A_off, const std::vector<int>& A_len,
                                   const std::vector<int64_t>& A_starts, const std::vector<int>& B_off,
                                   const std::vector<int>& B_len, const std::vector<int64_t>& B_starts,
                                   bool want_lookup)
{
    const int na = static_cast<int>(A_off.size()), nb = static_cast<int>(B_off.size());
    const int64_t ccap = std::max<int64_t>(1, std::min<int64_t>(int64_t(na) * nb, 2 * int64_t(n) - 1));
    const int64_t pcap = std::max<int64_t>(1, int64_t(na) * nb);
    DeviceArray<int> dAo(A_off), dAl(A_len), dBo(B_off), dBl(B_len);
    DeviceArray<int64_t> dAs(A_starts), dBs(B_starts);
    DeviceArray<int> dCo(ccap), dCl(ccap);
    DeviceArray<int64_t> dCs(ccap), dPtr(ccap + 1);
    DeviceArray<diagpu_gpair> dPairs(pcap);
    DeviceArray<int> dLk(want_lookup ? static_cast<size_t>(2 * int64_t(n) - 1) : 0);
    size_t ws_bytes = 0;
    check(diagpu_spgemm_symbolic_workspace(n, na, nb, &ws_bytes));
    DeviceArray<char> ws(ws_bytes);
    SymbolicResult r;
    check(diagpu_spgemm_symbolic(n, dAo.data(), dAl.data(), dAs.data(), na, dBo.data(), dBl.data(),
                                 dBs.data(), nb, dCo.data(), dCl.data(), dCs.data(), ccap,
                                 dPtr.data(), dPairs.data(), pcap,
                                 want_lookup ? dLk.data() : nullptr, ws.data(), ws_bytes, &r.info,
                                 nullptr));
    const size_t nc = static_cast<size_t>(r.info.c_ndiag);
    r.C_off = dCo.download(nc);
    r.C_len = dCl.download(nc);
    r.C_starts = dCs.download(nc);
    r.pair_ptr = dPtr.download(nc + 1);
    const auto gp = dPairs.download(static_cast<size_t>(r.info.n_pairs));
    r.pairs.resize(gp.size());
    if (!gp.empty()) std::memcpy(r.pairs.data(), gp.data(), gp.size() * sizeof(GPair));
    if (want_lookup) r.lookup = dLk.download();
    return r;
}

inline std::vector<int64_t> hm_starts(int n, const std::vector<int>& offsets)
{
    std::vector<int64_t> s;
    int64_t o = 0;
    for (int d : offsets) { s.push_back(o); o += n - std::abs(d); }
    return s;
}

}  // namespace diagpu

// compute_c_hm_structure (spmspm/paper_hm.cuh:87-117): every da + db inside
// the matrix, ascending, lengths n - |d|, starts the prefix sums, values zero.
inline HMMatrix compute_c_hm_structure(const HMMatrix& A, const HMMatrix& B, int n)
{
    const auto r = diagpu::run_symbolic(n, A.diag_offsets, A.diag_lengths, A.diag_starts,
                                        B.diag_offsets, B.diag_lengths, B.diag_starts, false);
    HMMatrix C;
    C.n = n;
    C.num_diags = static_cast<int>(r.C_off.size());
    C.diag_offsets = r.C_off;
    C.diag_lengths = r.C_len;
    C.diag_starts = r.C_starts;
    C.total_nz = r.info.c_nnz;
    C.values.assign(static_cast<size_t>(C.total_nz), 0.0f);
    return C;
}

// The bench's schedule types and planner under their reference names
// (spmspm/spmspm.cu:40-46, spmspm/bench_spmspm.cu:137-243), over HM
// operands and C (e.g. from compute_c_hm_structure).
using PairEntry = diagpu::PairEntry;
using Schedule = diagpu::Schedule;

inline Schedule build_schedule(const HMMatrix& A, const HMMatrix& B, const HMMatrix& C, int n)
{
    return diagpu::build_schedule(n, A.diag_offsets, B.diag_offsets, C.diag_offsets);
}

// build_c_diag_lookup (:121-130): lookup[d + n - 1] = C index, -1 elsewhere.
inline std::vector<int> build_c_diag_lookup(const HMMatrix& C, int n)
{
    std::vector<int> lookup(static_cast<size_t>(2 * int64_t(n) - 1), -1);
    for (int i = 0; i < C.num_diags; ++i) lookup[C.diag_offsets[i] + (n - 1)] = i;
    return lookup;
}

// build_pairs_only (spmspm/gather_flat.cuh:231-255) for the requested C
// offsets (each |dc| < n): per C diagonal, per B diagonal in B's order, the A
// diagonal with da = dc - db found through Alookup.
inline PairPlan build_pairs_only(int n, const std::vector<int>& A_len,
                                 const std::vector<size_t>& A_starts, const std::vector<int>& B_off,
                                 const std::vector<int>& B_len, const std::vector<size_t>& B_starts,
                                 const std::vector<int>& Alookup, const std::vector<int>& C_off)
{
    // The A offsets are the positions of the lookup's entries.
    std::vector<int> A_off(A_len.size(), 0);
    std::vector<char> seen(A_len.size(), 0);
    for (int64_t i = 0; i < int64_t(Alookup.size()); ++i) {
        const int ai = Alookup[static_cast<size_t>(i)];
        if (ai >= 0 && ai < int(A_off.size())) { A_off[ai] = int(i - (n - 1)); seen[ai] = 1; }
    }
    std::vector<int> A_off_used, A_len_used;
    std::vector<int64_t> A_st_used;
    for (size_t a = 0; a < A_off.size(); ++a)
        if (seen[a]) {
            A_off_used.push_back(A_off[a]);
            A_len_used.push_back(A_len[a]);
            A_st_used.push_back(static_cast<int64_t>(A_starts[a]));
        }
    const std::vector<int64_t> B_st(B_starts.begin(), B_starts.end());
    const auto r = diagpu::run_symbolic(n, A_off_used, A_len_used, A_st_used, B_off, B_len, B_st, true);
    PairPlan pp;
    pp.pairPtr.assign(C_off.size() + 1, 0);
    for (size_t k = 0; k < C_off.size(); ++k) {
        const int dc = C_off[k];
        if (dc <= -n || dc >= n) throw std::invalid_argument("build_pairs_only: |C offset| >= n");
        pp.pairPtr[k] = static_cast<int64_t>(pp.pairs.size());
        const int ci = r.lookup[static_cast<size_t>(dc + (n - 1))];
        if (ci < 0) continue;
        pp.pairs.insert(pp.pairs.end(), r.pairs.begin() + r.pair_ptr[ci],
                        r.pairs.begin() + r.pair_ptr[ci + 1]);
    }
    pp.pairPtr[C_off.size()] = static_cast<int64_t>(pp.pairs.size());
    return pp;
}

// build_flat_plan (gather_flat.cuh:264-292): the pair plan plus tiles.
inline FlatPlan build_flat_plan(int n, const std::vector<int>& A_off, const std::vector<int>& A_len,
                                const std::vector<size_t>& A_starts, const std::vector<int>& B_off,
                                const std::vector<int>& B_len, const std::vector<size_t>& B_starts,
                                const std::vector<int>& Alookup, const std::vector<int>& C_off,
                                const std::vector<int>& C_len, int POS)
{
    (void)A_off;
    PairPlan pp = build_pairs_only(n, A_len, A_starts, B_off, B_len, B_starts, Alookup, C_off);
    FlatPlan fp;
    fp.pairPtr = std::move(pp.pairPtr);
    fp.pairs = std::move(pp.pairs);
    for (size_t k = 0; k < C_off.size(); ++k)
        for (int ts = 0; ts < C_len[k]; ts += POS) fp.tiles.push_back(make_int2(int(k), ts));
    fp.nTiles = static_cast<int64_t>(fp.tiles.size());
    return fp;
}

namespace diagpu {

// Which numeric kernel SpgemmPlan::numeric runs for fp32 values.
//   Auto:        Band where the plan qualifies (SpgemmPlan::uses_band), else
//                AStationary where it qualifies (uses_astat), else Gather;
//   Gather:      diagpu_spgemm_numeric_f32, any plan;
//   Band:        diagpu_spgemm_numeric_band_f32 (operands staged in LDS;
//                narrow bands only, else diagpu::Error with DIAGPU_ERR_CAPACITY);
//   AStationary: diagpu_spgemm_numeric_astat_f32 (A held in LDS; at most
//                DIAGPU_ASTAT_MAX_A A diagonals, else DIAGPU_ERR_CAPACITY).
// All return the same bits.
enum class NumericKernel { Auto, Gather, Band, AStationary };

// Device-resident C = A * B for HM operands whose offsets, lengths and starts
// are device arrays: the plan is built once (symbolic), numeric() may run
// many times on new values with the same structure.  The plan keeps its own
// copies of the operands' offsets and starts; the caller's arrays need not
// outlive the constructor.
class SpgemmPlan {
public:
    SpgemmPlan(int n, const int* dA_off, const int* dA_len, const int64_t* dA_starts, int a_ndiag,
               const int* dB_off, const int* dB_len, const int64_t* dB_starts, int b_ndiag,
               bool want_lookup = false, hipStream_t stream = 0)
        : n_(n)
    {
        const int64_t ccap = std::max<int64_t>(1, std::min<int64_t>(int64_t(a_ndiag) * b_ndiag, 2 * int64_t(n) - 1));
        const int64_t pcap = std::max<int64_t>(1, int64_t(a_ndiag) * b_ndiag);
        C_off_.resize(ccap);
        C_len_.resize(ccap);
        C_starts_.resize(ccap);
        ptr_.resize(ccap + 1);
        pairs_.resize(pcap);
        if (want_lookup) lookup_.resize(static_cast<size_t>(2 * int64_t(n) - 1));
        size_t ws_bytes = 0;
        check(diagpu_spgemm_symbolic_workspace(n, a_ndiag, b_ndiag, &ws_bytes));
        DeviceArray<char> ws(ws_bytes);
        // Where the A-stationary kernel may take the plan, the symbolic call
        // also builds its records (diagpu_spgemm_symbolic_astat: one stream
        // synchronisation for both).
        const bool fused = int64_t(n) >= 4096 && int64_t(n) < (int64_t(1) << 30) &&
                           pcap < (int64_t(1) << 28) &&
                           a_ndiag <= std::max(DIAGPU_ASTAT_MAX_A, DIAGPU_ASTAT_MAX_A_C64);
        int32_t rstat = DIAGPU_OK;
        if (fused) {
            records_.resize(size_t(4 * pcap + 4));
            check(diagpu_spgemm_symbolic_astat(
                n, dA_off, dA_len, dA_starts, a_ndiag, dB_off, dB_len, dB_starts, b_ndiag,
                C_off_.data(), C_len_.data(), C_starts_.data(), ccap, ptr_.data(), pairs_.data(),
                pcap, want_lookup ? lookup_.data() : nullptr, ws.data(), ws_bytes,
                records_.data(), &rstat, &info_, stream));
            if (rstat != DIAGPU_OK && rstat != DIAGPU_ERR_CAPACITY) check(rstat);
            astat_prepared_ = rstat == DIAGPU_OK;
        } else {
            check(diagpu_spgemm_symbolic(n, dA_off, dA_len, dA_starts, a_ndiag, dB_off, dB_len,
                                         dB_starts, b_ndiag, C_off_.data(), C_len_.data(),
                                         C_starts_.data(), ccap, ptr_.data(), pairs_.data(), pcap,
                                         want_lookup ? lookup_.data() : nullptr, ws.data(),
                                         ws_bytes, &info_, stream));
        }
        nA_ = a_ndiag;
        nB_ = b_ndiag;
        A_off_.resize(a_ndiag);
        A_starts_.resize(a_ndiag);
        B_off_.resize(b_ndiag);
        B_starts_.resize(b_ndiag);
        copy_d2d(A_off_.data(), dA_off, a_ndiag, stream);
        copy_d2d(A_starts_.data(), dA_starts, a_ndiag, stream);
        copy_d2d(B_off_.data(), dB_off, b_ndiag, stream);
        copy_d2d(B_starts_.data(), dB_starts, b_ndiag, stream);
        // The band kernel's tables for plans the automatic choice may take
        // (one more stream synchronisation); others prepare on demand.
        band_auto_ = info_.c_ndiag > 0 && a_ndiag <= 65535 && b_ndiag <= 32767 &&
                     info_.n_pairs >= 3 * info_.c_ndiag && int64_t(n) >= 1024 * 256;
        if (band_auto_) prepare_band(stream);
        // The A-stationary kernel's records where the automatic choice may
        // take it.  The records serve both value types (the band kernel is
        // fp32 only); the rules are SpgemmPlan.uses_astat's in
        // diagpu_amd/spgemm.py, with the measurements behind them.
        const int64_t np = info_.n_pairs, nc = info_.c_ndiag, na = a_ndiag;
        const bool sized = nc > 0 && int64_t(n) >= 4096 && int64_t(n) < (int64_t(1) << 30) &&
                           nc < (int64_t(1) << 29) && np < (int64_t(1) << 28);
        const bool thin_mid = np < 16 && 2 * np >= 3 * nc && int64_t(n) >= (1 << 19) &&
                              int64_t(n) < (1 << 20);
        astat_auto_ = !uses_band() && sized && na <= DIAGPU_ASTAT_MAX_A && !thin_mid;
        astat_auto_c64_ = sized && na <= DIAGPU_ASTAT_MAX_A_C64 &&
                          (int64_t(n) >= (1 << 16) || np >= 3 * na);
        if (fused && rstat == DIAGPU_ERR_CAPACITY) {   // B indices beyond 2^30
            astat_auto_ = astat_auto_c64_ = false;
        } else if ((astat_auto_ || astat_auto_c64_) && !astat_prepared_) {
            try {
                prepare_astat(stream);
            } catch (const Error& e) {
                if (e.status != DIAGPU_ERR_CAPACITY) throw;   // B indices beyond 2^30
                astat_auto_ = astat_auto_c64_ = false;
            }
        }
    }

    // True where NumericKernel::Auto runs the band kernel for fp32 values:
    // the staged operands fit in LDS, the C diagonals average >= 3 plan
    // entries (each staged operand run then feeds several entries) and there
    // are >= 1024 row blocks of 256 (below that the A-stationary kernel or
    // the gather is faster).
    bool uses_band() const { return band_auto_ && band_.eligible; }
    // True where NumericKernel::Auto runs the A-stationary kernel for fp32
    // values: the band kernel does not take the plan, A has at most
    // DIAGPU_ASTAT_MAX_A diagonals, 4096 <= n < 2^30 (with fewer than 2^29 C
    // diagonals, 2^28 entries and 2^30 B values), and the plan is not one of
    // fewer than 16 entries and at least 1.5 per C diagonal at 2^19 <= n <
    // 2^20 (there the gather has more work per launch to hide its operand
    // reads: the tridiagonal square at n = 2^19 takes 10.2 us on the gather,
    // 13.4 on this kernel).
    bool uses_astat() const { return astat_auto_; }
    // The same for complex64 values: A has at most DIAGPU_ASTAT_MAX_A_C64
    // diagonals, 4096 <= n < 2^30, and n >= 2^16 or >= 3 entries per A diagonal.
    bool uses_astat_c64() const { return astat_auto_c64_; }

    // C_vals (device, info().c_nnz values) = A * B; asynchronous on `stream`
    // (NumericKernel::Band or AStationary on a plan not yet prepared for it
    // synchronises once to prepare).
    void numeric(const float* dA_vals, const float* dB_vals, float* dC_vals, hipStream_t stream = 0,
                 NumericKernel kernel = NumericKernel::Auto) const
    {
        if (kernel == NumericKernel::Auto)
            kernel = uses_band() ? NumericKernel::Band
                                 : (uses_astat() ? NumericKernel::AStationary : NumericKernel::Gather);
        if (kernel == NumericKernel::AStationary) {
            if (!astat_prepared_) prepare_astat(stream);
            check(diagpu_spgemm_numeric_astat_f32(
                n_, A_off_.data(), A_starts_.data(), nA_, dA_vals, dB_vals, C_off_.data(),
                C_len_.data(), C_starts_.data(), info_.c_ndiag, ptr_.data(), records_.data(),
                info_.n_pairs, dC_vals, stream));
            return;
        }
        if (kernel == NumericKernel::Band && !band_prepared_) prepare_band(stream);
        if (kernel == NumericKernel::Band) {
            check(diagpu_spgemm_numeric_band_f32(
                n_, A_off_.data(), A_starts_.data(), nA_, dA_vals, B_off_.data(), B_starts_.data(),
                nB_, dB_vals, C_off_.data(), C_starts_.data(), info_.c_ndiag, ptr_.data(),
                entries_.data(), &band_, dC_vals, stream));
            return;
        }
        check(diagpu_spgemm_numeric_f32(n_, dA_vals, dB_vals, C_off_.data(), C_len_.data(),
                                        C_starts_.data(), info_.c_ndiag, ptr_.data(), pairs_.data(),
                                        info_.max_pairs, dC_vals, stream));
    }

    // The same product with complex64 operands and C (same plan): Auto runs
    // the A-stationary kernel where uses_astat_c64(), else the gather; Band
    // is refused (fp32 only) with DIAGPU_ERR_ARG.
    void numeric(const diagpu_complex64* dA_vals, const diagpu_complex64* dB_vals,
                 diagpu_complex64* dC_vals, hipStream_t stream = 0,
                 NumericKernel kernel = NumericKernel::Auto) const
    {
        if (kernel == NumericKernel::Auto)
            kernel = uses_astat_c64() ? NumericKernel::AStationary : NumericKernel::Gather;
        if (kernel == NumericKernel::Band)
            throw Error(DIAGPU_ERR_ARG, "SpgemmPlan::numeric: the band kernel takes fp32 values only");
        if (kernel == NumericKernel::AStationary) {
            if (!astat_prepared_) prepare_astat(stream);
            check(diagpu_spgemm_numeric_astat_c64(
                n_, A_off_.data(), A_starts_.data(), nA_, dA_vals, dB_vals, C_off_.data(),
                C_len_.data(), C_starts_.data(), info_.c_ndiag, ptr_.data(), records_.data(),
                info_.n_pairs, dC_vals, stream));
            return;
        }
        check(diagpu_spgemm_numeric_c64(n_, dA_vals, dB_vals, C_off_.data(), C_len_.data(),
                                        C_starts_.data(), info_.c_ndiag, ptr_.data(), pairs_.data(),
                                        info_.max_pairs, dC_vals, stream));
    }

    // C_vals = (alpha A) B + sigma I in one pass on the A-stationary kernel
    // (diagpu_spgemm_numeric_astat_scaled_f32 / _c64: A scaled in LDS, sigma
    // added to C's main diagonal, none where C has no main diagonal);
    // asynchronous on `stream` (a plan not yet prepared for that kernel
    // synchronises once to prepare).  For any plan the kernel takes, as
    // numeric() with NumericKernel::AStationary (its limits are errors).
    void numeric_scaled(const float* dA_vals, float alpha, const float* dB_vals, float sigma,
                        float* dC_vals, hipStream_t stream = 0) const
    {
        if (!astat_prepared_) prepare_astat(stream);
        check(diagpu_spgemm_numeric_astat_scaled_f32(
            n_, A_off_.data(), A_starts_.data(), nA_, dA_vals, alpha, dB_vals, C_off_.data(),
            C_len_.data(), C_starts_.data(), info_.c_ndiag, ptr_.data(), records_.data(),
            info_.n_pairs, sigma, dC_vals, stream));
    }
    void numeric_scaled(const diagpu_complex64* dA_vals, diagpu_complex64 alpha,
                        const diagpu_complex64* dB_vals, diagpu_complex64 sigma,
                        diagpu_complex64* dC_vals, hipStream_t stream = 0) const
    {
        if (!astat_prepared_) prepare_astat(stream);
        check(diagpu_spgemm_numeric_astat_scaled_c64(
            n_, A_off_.data(), A_starts_.data(), nA_, dA_vals, alpha, dB_vals, C_off_.data(),
            C_len_.data(), C_starts_.data(), info_.c_ndiag, ptr_.data(), records_.data(),
            info_.n_pairs, sigma, dC_vals, stream));
    }

    const diagpu_spgemm_info& info() const { return info_; }
    const int* c_offsets() const { return C_off_.data(); }
    const int* c_lengths() const { return C_len_.data(); }
    const int64_t* c_starts() const { return C_starts_.data(); }
    const int64_t* pair_ptr() const { return ptr_.data(); }
    const diagpu_gpair* pairs() const { return pairs_.data(); }
    const int* c_lookup() const { return lookup_.size() ? lookup_.data() : nullptr; }

    // The grouped pair schedule of this plan (build_schedule,
    // spmspm/bench_spmspm.cu:137-243): the plan is copied to the host after
    // `stream` finishes and each C diagonal's entries re-ordered into A order
    // (schedule_from_plan).  Groups of t_diags C diagonals, n_tile-wide blocks.
    Schedule schedule(int t_diags = 8, int n_tile = 256, hipStream_t stream = 0) const
    {
        check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
        return schedule_from_plan(n_, A_starts_.download(), B_starts_.download(), info_.c_ndiag,
                                  ptr_.download(size_t(info_.c_ndiag + 1)),
                                  pairs_.download(size_t(info_.n_pairs)), t_diags, n_tile);
    }

private:
    template <typename T>
    static void copy_d2d(T* dst, const T* src, int count, hipStream_t stream)
    {
        if (count > 0)
            check_hip(hipMemcpyAsync(dst, src, size_t(count) * sizeof(T), hipMemcpyDeviceToDevice, stream),
                      "hipMemcpyAsync");
    }
    void prepare_band(hipStream_t stream) const
    {
        entries_.resize(size_t(4 * info_.n_pairs + 8));
        check(diagpu_spgemm_band_prepare(n_, A_off_.data(), A_starts_.data(), nA_, B_off_.data(),
                                         B_starts_.data(), nB_, pairs_.data(), info_.n_pairs,
                                         entries_.data(), &band_, stream));
        band_prepared_ = true;
    }
    void prepare_astat(hipStream_t stream) const
    {
        records_.resize(size_t(4 * info_.n_pairs + 4));
        check(diagpu_spgemm_astat_prepare(n_, A_off_.data(), A_starts_.data(), nA_, B_off_.data(),
                                          B_starts_.data(), nB_, C_off_.data(), ptr_.data(),
                                          info_.c_ndiag, pairs_.data(), info_.n_pairs,
                                          records_.data(), stream));
        astat_prepared_ = true;
    }

    int n_;
    int nA_ = 0, nB_ = 0;
    DeviceArray<int> C_off_, C_len_, lookup_, A_off_, B_off_;
    DeviceArray<int64_t> C_starts_, ptr_, A_starts_, B_starts_;
    DeviceArray<diagpu_gpair> pairs_;
    diagpu_spgemm_info info_{};
    bool band_auto_ = false;
    bool astat_auto_ = false;
    bool astat_auto_c64_ = false;
    mutable DeviceArray<int32_t> records_;
    mutable bool astat_prepared_ = false;
    mutable DeviceArray<int32_t> entries_;
    mutable diagpu_band_info band_{};
    mutable bool band_prepared_ = false;
};

}  // namespace diagpu

namespace diagpu {

// make_banded of the reference SpGEMM benchmark (spmspm/bench_spmspm.cu:89-106)
// as an HMMatrix: offsets -w..w ascending (those with n - |d| > 0), each
// diagonal's n - |d| values drawn in order from U(-1, 1) with
// std::mt19937(seed).  The draws are the reference's; the values equal its
// wherever the standard library's uniform_real_distribution is the same.
inline HMMatrix make_banded(int n, int w, unsigned seed)
{
    HMMatrix M;
    M.n = n;
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    int64_t start = 0;
    for (int d = -w; d <= w; ++d) {
        const int len = n - std::abs(d);
        if (len <= 0) continue;
        M.diag_offsets.push_back(d);
        M.diag_starts.push_back(start);
        M.diag_lengths.push_back(len);
        for (int p = 0; p < len; ++p) M.values.push_back(dist(rng));
        start += len;
    }
    M.num_diags = static_cast<int>(M.diag_offsets.size());
    M.total_nz = start;
    return M;
}

}  // namespace diagpu

// C = A * B for host HM matrices (upload, symbolic + numeric on the GPU,
// download): compute_c_hm_structure's C with its values filled.
inline HMMatrix spgemm_hm(const HMMatrix& A, const HMMatrix& B)
{
    using namespace diagpu;
    const int n = A.n;
    DeviceArray<int> ao(A.diag_offsets), al(A.diag_lengths), bo(B.diag_offsets), bl(B.diag_lengths);
    DeviceArray<int64_t> as(A.diag_starts), bs(B.diag_starts);
    DeviceArray<float> av(A.values), bv(B.values);
    SpgemmPlan plan(n, ao.data(), al.data(), as.data(), A.num_diags, bo.data(), bl.data(), bs.data(),
                    B.num_diags);
    const auto& inf = plan.info();
    DeviceArray<float> cv(static_cast<size_t>(inf.c_nnz));
    plan.numeric(av.data(), bv.data(), cv.data());
    check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
    HMMatrix C;
    C.n = n;
    C.num_diags = static_cast<int>(inf.c_ndiag);
    C.diag_offsets.resize(C.num_diags);
    C.diag_lengths.resize(C.num_diags);
    C.diag_starts.resize(C.num_diags);
    if (C.num_diags) {
        check_hip(hipMemcpy(C.diag_offsets.data(), plan.c_offsets(), sizeof(int) * C.num_diags, hipMemcpyDeviceToHost), "hipMemcpy");
        check_hip(hipMemcpy(C.diag_lengths.data(), plan.c_lengths(), sizeof(int) * C.num_diags, hipMemcpyDeviceToHost), "hipMemcpy");
        check_hip(hipMemcpy(C.diag_starts.data(), plan.c_starts(), sizeof(int64_t) * C.num_diags, hipMemcpyDeviceToHost), "hipMemcpy");
    }
    C.total_nz = inf.c_nnz;
    C.values = cv.download();
    return C;
}
