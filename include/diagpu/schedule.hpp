// The grouped pair schedule of the reference's SpGEMM bench (host C++, no
// HIP dependency): PairEntry (spmspm/spmspm.cu:40-46) and Schedule /
// build_schedule (spmspm/bench_spmspm.cu:137-243), with the same members,
// padding and block mapping, for callers that feed a group-tiled kernel of
// their own.  (This library's LDS-tiled numeric phase, the band kernel, takes
// the pair plan instead: it stages a row block's operand windows, so it has no
// global halo and also runs products whose offsets are too wide for one.)
//
// The C diagonals are taken in groups of t_diags consecutive ones.  Within a
// group, for each C diagonal in order and each A diagonal in A's order whose
// partner offset db = dc - da is a B diagonal, one PairEntry
//   {a_local, b_local, c_local, a_shift = min0(da) - min0(dc),
//    b_shift = da + min0(db) - min0(dc)}
// where a_local / b_local number the group's A / B diagonals in order of first
// use.  a_halo / b_halo are the largest |a_shift| / |b_shift| of all groups.
// The per-group lists are padded to the largest group and stored
// group-strided (zeros in the padding); block b works on group
// block_group[b] and C positions [block_tile[b], block_tile[b] + n_tile).
//
// The shifts are the GPair shifts ash / bsh of the pair plan
// (spmspm/gather_flat.cuh:231-255) of the same (dc, da, db), so
// schedule_from_plan builds the schedule from a plan the GPU symbolic phase
// made, re-ordering each C diagonal's entries from B order to A order.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <utility>
#include <vector>

#include "diagpu.h"

namespace diagpu {

// Same members, order and types as PairEntry (spmspm/spmspm.cu:40-46).
struct PairEntry {
    int a_local;
    int b_local;
    int c_local;
    int a_shift;
    int b_shift;
};

// Same members as Schedule (spmspm/bench_spmspm.cu:137-146).
struct Schedule {
    int a_halo = 0, b_halo = 0;
    int num_groups = 0;
    int max_a = 0, max_b = 0, max_pairs = 0;
    int num_ntiles = 0, num_blocks = 0;
    std::vector<int> a_count, b_count, pair_count, t_out;
    std::vector<int> a_globals, b_globals, c_globals;   // padded, group-strided
    std::vector<PairEntry> pairs;                      // padded, group-strided
    std::vector<int> block_group, block_tile;
};

namespace detail {

// One plan entry of C diagonal c: A diagonal a, B diagonal b, its shifts.
struct SchedEntry {
    int a, b, ash, bsh;
};

// Groups, locals, padding and blocks from each C diagonal's entries, already
// in A order (entries[ptr[c] .. ptr[c + 1])).
inline Schedule assemble(int n, int nA, int nB, int nC, const std::vector<int64_t>& ptr,
                         const std::vector<SchedEntry>& entries, int t_diags, int n_tile)
{
    if (t_diags < 1 || n_tile < 1) throw std::invalid_argument("build_schedule: t_diags, n_tile >= 1");
    Schedule S;
    S.num_groups = (nC + t_diags - 1) / t_diags;
    const int G = S.num_groups;
    S.a_count.assign(G, 0);
    S.b_count.assign(G, 0);
    S.pair_count.assign(G, 0);
    S.t_out.assign(G, 0);
    // first use of an A / B diagonal within group g: stamp == g
    std::vector<int> a_stamp(nA, -1), a_loc(nA), b_stamp(nB, -1), b_loc(nB);
    std::vector<std::vector<int>> ga(G), gb(G);
    for (int g = 0; g < G; ++g) {
        const int c0 = g * t_diags, c1 = std::min(nC, c0 + t_diags);
        S.t_out[g] = c1 - c0;
        for (int64_t q = ptr[c0]; q < ptr[c1]; ++q) {
            const SchedEntry& e = entries[q];
            if (a_stamp[e.a] != g) { a_stamp[e.a] = g; a_loc[e.a] = (int)ga[g].size(); ga[g].push_back(e.a); }
            if (b_stamp[e.b] != g) { b_stamp[e.b] = g; b_loc[e.b] = (int)gb[g].size(); gb[g].push_back(e.b); }
            S.a_halo = std::max(S.a_halo, std::abs(e.ash));
            S.b_halo = std::max(S.b_halo, std::abs(e.bsh));
        }
        S.a_count[g] = (int)ga[g].size();
        S.b_count[g] = (int)gb[g].size();
        S.pair_count[g] = (int)(ptr[c1] - ptr[c0]);
        S.max_a = std::max(S.max_a, S.a_count[g]);
        S.max_b = std::max(S.max_b, S.b_count[g]);
        S.max_pairs = std::max(S.max_pairs, S.pair_count[g]);
    }
    S.a_globals.assign(size_t(G) * S.max_a, 0);
    S.b_globals.assign(size_t(G) * S.max_b, 0);
    S.c_globals.assign(size_t(G) * t_diags, 0);
    S.pairs.assign(size_t(G) * S.max_pairs, PairEntry{0, 0, 0, 0, 0});
    for (int g = 0; g < G; ++g) {
        std::copy(ga[g].begin(), ga[g].end(), S.a_globals.begin() + size_t(g) * S.max_a);
        std::copy(gb[g].begin(), gb[g].end(), S.b_globals.begin() + size_t(g) * S.max_b);
        const int c0 = g * t_diags;
        for (int c = 0; c < S.t_out[g]; ++c) S.c_globals[size_t(g) * t_diags + c] = c0 + c;
        // local indices of this group (the stamps are rewritten per group)
        for (size_t i = 0; i < ga[g].size(); ++i) a_loc[ga[g][i]] = (int)i;
        for (size_t i = 0; i < gb[g].size(); ++i) b_loc[gb[g][i]] = (int)i;
        PairEntry* out = S.pairs.data() + size_t(g) * S.max_pairs;
        for (int c = 0; c < S.t_out[g]; ++c)
            for (int64_t q = ptr[c0 + c]; q < ptr[c0 + c + 1]; ++q) {
                const SchedEntry& e = entries[q];
                *out++ = PairEntry{a_loc[e.a], b_loc[e.b], c, e.ash, e.bsh};
            }
    }
    S.num_ntiles = (int)((int64_t(n) + n_tile - 1) / n_tile);
    S.num_blocks = G * S.num_ntiles;
    S.block_group.resize(S.num_blocks);
    S.block_tile.resize(S.num_blocks);
    for (int g = 0; g < G; ++g)
        for (int t = 0; t < S.num_ntiles; ++t) {
            S.block_group[size_t(g) * S.num_ntiles + t] = g;
            S.block_tile[size_t(g) * S.num_ntiles + t] = t * n_tile;
        }
    return S;
}

inline int min0(int x) { return x < 0 ? x : 0; }

}  // namespace detail

// build_schedule(A, B, C, n) of spmspm/bench_spmspm.cu:147 on the operands'
// and C's diagonal offsets (in their stored order; a B offset held twice
// resolves to its last index, as the reference's offset map does).
inline Schedule build_schedule(int n, const std::vector<int>& A_off, const std::vector<int>& B_off,
                               const std::vector<int>& C_off, int t_diags = 8, int n_tile = 256)
{
    // B offsets sorted, each with its last index
    std::vector<std::pair<int, int>> bs;
    for (int i = 0; i < (int)B_off.size(); ++i) bs.emplace_back(B_off[i], i);
    std::stable_sort(bs.begin(), bs.end(),
                     [](const std::pair<int, int>& x, const std::pair<int, int>& y) { return x.first < y.first; });
    const int nC = (int)C_off.size();
    std::vector<int64_t> ptr(nC + 1, 0);
    std::vector<detail::SchedEntry> entries;
    for (int c = 0; c < nC; ++c) {
        const int dc = C_off[c];
        for (int a = 0; a < (int)A_off.size(); ++a) {
            const int64_t db64 = int64_t(dc) - A_off[a];
            if (db64 <= -int64_t(n) || db64 >= n) continue;
            const int db = (int)db64;
            auto hi = std::upper_bound(bs.begin(), bs.end(), db,
                                       [](int v, const std::pair<int, int>& p) { return v < p.first; });
            if (hi == bs.begin() || (hi - 1)->first != db) continue;
            const int da = A_off[a];
            entries.push_back({a, (hi - 1)->second, detail::min0(da) - detail::min0(dc),
                               da + detail::min0(db) - detail::min0(dc)});
        }
        ptr[c + 1] = (int64_t)entries.size();
    }
    return detail::assemble(n, (int)A_off.size(), (int)B_off.size(), nC, ptr, entries, t_diags,
                            n_tile);
}

// The same schedule from a pair plan (host copies of what
// diagpu_spgemm_symbolic wrote: nC C diagonals, pair_ptr, pairs) and the
// operands' starts, which identify each entry's A and B diagonal.
inline Schedule schedule_from_plan(int n, const std::vector<int64_t>& A_starts,
                                   const std::vector<int64_t>& B_starts, int64_t nC,
                                   const std::vector<int64_t>& pair_ptr,
                                   const std::vector<diagpu_gpair>& pairs, int t_diags = 8,
                                   int n_tile = 256)
{
    auto index_of = [](const std::vector<int64_t>& starts) {
        std::vector<std::pair<int64_t, int>> v;
        for (int i = 0; i < (int)starts.size(); ++i) v.emplace_back(starts[i], i);
        std::sort(v.begin(), v.end());
        return v;
    };
    const auto as = index_of(A_starts), bs = index_of(B_starts);
    auto find = [](const std::vector<std::pair<int64_t, int>>& v, uint64_t s) {
        auto it = std::lower_bound(v.begin(), v.end(), std::make_pair((int64_t)s, -1));
        if (it == v.end() || it->first != (int64_t)s)
            throw std::invalid_argument("schedule_from_plan: a plan entry's start is no operand diagonal's start");
        return it->second;
    };
    std::vector<detail::SchedEntry> entries(pairs.size());
    for (size_t q = 0; q < pairs.size(); ++q)
        entries[q] = {find(as, pairs[q].ab), find(bs, pairs[q].bb), pairs[q].ash, pairs[q].bsh};
    // each C diagonal's entries from B order into A order
    for (int64_t c = 0; c < nC; ++c)
        std::sort(entries.begin() + pair_ptr[c], entries.begin() + pair_ptr[c + 1],
                  [](const detail::SchedEntry& x, const detail::SchedEntry& y) { return x.a < y.a; });
    return detail::assemble(n, (int)A_starts.size(), (int)B_starts.size(), (int)nC, pair_ptr,
                            entries, t_diags, n_tile);
}

}  // namespace diagpu
