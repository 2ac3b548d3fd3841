/*
 * ref_schedule.cpp -- driver around the reference's SpGEMM host planner.
 *
 * TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (target `ref`) where the
 * reference checkout exists, run only by tests/golden/make_schedule_golden.py
 * to write the fixture that pins the oracle's restatement of the grouped pair
 * schedule (orc_build_schedule) and of the C structure.  Nothing in the
 * product or on the GPU box runs it.
 *
 * The planner is not in this file: the Makefile cuts it out of the reference
 * sources by line range into a temporary directory and this driver includes
 * it, so the program runs the reference's text as written:
 *   ref_cfg.inc          T_DIAGS, N_TILE, THREADS   spmspm/bench_spmspm.cu:49-60
 *   ref_min0.inc         min0                       spmspm/bench_spmspm.cu:72
 *   ref_make_banded.inc  DiaMatrix, make_banded     spmspm/bench_spmspm.cu:79-106
 *   ref_c_structure.inc  make_c_structure           spmspm/bench_spmspm.cu:109-131
 *   ref_pair_entry.inc   PairEntry                  spmspm/spmspm.cu:40-46
 *   ref_schedule.inc     Schedule, build_schedule   spmspm/bench_spmspm.cu:137-243
 *
 * Usage (text on stdout, one array per line, "name count v0 v1 ..."):
 *   banded n w seedA seedB       A = make_banded(n, w, seedA), B likewise
 *   offsets n nA a... b...       A and B with the given offsets (values unused)
 * prints the C offsets of make_c_structure(A, B), then every member of
 * build_schedule(A, B, C, n).
 */
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "ref_cfg.inc"
#include "ref_min0.inc"
#include "ref_make_banded.inc"
#include "ref_c_structure.inc"
#include "ref_pair_entry.inc"
#include "ref_schedule.inc"

static void line(const char* name, const std::vector<int>& v)
{
    std::printf("%s %zu", name, v.size());
    for (int x : v) std::printf(" %d", x);
    std::printf("\n");
}

static DiaMatrix with_offsets(int n, const std::vector<int>& offs)
{
    DiaMatrix M;
    M.n = n;
    M.offsets = offs;
    for (int d : offs) M.lengths.push_back(n - std::abs(d));
    return M;
}

int main(int argc, char** argv)
{
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s banded n w seedA seedB | offsets n nA a... b...\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    const int n = std::atoi(argv[2]);
    DiaMatrix A, B;
    if (mode == "banded" && argc == 6) {
        const int w = std::atoi(argv[3]);
        A = make_banded(n, w, (unsigned)std::strtoul(argv[4], nullptr, 10));
        B = make_banded(n, w, (unsigned)std::strtoul(argv[5], nullptr, 10));
    } else if (mode == "offsets" && argc >= 4) {
        const int na = std::atoi(argv[3]);
        std::vector<int> a, b;
        for (int i = 4; i < argc; ++i) (i < 4 + na ? a : b).push_back(std::atoi(argv[i]));
        A = with_offsets(n, a);
        B = with_offsets(n, b);
    } else {
        std::fprintf(stderr, "bad arguments\n");
        return 2;
    }
    const DiaMatrix C = make_c_structure(A, B);
    const Schedule S = build_schedule(A, B, C, n);
    line("c_offsets", C.offsets);
    line("scalars", {S.a_halo, S.b_halo, S.num_groups, S.max_a, S.max_b, S.max_pairs,
                     S.num_ntiles, S.num_blocks, T_DIAGS, N_TILE});
    line("a_count", S.a_count);
    line("b_count", S.b_count);
    line("pair_count", S.pair_count);
    line("t_out", S.t_out);
    line("a_globals", S.a_globals);
    line("b_globals", S.b_globals);
    line("c_globals", S.c_globals);
    std::vector<int> p;
    for (const PairEntry& e : S.pairs) {
        p.push_back(e.a_local);
        p.push_back(e.b_local);
        p.push_back(e.c_local);
        p.push_back(e.a_shift);
        p.push_back(e.b_shift);
    }
    line("pairs", p);
    line("block_group", S.block_group);
    line("block_tile", S.block_tile);
    return std::fflush(stdout) == 0 ? 0 : 1;
}
