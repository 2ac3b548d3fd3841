// CPU test of include/diagpu/schedule.hpp: build_schedule (offsets) and
// schedule_from_plan (a pair plan, here the oracle's build_pairs_only) against
// the oracle's restatement of the reference planner (orc_build_schedule,
// pinned to spmspm/bench_spmspm.cu:137-243 by tests/golden/schedule.json),
// every member compared, on the bench's make_banded(100000, 16) operands,
// BASELINE config 4 and 5 shapes and random offset sets.
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "diagpu/schedule.hpp"

extern "C" {
int orc_c_structure(int n, const int* A_off, int nA, const int* B_off, int nB, int* C_off,
                    int* C_len, int64_t* C_starts, int64_t* nnz);
int64_t orc_pairs_only(int n, const int* A_off, int nA, const int* A_len, const int64_t* A_starts,
                       const int* B_off, int nB, const int* B_len, const int64_t* B_starts,
                       const int* C_off, int nC, int64_t* pair_ptr, void* pairs);
void orc_build_schedule(int n, const int* A_off, int nA, const int* B_off, int nB,
                        const int* C_off, int nC, int T, int n_tile, int* scalars, int* a_count,
                        int* b_count, int* pair_count, int* t_out, int* a_globals, int* b_globals,
                        int* c_globals, void* pairs, int* block_group, int* block_tile);
}

static bool g_all = true;

static bool same(const diagpu::Schedule& x, const diagpu::Schedule& y)
{
    return x.a_halo == y.a_halo && x.b_halo == y.b_halo && x.num_groups == y.num_groups &&
           x.max_a == y.max_a && x.max_b == y.max_b && x.max_pairs == y.max_pairs &&
           x.num_ntiles == y.num_ntiles && x.num_blocks == y.num_blocks && x.a_count == y.a_count &&
           x.b_count == y.b_count && x.pair_count == y.pair_count && x.t_out == y.t_out &&
           x.a_globals == y.a_globals && x.b_globals == y.b_globals && x.c_globals == y.c_globals &&
           x.pairs.size() == y.pairs.size() &&
           std::memcmp(x.pairs.data(), y.pairs.data(), x.pairs.size() * sizeof(diagpu::PairEntry)) == 0 &&
           x.block_group == y.block_group && x.block_tile == y.block_tile;
}

static diagpu::Schedule oracle_schedule(int n, const std::vector<int>& a, const std::vector<int>& b,
                                        const std::vector<int>& c, int T, int tile)
{
    int sc[8];
    orc_build_schedule(n, a.data(), (int)a.size(), b.data(), (int)b.size(), c.data(), (int)c.size(),
                       T, tile, sc, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, nullptr);
    diagpu::Schedule S;
    S.a_halo = sc[0]; S.b_halo = sc[1]; S.num_groups = sc[2]; S.max_a = sc[3]; S.max_b = sc[4];
    S.max_pairs = sc[5]; S.num_ntiles = sc[6]; S.num_blocks = sc[7];
    const size_t G = S.num_groups;
    S.a_count.resize(G); S.b_count.resize(G); S.pair_count.resize(G); S.t_out.resize(G);
    S.a_globals.resize(G * S.max_a); S.b_globals.resize(G * S.max_b); S.c_globals.resize(G * T);
    S.pairs.resize(G * S.max_pairs);
    S.block_group.resize(S.num_blocks); S.block_tile.resize(S.num_blocks);
    orc_build_schedule(n, a.data(), (int)a.size(), b.data(), (int)b.size(), c.data(), (int)c.size(),
                       T, tile, sc, S.a_count.data(), S.b_count.data(), S.pair_count.data(),
                       S.t_out.data(), S.a_globals.data(), S.b_globals.data(), S.c_globals.data(),
                       S.pairs.data(), S.block_group.data(), S.block_tile.data());
    return S;
}

static void check(const char* name, int n, const std::vector<int>& a, const std::vector<int>& b,
                  int T = 8, int tile = 256)
{
    const int cap = (int)std::min<int64_t>(int64_t(a.size()) * b.size(), 2 * int64_t(n) - 1);
    std::vector<int> c(cap), cl(cap);
    std::vector<int64_t> cs(cap);
    int64_t nnz = 0;
    c.resize(orc_c_structure(n, a.data(), (int)a.size(), b.data(), (int)b.size(), c.data(),
                             cl.data(), cs.data(), &nnz));
    const diagpu::Schedule want = oracle_schedule(n, a, b, c, T, tile);
    const diagpu::Schedule got = diagpu::build_schedule(n, a, b, c, T, tile);
    // the plan route: lengths and starts of A and B in their stored order
    auto layout = [n](const std::vector<int>& off, std::vector<int>& len, std::vector<int64_t>& st) {
        int64_t s = 0;
        for (int d : off) {
            len.push_back(n - std::abs(d));
            st.push_back(s);
            s += n - std::abs(d);
        }
    };
    std::vector<int> al, bl;
    std::vector<int64_t> ast, bst;
    layout(a, al, ast);
    layout(b, bl, bst);
    std::vector<int64_t> ptr(c.size() + 1);
    const int64_t np = orc_pairs_only(n, a.data(), (int)a.size(), al.data(), ast.data(), b.data(),
                                      (int)b.size(), bl.data(), bst.data(), c.data(), (int)c.size(),
                                      ptr.data(), nullptr);
    std::vector<diagpu_gpair> pairs(np);
    orc_pairs_only(n, a.data(), (int)a.size(), al.data(), ast.data(), b.data(), (int)b.size(),
                   bl.data(), bst.data(), c.data(), (int)c.size(), ptr.data(), pairs.data());
    const diagpu::Schedule from_plan =
        diagpu::schedule_from_plan(n, ast, bst, (int64_t)c.size(), ptr, pairs, T, tile);
    const bool ok = same(got, want) && same(from_plan, want);
    std::printf("  %-44s %s groups=%d halos=(%d,%d) max=(%d,%d,%d)\n", name, ok ? "[OK]" : "[FAIL]",
                want.num_groups, want.a_halo, want.b_halo, want.max_a, want.max_b, want.max_pairs);
    g_all &= ok;
}

static std::vector<int> range(int lo, int hi)
{
    std::vector<int> v;
    for (int d = lo; d <= hi; ++d) v.push_back(d);
    return v;
}

static std::vector<int> draw(std::mt19937& g, int count, int span)
{
    std::vector<int> v;
    std::uniform_int_distribution<int> u(-span, span);
    while ((int)v.size() < count) {
        const int d = u(g);
        if (std::find(v.begin(), v.end(), d) == v.end()) v.push_back(d);
    }
    return v;
}

int main()
{
    std::printf("grouped pair schedule (schedule.hpp) vs oracle\n");
    check("bench make_banded(100000, 16) offsets", 100000, range(-16, 16), range(-16, 16));
    check("config 4 (band -4..4 x 7-point stencil)", 1 << 20, range(-4, 4),
          {-16384, -128, -1, 0, 1, 128, 16384});
    check("offsets reaching past n (n = 6, w = 4)", 6, range(-4, 4), range(-4, 4));
    check("T = 3, tile = 100", 5000, range(-7, 7), {-40, -3, 0, 9});
    std::mt19937 g(7);
    for (int rep = 0; rep < 6; ++rep) {
        const int n = 50 + 997 * rep;
        auto a = draw(g, 3 + 5 * rep, std::min(n - 1, 300 * (rep + 1)));
        auto b = draw(g, 2 + 4 * rep, std::min(n - 1, 200 * (rep + 1)));   // unsorted B
        char name[64];
        std::snprintf(name, sizeof name, "random n=%d |A|=%zu |B|=%zu", n, a.size(), b.size());
        check(name, n, a, b);
    }
    std::vector<int> a5 = draw(g, 128, 4096), b5 = draw(g, 128, 4096);
    std::sort(a5.begin(), a5.end());
    std::sort(b5.begin(), b5.end());
    check("config 5 shape (128 x 128 in +-4096)", 262144, a5, b5);
    std::printf(g_all ? "ALL TESTS PASSED\n" : "SOME TESTS FAILED\n");
    return g_all ? 0 : 1;
}
