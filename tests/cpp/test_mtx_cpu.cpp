// CPU test of include/diagpu/mtx.hpp: the band writer reproduces the
// reference's gen_banded_mtx output byte for byte (golden file and, where it
// is built, the live reference program); the reader inverts it.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "diagpu/mtx.hpp"

extern "C" float orc_hval(int r, int d);

static std::string slurp(const std::string& p)
{
    std::ifstream f(p, std::ios::binary);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// The SpMV bench's 9-diagonal hash band (spmv/bench/bench_cusparse.cu:84-87).
static diagpu::MtxBand hash_band(int N)
{
    diagpu::MtxBand B;
    B.rows = B.cols = N;
    const int offs[] = {9, -9, 0, 5, -5, 2, -2, 1, -1};   // any order: written ascending
    int64_t s = 0;
    for (int d : offs) {
        B.offsets.push_back(d);
        B.starts.push_back(s);
        const int sr = d >= 0 ? 0 : -d;
        const int len = N - (d >= 0 ? d : -d);
        for (int j = 0; j < len; ++j) B.values.push_back(orc_hval(sr + j, d));
        s += len;
    }
    return B;
}

int main(int argc, char** argv)
{
    if (argc < 3) { std::fprintf(stderr, "usage: %s golden_n64.mtx tmpdir [ref_gen_banded_mtx]\n", argv[0]); return 2; }
    bool ok = true;
    const std::string tmp = std::string(argv[2]) + "/w64.mtx";
    diagpu::write_mtx_band(tmp, hash_band(64));
    const bool same = slurp(tmp) == slurp(argv[1]);
    std::printf("  writer == reference output (N=64, golden)   %s\n", same ? "[OK]" : "[FAIL]");
    ok &= same;
    if (argc > 3) {
        const std::string ref = std::string(argv[2]) + "/ref300.mtx", mine = std::string(argv[2]) + "/w300.mtx";
        const std::string cmd = std::string(argv[3]) + " 300 " + ref + " 2>/dev/null";
        const bool ran = std::system(cmd.c_str()) == 0;
        diagpu::write_mtx_band(mine, hash_band(300));
        const bool s2 = ran && slurp(ref) == slurp(mine);
        std::printf("  writer == live reference program (N=300)    %s\n", s2 ? "[OK]" : "[FAIL]");
        ok &= s2;
    }
    // reader: back to compact DIA with the hash values
    const diagpu::MtxDia D = diagpu::read_mtx_dia(argv[1]);
    bool rd = D.rows == 64 && D.cols == 64 &&
              D.offsets == std::vector<int>({-9, -5, -2, -1, 0, 1, 2, 5, 9});
    for (size_t k = 0; rd && k < D.offsets.size(); ++k) {
        const int d = D.offsets[k], sr = d >= 0 ? 0 : -d;
        rd &= D.lengths[k] == 64 - (d >= 0 ? d : -d);
        for (int j = 0; rd && j < D.lengths[k]; ++j) {
            char a[32], b[32];
            std::snprintf(a, sizeof a, "%.7g", (double)D.values[D.starts[k] + j]);
            std::snprintf(b, sizeof b, "%.7g", (double)orc_hval(sr + j, d));
            rd &= std::strcmp(a, b) == 0;
        }
    }
    std::printf("  reader recovers offsets, lengths, values    %s\n", rd ? "[OK]" : "[FAIL]");
    ok &= rd;
    // symmetric + pattern + duplicates
    const std::string sp = std::string(argv[2]) + "/sym.mtx";
    {
        FILE* f = std::fopen(sp.c_str(), "w");
        std::fprintf(f, "%%%%MatrixMarket matrix coordinate real symmetric\n%% c\n4 4 5\n1 1 2\n2 1 -1\n3 2 -1\n3 2 -0.5\n4 4 7\n");
        std::fclose(f);
    }
    const diagpu::MtxDia S = diagpu::read_mtx_dia(sp);
    bool sy = S.offsets == std::vector<int>({-1, 0, 1}) && S.values.size() == 3 + 4 + 3;
    // diag -1: rows 1..3 -> (2,1)=-1, (3,2)=-1.5, (4,3)=0; diag 0: 2,0,0,7; diag +1 mirrored
    const std::vector<float> want = {-1, -1.5f, 0, 2, 0, 0, 7, -1, -1.5f, 0};
    sy &= S.values == want;
    std::printf("  reader: symmetric expansion, duplicates     %s\n", sy ? "[OK]" : "[FAIL]");
    ok &= sy;
    std::printf("%s\n", ok ? "ALL TESTS PASSED" : "SOME TESTS FAILED");
    return ok ? 0 : 1;
}
