// MatrixMarket I/O for diagonal matrices (host C++, no HIP dependency).
//
// write_mtx_band writes the coordinate format of spmv/tools/gen_banded_mtx.cpp
// (:37-48): header, a "% banded, offsets {...}" comment, "rows cols nnz",
// then every in-range entry of the listed diagonals row by row, offsets
// ascending within a row, 1-based indices, values as "%.7g" of the float
// widened to double.  Given the same diagonals and values its output is byte
// for byte the reference program's.
//
// read_mtx_dia reads "matrix coordinate real|integer|pattern general|symmetric"
// files into the compact DIA form of spmv/src/dia_reconstruct.cuh:52-59
// (offsets ascending, one diagonal per distinct c - r, structural entries
// kept even when their value is zero); duplicate entries are summed.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace diagpu {

// A band given by its diagonals: value(row, d) for 0 <= row, row + d < n.
struct MtxBand {
    int rows = 0, cols = 0;
    std::vector<int> offsets;            // any order; written ascending
    std::vector<int64_t> starts;         // element j of diagonal k at values[starts[k] + j]
    std::vector<float> values;           // element j is row max(-d, 0) + j
};

inline void write_mtx_band(const std::string& path, const MtxBand& B)
{
    std::vector<int> order(B.offsets.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<int>(i);
    std::sort(order.begin(), order.end(), [&](int a, int b) { return B.offsets[a] < B.offsets[b]; });
    int64_t nnz = 0;
    for (int k : order) {
        const int d = B.offsets[k];
        const int64_t r0 = std::max(0, -d), r1 = std::min<int64_t>(B.rows, int64_t(B.cols) - d);
        if (r1 > r0) nnz += r1 - r0;
    }
    FILE* f = std::fopen(path.c_str(), "w");
    if (!f) throw std::runtime_error("write_mtx_band: cannot open " + path);
    std::fprintf(f, "%%%%MatrixMarket matrix coordinate real general\n");
    std::fprintf(f, "%% banded, offsets {");
    for (size_t i = 0; i < order.size(); ++i)
        std::fprintf(f, "%s%d", i ? "," : "", B.offsets[order[i]]);
    std::fprintf(f, "}\n");
    std::fprintf(f, "%d %d %lld\n", B.rows, B.cols, static_cast<long long>(nnz));
    for (int r = 0; r < B.rows; ++r)
        for (int k : order) {
            const int d = B.offsets[k];
            const int64_t c = int64_t(r) + d;
            if (c < 0 || c >= B.cols) continue;
            const int64_t j = r - std::max(0, -d);
            std::fprintf(f, "%d %lld %.7g\n", r + 1, static_cast<long long>(c + 1),
                         static_cast<double>(B.values[B.starts[k] + j]));
        }
    std::fclose(f);
}

// Compact DIA read from a MatrixMarket file.
struct MtxDia {
    int rows = 0, cols = 0;
    std::vector<int> offsets;        // ascending
    std::vector<int64_t> starts;
    std::vector<int> lengths;        // min(rows - sr, cols - sc)
    std::vector<float> values;
};

inline MtxDia read_mtx_dia(const std::string& path)
{
    FILE* f = std::fopen(path.c_str(), "r");
    if (!f) throw std::runtime_error("read_mtx_dia: cannot open " + path);
    char line[4096];
    if (!std::fgets(line, sizeof line, f)) { std::fclose(f); throw std::runtime_error("read_mtx_dia: empty file"); }
    std::string banner(line);
    for (auto& ch : banner) ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
    if (banner.rfind("%%matrixmarket", 0) != 0 || banner.find("coordinate") == std::string::npos) {
        std::fclose(f);
        throw std::runtime_error("read_mtx_dia: not a coordinate MatrixMarket file");
    }
    const bool pattern = banner.find("pattern") != std::string::npos;
    const bool symmetric = banner.find("symmetric") != std::string::npos;
    if (banner.find("complex") != std::string::npos) {
        std::fclose(f);
        throw std::runtime_error("read_mtx_dia: complex entries are not supported");
    }
    long long rows = 0, cols = 0, nnz = 0;
    while (std::fgets(line, sizeof line, f)) {
        if (line[0] == '%' || line[0] == '\n') continue;
        if (std::sscanf(line, "%lld %lld %lld", &rows, &cols, &nnz) != 3) {
            std::fclose(f);
            throw std::runtime_error("read_mtx_dia: bad size line");
        }
        break;
    }
    if (rows <= 0 || cols <= 0 || rows > (1ll << 30) || cols > (1ll << 30)) {
        std::fclose(f);
        throw std::runtime_error("read_mtx_dia: unsupported dimensions");
    }
    // offset -> (row -> value), rows ascending within a diagonal
    std::map<int, std::map<int, double>> diags;
    for (long long e = 0; e < nnz; ++e) {
        if (!std::fgets(line, sizeof line, f)) { std::fclose(f); throw std::runtime_error("read_mtx_dia: truncated"); }
        long long r = 0, c = 0;
        double v = 1.0;
        const int got = pattern ? std::sscanf(line, "%lld %lld", &r, &c)
                                : std::sscanf(line, "%lld %lld %lf", &r, &c, &v);
        if (got < (pattern ? 2 : 3) || r < 1 || c < 1 || r > rows || c > cols) {
            std::fclose(f);
            throw std::runtime_error("read_mtx_dia: bad entry line");
        }
        diags[int(c - r)][int(r - 1)] += v;
        if (symmetric && r != c) diags[int(r - c)][int(c - 1)] += v;
    }
    std::fclose(f);
    MtxDia D;
    D.rows = int(rows);
    D.cols = int(cols);
    int64_t off = 0;
    for (const auto& [d, entries] : diags) {
        const int sr = d >= 0 ? 0 : -d, sc = d >= 0 ? d : 0;
        const int len = std::min(D.rows - sr, D.cols - sc);
        D.offsets.push_back(d);
        D.starts.push_back(off);
        D.lengths.push_back(len);
        D.values.resize(static_cast<size_t>(off + len), 0.0f);
        for (const auto& [r, v] : entries) D.values[static_cast<size_t>(off + (r - sr))] = static_cast<float>(v);
        off += len;
    }
    return D;
}

}  // namespace diagpu
