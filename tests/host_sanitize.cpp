// Host layer of the engine (csrc/host/*.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer: every host entry point, including the error
// paths the reference throws on, on small inputs.  Built with g++ (no device
// code) by tests/test_host_sanitize.py; exits non-zero on a failed check, and
// the sanitizers abort on a memory or UB error.

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "spmm/bsr.h"
#include "spmm/csr.h"
#include "spmm/metrics.h"
#include "spmm/partition.h"
#include "spmm/patterns.h"

namespace {

int g_failures = 0;

void check(bool ok, const char* what) {
    if (!ok) {
        std::fprintf(stderr, "FAILED: %s\n", what);
        ++g_failures;
    }
}

template <typename F>
void expect_throw(F fn, const char* what) {
    bool thrown = false;
    try {
        fn();
    } catch (const std::runtime_error&) {
        thrown = true;
    }
    check(thrown, what);
}

bool csr_valid(const spmm::CSR& m) {
    if (m.row_ptr[0] != 0 || m.row_ptr[m.num_rows] != m.nnz) return false;
    for (int r = 0; r < m.num_rows; ++r) {
        if (m.row_ptr[r + 1] < m.row_ptr[r]) return false;
        for (int p = m.row_ptr[r]; p < m.row_ptr[r + 1]; ++p) {
            if (m.col_idx[p] < 0 || m.col_idx[p] >= m.num_cols) return false;
            if (p > m.row_ptr[r] && m.col_idx[p] < m.col_idx[p - 1]) return false;
        }
    }
    return true;
}

void test_csr() {
    // COO -> CSR: unsorted input, duplicates kept, empty rows
    const std::vector<int> r = {3, 0, 3, 1, 3, 0};
    const std::vector<int> c = {2, 4, 2, 0, 1, 4};
    const std::vector<float> v = {1, 2, 3, 4, 5, 6};
    spmm::CSR a = spmm::csr_from_coo_host(5, 6, r, c, v);
    check(a.nnz == 6 && csr_valid(a), "coo->csr sorted and complete");
    check(a.row_ptr[2] - a.row_ptr[1] == 1 && a.row_ptr[3] == a.row_ptr[2], "row lengths");
    expect_throw([] { spmm::csr_from_coo_host(2, 2, {0}, {0, 1}, {1.f}); }, "coo size mismatch");
    expect_throw([] { spmm::csr_from_coo_host(2, 2, {5}, {0}, {1.f}); }, "coo row out of range");

    // row slice and binary round trip
    spmm::CSR s = spmm::csr_row_slice_host(a, 1, 4);
    check(s.num_rows == 3 && s.nnz == a.row_ptr[4] - a.row_ptr[1] && csr_valid(s), "row slice");
    expect_throw([&] { spmm::csr_row_slice_host(a, 3, 1); }, "bad slice range");
    const std::string path = "host_sanitize_tmp.bin";
    spmm::csr_write_binary_host(a, path);
    spmm::CSR b = spmm::csr_read_binary_host(path);
    bool same = b.num_rows == a.num_rows && b.num_cols == a.num_cols && b.nnz == a.nnz;
    for (int i = 0; same && i <= a.num_rows; ++i) same = b.row_ptr[i] == a.row_ptr[i];
    for (int i = 0; same && i < a.nnz; ++i) same = b.col_idx[i] == a.col_idx[i] && b.values[i] == a.values[i];
    check(same, "binary round trip");
    std::remove(path.c_str());
    expect_throw([] { spmm::csr_read_binary_host("does/not/exist.bin"); }, "missing file");
    {
        FILE* f = std::fopen(path.c_str(), "wb");
        const int hdr[3] = {4, 4, 100};  // claims 100 nonzeros, holds none
        std::fwrite(hdr, sizeof(int), 3, f);
        std::fclose(f);
        expect_throw([&] { spmm::csr_read_binary_host(path); }, "short file");
        std::remove(path.c_str());
    }

    // generator: density bounds, structure
    spmm::CSR g = spmm::generate_uniform_random_csr(64, 48, 0.1f, 42);
    check(csr_valid(g) && g.nnz > 0, "uniform generator structure");
    expect_throw([] { spmm::generate_uniform_random_csr(4, 4, 1.5f, 1); }, "density > 1");
    spmm::CSR z = spmm::generate_uniform_random_csr(8, 8, 0.0f, 1);
    check(z.nnz == 0 && csr_valid(z), "density 0");

    spmm::csr_free_host(a);
    spmm::csr_free_host(s);
    spmm::csr_free_host(b);
    spmm::csr_free_host(g);
    spmm::csr_free_host(z);
    check(a.row_ptr == nullptr && a.nnz == 0, "free clears the struct");
}

void test_patterns_and_bsr() {
    // banded: |i - j| <= hb, every in-band entry present
    spmm::CSR bd = spmm::generate_banded_csr(37, 37, 3, 5);
    long want = 0;
    for (int i = 0; i < 37; ++i) want += std::min(36, i + 3) - std::max(0, i - 3) + 1;
    check(csr_valid(bd) && bd.nnz == want, "banded closed form");
    spmm::CSR bl = spmm::generate_block_diagonal_csr(50, 50, 16, 6);
    check(csr_valid(bl) && bl.nnz == 3 * 16 * 16, "block-diagonal: 3 full blocks of 16");
    spmm::CSR pl = spmm::generate_power_law_csr(300, 200, 20.0, 1.5, 150, 7);
    bool capped = csr_valid(pl);
    for (int r = 0; capped && r < pl.num_rows; ++r) {
        const int len = pl.row_ptr[r + 1] - pl.row_ptr[r];
        capped = len >= 1 && len <= 150;
    }
    check(capped, "power-law rows in [1, cap]");

    // BSR build: ragged dims (block rows/cols by ceil-div), stats, dense equality
    spmm::CSR g = spmm::generate_uniform_random_csr(45, 70, 0.08f, 6);
    spmm::csr_round_values_to_fp16(g);
    spmm::BSR_host h = spmm::bsr_from_csr_host(g);
    check(h.block_rows == 3 && h.block_cols == 5, "ceil-div block dims");
    check(static_cast<int>(h.row_ptr.size()) == h.block_rows + 1 &&
              static_cast<int>(h.col_idx.size()) == h.num_blocks &&
              h.values.size() == static_cast<size_t>(h.num_blocks) * 256,
          "BSR array sizes");
    std::vector<float> dense_csr(45 * 70, 0.f), dense_bsr(45 * 70, 0.f);
    for (int r = 0; r < 45; ++r)
        for (int p = g.row_ptr[r]; p < g.row_ptr[r + 1]; ++p) dense_csr[r * 70 + g.col_idx[p]] += g.values[p];
    for (int br = 0; br < h.block_rows; ++br)
        for (int b = h.row_ptr[br]; b < h.row_ptr[br + 1]; ++b)
            for (int e = 0; e < 256; ++e) {
                const int rr = br * 16 + e / 16, cc = h.col_idx[b] * 16 + e % 16;
                const float x = static_cast<float>(h.values[static_cast<size_t>(b) * 256 + e]);
                if (rr < 45 && cc < 70) dense_bsr[rr * 70 + cc] = x;
                else check(x == 0.f, "padding outside the matrix is zero");
            }
    check(dense_csr == dense_bsr, "BSR densifies to the CSR (fp16-exact values)");
    const spmm::BSR_stats st = spmm::bsr_compute_stats(h);
    const spmm::BSR_stats st2 = spmm::bsr_stats_from_csr_host(g);
    check(st.num_blocks == st2.num_blocks && st.fill_in_ratio == st2.fill_in_ratio &&
              st.stored_elements == 256L * h.num_blocks,
          "stats agree (counting pass vs build)");

    // host references: BSR fp32 path vs fp64 CSR path on fp16-exact operands
    const int N = 9;
    std::vector<float> B = spmm::generate_dense_row_major(70, N, 8);
    spmm::dense_round_to_fp16(B.data(), static_cast<long>(B.size()));
    std::vector<float> c64 = spmm::spmm_host_reference_f64(g, B.data(), N, 3);
    std::vector<float> c32 = spmm::spmm_host_reference_bsr_f32(h, B.data(), N, 2);
    check(spmm::rel_l2(c32, c64) < 1e-6f, "BSR fp32 reference vs fp64 CSR reference");
    std::vector<float> c1 = spmm::spmm_host_reference_f64(g, B.data(), N, 1);
    check(c1 == c64, "fp64 reference independent of thread count");

    spmm::csr_free_host(bd);
    spmm::csr_free_host(bl);
    spmm::csr_free_host(pl);
    spmm::csr_free_host(g);
}

void test_partition_and_metrics() {
    spmm::CSR p = spmm::generate_power_law_csr(500, 400, 30.0, 1.5, 400, 9);
    for (int parts : {1, 2, 7, 64, 499, 500, 2000}) {
        const std::vector<int> b = spmm::nnz_balanced_bounds(p, parts);
        bool ok = static_cast<int>(b.size()) == parts + 1 && b.front() == 0 && b.back() == p.num_rows;
        for (int i = 0; ok && i < parts; ++i) ok = b[i] <= b[i + 1];
        check(ok, "nnz-balanced bounds cover the rows, monotone");
        const std::vector<int> sr = spmm::nnz_split_rows(p, parts);
        bool ok2 = static_cast<int>(sr.size()) == parts + 1 && sr.front() == 0 && sr.back() == p.num_rows;
        for (int g = 0; ok2 && g < parts; ++g) {
            const long lo = static_cast<long>(p.nnz) * g / parts;
            ok2 = sr[g] <= sr[g + 1] && (lo >= p.nnz || (p.row_ptr[sr[g]] <= lo && lo < p.row_ptr[sr[g] + 1]) ||
                                         p.row_ptr[sr[g]] == lo);
        }
        check(ok2, "split rows hold each part's first nonzero");
    }
    expect_throw([&] { spmm::nnz_balanced_bounds(p, 0); }, "parts < 1");
    spmm::csr_free_host(p);

    const std::vector<float> ref = {1.f, -2.f, 0.f, 4.f};
    const std::vector<float> ours = {1.f, -2.f, 0.5f, 4.f};
    const spmm::ErrorStats e = spmm::compare(ours, ref);
    check(e.max_abs == 0.5f, "compare max_abs");
    check(std::fabs(e.rel_l2 - 0.5f / std::sqrt(21.f)) < 1e-6f, "compare rel_l2");
    check(spmm::median({3.f, 1.f, 2.f}) == 2.f && spmm::median({}) == 0.f, "median");
}

}  // namespace

int main() {
    test_csr();
    test_patterns_and_bsr();
    test_partition_and_metrics();
    if (g_failures) {
        std::fprintf(stderr, "%d check(s) failed\n", g_failures);
        return 1;
    }
    std::printf("host sanitize: all checks passed\n");
    return 0;
}
