// Synthetic inputs (structure: scripts/gen_matrices.py:30-81; dense B:
// harness.cu:114-120).

#include "spmm/patterns.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <random>
#include <stdexcept>

#include <hip/hip_fp16.h>

namespace spmm {

namespace {

// Builds a host CSR from per-row column lists that are already ascending.
CSR csr_from_rows(int rows, int cols, const std::vector<int>& row_ptr,
                  const std::vector<int>& col_idx, const std::vector<float>& vals) {
    CSR m = csr_alloc_host(rows, cols, static_cast<int>(col_idx.size()));
    std::copy(row_ptr.begin(), row_ptr.end(), m.row_ptr);
    std::copy(col_idx.begin(), col_idx.end(), m.col_idx);
    std::copy(vals.begin(), vals.end(), m.values);
    return m;
}

void check_dims(int rows, int cols, const char* who) {
    if (rows < 0 || cols < 0) throw std::runtime_error(std::string(who) + ": negative dimension");
}

}  // namespace

std::vector<float> generate_dense_row_major(int rows, int cols, int seed) {
    check_dims(rows, cols, "generate_dense_row_major");
    std::mt19937 rng(static_cast<uint32_t>(seed));
    std::uniform_real_distribution<float> uni(-1.f, 1.f);
    std::vector<float> v(static_cast<size_t>(rows) * cols);
    for (float& x : v) x = uni(rng);
    return v;
}

CSR generate_banded_csr(int rows, int cols, int half_bandwidth, int seed) {
    check_dims(rows, cols, "generate_banded_csr");
    if (half_bandwidth < 0) throw std::runtime_error("generate_banded_csr: negative bandwidth");
    std::mt19937 rng(static_cast<uint32_t>(seed));
    std::uniform_real_distribution<float> uni(-1.f, 1.f);
    std::vector<int> rp(static_cast<size_t>(rows) + 1, 0);
    std::vector<int> ci;
    std::vector<float> va;
    for (int r = 0; r < rows; ++r) {
        const long lo = std::max<long>(0, static_cast<long>(r) - half_bandwidth);
        const long hi = std::min<long>(cols, static_cast<long>(r) + half_bandwidth + 1);
        for (long c = lo; c < hi; ++c) {
            ci.push_back(static_cast<int>(c));
            va.push_back(uni(rng));
        }
        rp[static_cast<size_t>(r) + 1] = static_cast<int>(ci.size());
    }
    return csr_from_rows(rows, cols, rp, ci, va);
}

CSR generate_block_diagonal_csr(int rows, int cols, int block, int seed, float value_scale) {
    check_dims(rows, cols, "generate_block_diagonal_csr");
    if (block < 1) throw std::runtime_error("generate_block_diagonal_csr: block must be >= 1");
    std::mt19937 rng(static_cast<uint32_t>(seed));
    std::uniform_real_distribution<double> canon(0.0, 1.0);
    const double two_pi = 6.283185307179586476925286766559;
    const int nblk = std::min(rows, cols) / block;
    std::vector<int> rp(static_cast<size_t>(rows) + 1, 0);
    std::vector<int> ci;
    std::vector<float> va;
    for (int r = 0; r < rows; ++r) {
        const int b = r / block;
        if (b < nblk) {
            for (int c = b * block; c < (b + 1) * block; ++c) {
                const double u1 = 1.0 - canon(rng);  // (0, 1]
                const double u2 = canon(rng);
                const double z  = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
                ci.push_back(c);
                va.push_back(static_cast<float>(z * value_scale));
            }
        }
        rp[static_cast<size_t>(r) + 1] = static_cast<int>(ci.size());
    }
    return csr_from_rows(rows, cols, rp, ci, va);
}

CSR generate_block_diagonal_uniform_csr(int rows, int cols, int block, int seed) {
    check_dims(rows, cols, "generate_block_diagonal_uniform_csr");
    if (block < 1) throw std::runtime_error("generate_block_diagonal_uniform_csr: block must be >= 1");
    std::mt19937 rng(static_cast<uint32_t>(seed));
    std::uniform_real_distribution<float> uni(-1.f, 1.f);
    const int nblk = std::min(rows, cols) / block;
    std::vector<int> rp(static_cast<size_t>(rows) + 1, 0);
    std::vector<int> ci;
    std::vector<float> va;
    for (int r = 0; r < rows; ++r) {
        const int b = r / block;
        if (b < nblk) {
            for (int c = b * block; c < (b + 1) * block; ++c) {
                ci.push_back(c);
                va.push_back(uni(rng));
            }
        }
        rp[static_cast<size_t>(r) + 1] = static_cast<int>(ci.size());
    }
    return csr_from_rows(rows, cols, rp, ci, va);
}

CSR generate_power_law_csr(int rows, int cols, double mean_deg, double alpha,
                           int max_row_nnz, int seed) {
    check_dims(rows, cols, "generate_power_law_csr");
    if (!(alpha > 0.0) || !(mean_deg > 0.0)) {
        throw std::runtime_error("generate_power_law_csr: alpha and mean_deg must be positive");
    }
    std::mt19937 rng(static_cast<uint32_t>(seed));
    std::uniform_real_distribution<double> canon(0.0, 1.0);
    std::uniform_real_distribution<float> uni(-1.f, 1.f);

    // Degrees for every row first (gen_matrices.py:68-71).
    std::vector<double> raw(static_cast<size_t>(rows));
    double sum = 0.0;
    for (double& x : raw) {
        x = std::pow(1.0 - canon(rng), -1.0 / alpha);
        sum += x;
    }
    const int cap = std::max(1, std::min(cols, max_row_nnz));
    const double scale = rows > 0 ? mean_deg / (sum / rows) : 0.0;
    std::vector<int> rp(static_cast<size_t>(rows) + 1, 0);
    for (int r = 0; r < rows; ++r) {
        double d = std::nearbyint(raw[r] * scale);  // round half to even
        d = std::min<double>(std::max<double>(d, 1.0), cap);
        rp[static_cast<size_t>(r) + 1] = rp[r] + (cols > 0 ? static_cast<int>(d) : 0);
    }

    // Columns: Floyd's sampling of d distinct values in [0, cols), then sorted.
    std::vector<int> ci(static_cast<size_t>(rp[rows]));
    std::vector<uint8_t> taken(static_cast<size_t>(cols), 0);
    for (int r = 0; r < rows; ++r) {
        const int d = rp[r + 1] - rp[r];
        int* out = ci.data() + rp[r];
        int n = 0;
        for (int j = cols - d; j < cols; ++j) {
            std::uniform_int_distribution<int> pick(0, j);
            const int t = pick(rng);
            const int v = taken[t] ? j : t;
            taken[v] = 1;
            out[n++] = v;
        }
        std::sort(out, out + d);
        for (int i = 0; i < d; ++i) taken[out[i]] = 0;
    }
    std::vector<float> va(ci.size());
    for (float& x : va) x = uni(rng);
    return csr_from_rows(rows, cols, rp, ci, va);
}

void dense_round_to_fp16(float* v, long n) {
    for (long i = 0; i < n; ++i) v[i] = __half2float(__float2half(v[i]));
}

void csr_round_values_to_fp16(CSR& h) { dense_round_to_fp16(h.values, h.nnz); }

}  // namespace spmm
