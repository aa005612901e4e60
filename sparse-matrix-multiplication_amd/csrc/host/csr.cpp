// Host CSR operations (reference behaviour: src/csr.cu:19-178).

#include "spmm/csr.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <numeric>
#include <random>
#include <stdexcept>

#include "spmm/utils.h"

namespace spmm {

namespace {

template <typename T>
T* host_array(size_t count) {
    // malloc(0) may return nullptr legitimately; ask for at least one element
    // so a null pointer always means out of memory.
    void* p = std::malloc(sizeof(T) * (count > 0 ? count : 1));
    if (!p) {
        std::fprintf(stderr, "csr_alloc_host: out of memory\n");
        std::exit(EXIT_FAILURE);
    }
    return static_cast<T*>(p);
}

}  // namespace

CSR csr_alloc_host(int rows, int cols, int nnz) {
    CSR m;
    m.num_rows = rows;
    m.num_cols = cols;
    m.nnz      = nnz;
    m.row_ptr  = host_array<int>(static_cast<size_t>(rows) + 1);
    m.col_idx  = host_array<int>(static_cast<size_t>(nnz));
    m.values   = host_array<float>(static_cast<size_t>(nnz));
    return m;
}

void csr_free_host(CSR& m) {
    std::free(m.row_ptr);
    std::free(m.col_idx);
    std::free(m.values);
    m = CSR{};
}

CSR csr_from_coo_host(int rows, int cols, const std::vector<int>& row_indices,
                      const std::vector<int>& col_indices,
                      const std::vector<float>& values) {
    const size_t n = values.size();
    if (row_indices.size() != n || col_indices.size() != n) {
        throw std::runtime_error("csr_from_coo_host: triplet size mismatch");
    }
    for (size_t i = 0; i < n; ++i) {
        if (row_indices[i] < 0 || row_indices[i] >= rows) {
            throw std::runtime_error("csr_from_coo_host: row index out of range");
        }
    }

    // Order by (row, col).  The reference uses an unstable std::sort, which
    // leaves the relative order of duplicate (row, col) entries unspecified;
    // a stable sort is one valid realisation of it and is deterministic.
    // Generators emit row-major triplets, so skip the sort when already ordered.
    auto less = [&](size_t a, size_t b) {
        if (row_indices[a] != row_indices[b]) return row_indices[a] < row_indices[b];
        return col_indices[a] < col_indices[b];
    };
    std::vector<size_t> order(n);
    std::iota(order.begin(), order.end(), size_t{0});
    bool sorted = true;
    for (size_t i = 1; i < n && sorted; ++i) sorted = !less(i, i - 1);
    if (!sorted) std::stable_sort(order.begin(), order.end(), less);

    CSR m = csr_alloc_host(rows, cols, static_cast<int>(n));
    std::fill(m.row_ptr, m.row_ptr + rows + 1, 0);
    for (size_t i = 0; i < n; ++i) {
        const size_t src = order[i];
        m.col_idx[i] = col_indices[src];
        m.values[i]  = values[src];
        m.row_ptr[row_indices[src] + 1] += 1;
    }
    for (int r = 0; r < rows; ++r) m.row_ptr[r + 1] += m.row_ptr[r];
    return m;
}

CSR generate_uniform_random_csr(int rows, int cols, float density, int seed) {
    if (!(density >= 0.f && density <= 1.f)) {
        throw std::runtime_error("generate_uniform_random_csr: invalid density");
    }
    std::mt19937 rng(static_cast<uint32_t>(seed));
    std::uniform_real_distribution<float> uni(0.f, 1.f);
    std::uniform_real_distribution<float> vals(-1.f, 1.f);

    // Cells are visited row-major, so hits arrive already in (row, col) order
    // and go straight into CSR arrays; the draw sequence is the reference's
    // (one uni() per cell, one vals() per hit, csr.cu:93-101).
    std::vector<int> row_ptr(static_cast<size_t>(rows) + 1, 0);
    std::vector<int> cs;
    std::vector<float> vs;
    const double expect = static_cast<double>(rows) * cols * density;
    cs.reserve(static_cast<size_t>(expect * 1.05 + 64));
    vs.reserve(cs.capacity());
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) {
            if (uni(rng) < density) {
                cs.push_back(c);
                vs.push_back(vals(rng));
            }
        }
        row_ptr[static_cast<size_t>(r) + 1] = static_cast<int>(cs.size());
    }
    CSR m = csr_alloc_host(rows, cols, static_cast<int>(cs.size()));
    std::copy(row_ptr.begin(), row_ptr.end(), m.row_ptr);
    std::copy(cs.begin(), cs.end(), m.col_idx);
    std::copy(vs.begin(), vs.end(), m.values);
    return m;
}

CSR csr_row_slice_host(const CSR& m, int row_begin, int row_end) {
    if (row_begin < 0 || row_end > m.num_rows || row_begin > row_end) {
        throw std::runtime_error("csr_row_slice_host: invalid row range");
    }
    const int first = m.row_ptr[row_begin];
    const int count = m.row_ptr[row_end] - first;
    CSR s = csr_alloc_host(row_end - row_begin, m.num_cols, count);
    for (int r = row_begin; r <= row_end; ++r) s.row_ptr[r - row_begin] = m.row_ptr[r] - first;
    std::copy(m.col_idx + first, m.col_idx + first + count, s.col_idx);
    std::copy(m.values + first, m.values + first + count, s.values);
    return s;
}

CSR csr_read_binary_host(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("csr_read_binary_host: cannot open " + path);
    int32_t hdr[3];
    in.read(reinterpret_cast<char*>(hdr), sizeof(hdr));
    if (!in) throw std::runtime_error("csr_read_binary_host: short read on header");
    if (hdr[0] < 0 || hdr[1] < 0 || hdr[2] < 0) {
        throw std::runtime_error("csr_read_binary_host: negative dimension in header");
    }
    CSR m = csr_alloc_host(hdr[0], hdr[1], hdr[2]);
    in.read(reinterpret_cast<char*>(m.row_ptr), sizeof(int) * (static_cast<size_t>(m.num_rows) + 1));
    in.read(reinterpret_cast<char*>(m.col_idx), sizeof(int) * static_cast<size_t>(m.nnz));
    in.read(reinterpret_cast<char*>(m.values), sizeof(float) * static_cast<size_t>(m.nnz));
    if (!in) {
        csr_free_host(m);
        throw std::runtime_error("csr_read_binary_host: short read on body");
    }
    return m;
}

void csr_write_binary_host(const CSR& m, const std::string& path) {
    std::ofstream out(path, std::ios::binary);
    if (!out) throw std::runtime_error("csr_write_binary_host: cannot open " + path);
    const int32_t hdr[3] = {m.num_rows, m.num_cols, m.nnz};
    out.write(reinterpret_cast<const char*>(hdr), sizeof(hdr));
    out.write(reinterpret_cast<const char*>(m.row_ptr), sizeof(int) * (static_cast<size_t>(m.num_rows) + 1));
    out.write(reinterpret_cast<const char*>(m.col_idx), sizeof(int) * static_cast<size_t>(m.nnz));
    out.write(reinterpret_cast<const char*>(m.values), sizeof(float) * static_cast<size_t>(m.nnz));
}

CSR csr_to_device(const CSR& host) {
    CSR d;
    d.num_rows = host.num_rows;
    d.num_cols = host.num_cols;
    d.nnz      = host.nnz;
    const size_t rp = sizeof(int) * (static_cast<size_t>(host.num_rows) + 1);
    const size_t ci = sizeof(int) * static_cast<size_t>(host.nnz);
    const size_t va = sizeof(float) * static_cast<size_t>(host.nnz);
    HIP_CHECK(hipMalloc(&d.row_ptr, rp));
    HIP_CHECK(hipMalloc(&d.col_idx, ci > 0 ? ci : sizeof(int)));
    HIP_CHECK(hipMalloc(&d.values, va > 0 ? va : sizeof(float)));
    HIP_CHECK(hipMemcpy(d.row_ptr, host.row_ptr, rp, hipMemcpyHostToDevice));
    if (ci > 0) HIP_CHECK(hipMemcpy(d.col_idx, host.col_idx, ci, hipMemcpyHostToDevice));
    if (va > 0) HIP_CHECK(hipMemcpy(d.values, host.values, va, hipMemcpyHostToDevice));
    return d;
}

void csr_free_device(CSR& d) {
    if (d.row_ptr) HIP_CHECK(hipFree(d.row_ptr));
    if (d.col_idx) HIP_CHECK(hipFree(d.col_idx));
    if (d.values) HIP_CHECK(hipFree(d.values));
    d = CSR{};
}

}  // namespace spmm
