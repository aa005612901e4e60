// Host BSR construction, upload and statistics (reference: src/bsr.cu:30-162).

#include "spmm/bsr.h"

#include <algorithm>
#include <stdexcept>

#include "spmm/utils.h"

namespace spmm {

BSR_host bsr_from_csr_host(const CSR& h) {
    constexpr int BS  = BSR_BLOCK;
    constexpr int BS2 = BSR_BLOCK * BSR_BLOCK;
    BSR_host out;
    out.num_rows   = h.num_rows;
    out.num_cols   = h.num_cols;
    out.block_rows = (h.num_rows + BS - 1) / BS;
    out.block_cols = (h.num_cols + BS - 1) / BS;
    out.nnz        = h.nnz;
    out.row_ptr.assign(static_cast<size_t>(out.block_rows) + 1, 0);
    for (int p = 0; p < h.nnz; ++p) {
        if (h.col_idx[p] < 0 || h.col_idx[p] >= h.num_cols) {
            throw std::runtime_error("bsr_from_csr_host: column index out of range");
        }
    }

    // stamp[bc] == br + 1 marks block-column bc as seen in block-row br;
    // slot[bc] is its position inside the block-row once the row is sorted.
    std::vector<int> stamp(static_cast<size_t>(out.block_cols), 0);
    std::vector<int> slot(static_cast<size_t>(out.block_cols), 0);
    std::vector<int> cols_of_row;

    // Pass 1: distinct block-columns per block-row, ascending.
    for (int br = 0; br < out.block_rows; ++br) {
        cols_of_row.clear();
        const int r_end = std::min(h.num_rows, (br + 1) * BS);
        for (int r = br * BS; r < r_end; ++r) {
            for (int p = h.row_ptr[r]; p < h.row_ptr[r + 1]; ++p) {
                const int bc = h.col_idx[p] / BS;
                if (stamp[bc] != br + 1) {
                    stamp[bc] = br + 1;
                    cols_of_row.push_back(bc);
                }
            }
        }
        std::sort(cols_of_row.begin(), cols_of_row.end());
        out.row_ptr[br + 1] = out.row_ptr[br] + static_cast<int>(cols_of_row.size());
        out.col_idx.insert(out.col_idx.end(), cols_of_row.begin(), cols_of_row.end());
    }
    out.num_blocks = out.row_ptr[out.block_rows];

    // Pass 2: scatter values; a repeated (row, col) overwrites, so the last
    // occurrence in CSR order is the one kept (bsr.cu:87-88).
    const half zero = __float2half(0.0f);
    out.values.assign(static_cast<size_t>(out.num_blocks) * BS2, zero);
    for (int br = 0; br < out.block_rows; ++br) {
        for (int b = out.row_ptr[br]; b < out.row_ptr[br + 1]; ++b) slot[out.col_idx[b]] = b;
        const int r_end = std::min(h.num_rows, (br + 1) * BS);
        for (int r = br * BS; r < r_end; ++r) {
            const int lr = r - br * BS;
            for (int p = h.row_ptr[r]; p < h.row_ptr[r + 1]; ++p) {
                const int c   = h.col_idx[p];
                const int blk = slot[c / BS];
                out.values[static_cast<size_t>(blk) * BS2 + lr * BS + (c % BS)] =
                    __float2half(h.values[p]);
            }
        }
    }
    return out;
}

BSR bsr_to_device(const BSR_host& h) {
    BSR d;
    d.num_rows   = h.num_rows;
    d.num_cols   = h.num_cols;
    d.block_rows = h.block_rows;
    d.block_cols = h.block_cols;
    d.num_blocks = h.num_blocks;
    d.nnz        = h.nnz;
    const size_t rp = sizeof(int) * (static_cast<size_t>(h.block_rows) + 1);
    const size_t ci = sizeof(int) * static_cast<size_t>(h.num_blocks);
    const size_t va = sizeof(half) * static_cast<size_t>(h.num_blocks) * BSR_BLOCK * BSR_BLOCK;
    HIP_CHECK(hipMalloc(&d.row_ptr, rp));
    HIP_CHECK(hipMalloc(&d.col_idx, ci > 0 ? ci : sizeof(int)));
    HIP_CHECK(hipMalloc(&d.values, va > 0 ? va : sizeof(half)));
    HIP_CHECK(hipMemcpy(d.row_ptr, h.row_ptr.data(), rp, hipMemcpyHostToDevice));
    if (ci > 0) HIP_CHECK(hipMemcpy(d.col_idx, h.col_idx.data(), ci, hipMemcpyHostToDevice));
    if (va > 0) HIP_CHECK(hipMemcpy(d.values, h.values.data(), va, hipMemcpyHostToDevice));
    return d;
}

void bsr_free_device(BSR& d) {
    if (d.row_ptr) { HIP_CHECK(hipFree(d.row_ptr)); d.row_ptr = nullptr; }
    if (d.col_idx) { HIP_CHECK(hipFree(d.col_idx)); d.col_idx = nullptr; }
    if (d.values)  { HIP_CHECK(hipFree(d.values));  d.values  = nullptr; }
}

BSR_stats bsr_stats_from_csr_host(const CSR& h) {
    constexpr int BS = BSR_BLOCK;
    const int block_rows = (h.num_rows + BS - 1) / BS;
    const int block_cols = (h.num_cols + BS - 1) / BS;
    std::vector<int> stamp(static_cast<size_t>(block_cols), 0);
    long blocks = 0;
    for (int br = 0; br < block_rows; ++br) {
        const int r_end = std::min(h.num_rows, (br + 1) * BS);
        for (int p = h.row_ptr[br * BS]; p < h.row_ptr[r_end]; ++p) {
            const int c = h.col_idx[p];
            if (c < 0 || c >= h.num_cols) {
                throw std::runtime_error("bsr_stats_from_csr_host: column index out of range");
            }
            if (stamp[c / BS] != br + 1) {
                stamp[c / BS] = br + 1;
                ++blocks;
            }
        }
    }
    BSR_host shape;  // the statistics read only the scalar fields
    shape.num_rows   = h.num_rows;
    shape.num_cols   = h.num_cols;
    shape.block_rows = block_rows;
    shape.block_cols = block_cols;
    shape.num_blocks = static_cast<int>(blocks);
    shape.nnz        = h.nnz;
    return bsr_compute_stats(shape);
}

BSR_stats bsr_compute_stats(const BSR_host& h) {
    BSR_stats s;
    s.num_blocks      = h.num_blocks;
    s.stored_elements = static_cast<long>(h.num_blocks) * BSR_BLOCK * BSR_BLOCK;
    s.original_nnz    = h.nnz;
    s.fill_in_ratio   = h.nnz > 0 ? static_cast<double>(s.stored_elements) / h.nnz : 0.0;
    const long all    = static_cast<long>(h.block_rows) * h.block_cols;
    s.block_density   = all > 0 ? static_cast<double>(h.num_blocks) / all : 0.0;
    return s;
}

}  // namespace spmm
