#pragma once
// Block-sparse-row matrix with fixed 16x16 fp16 blocks.
//
// Drop-in for the reference's src/bsr.h (bsr.h:19-80).  A 16x16 block is the
// K-extent of one half of a gfx950 v_mfma_f32_16x16x32_f16 A operand, so two
// blocks of one block-row feed one MFMA.  Block b occupies
// values[b*256 .. b*256+255], row-major inside the block (element (lr, lc) at
// b*256 + lr*16 + lc); missing entries are zero.

#include <hip/hip_fp16.h>

#include <vector>

#include "csr.h"

namespace spmm {

constexpr int BSR_BLOCK = 16;  // bsr.h:22

// Host BSR; owns its storage (bsr.h:25-42).
struct BSR_host {
    int num_rows   = 0;  // M
    int num_cols   = 0;  // K
    int block_rows = 0;  // ceil(M / 16)
    int block_cols = 0;  // ceil(K / 16)
    int num_blocks = 0;  // non-empty blocks
    int nnz        = 0;  // nonzeros of the source CSR (before padding)

    std::vector<int>  row_ptr;  // block_rows + 1
    std::vector<int>  col_idx;  // num_blocks, ascending inside each block-row
    std::vector<half> values;   // num_blocks * 256
};

// Device BSR; raw HBM pointers (bsr.h:45-56).
struct BSR {
    int num_rows   = 0;
    int num_cols   = 0;
    int block_rows = 0;
    int block_cols = 0;
    int num_blocks = 0;
    int nnz        = 0;

    int*  row_ptr = nullptr;
    int*  col_idx = nullptr;
    half* values  = nullptr;
};

// Fill-in statistics (bsr.h:59-65).
struct BSR_stats {
    int    num_blocks;
    long   stored_elements;  // num_blocks * 256
    int    original_nnz;
    double fill_in_ratio;    // stored_elements / original_nnz (0 when nnz == 0)
    double block_density;    // num_blocks / (block_rows * block_cols)
};

// CSR -> BSR on the host (bsr.cu:30-109).  When a (row, col) cell occurs more
// than once in the CSR the last occurrence in CSR order is the one stored, as
// in the reference's scatter.  Values are rounded fp32 -> fp16 to nearest-even.
BSR_host bsr_from_csr_host(const CSR& h_csr);

// hipMalloc + upload (bsr.cu:115-137).
BSR  bsr_to_device(const BSR_host& h);

// hipFree of the three arrays.  Like bsr.cu:139-143 the dimension fields are
// left as they were.
void bsr_free_device(BSR& d);

// bsr.cu:149-162.
BSR_stats bsr_compute_stats(const BSR_host& h);

// Additions (no counterpart in the reference, whose BSR build is host-only):

// bsr_compute_stats(bsr_from_csr_host(h_csr)) from one counting pass over the
// CSR, without building the fp16 blocks.
BSR_stats bsr_stats_from_csr_host(const CSR& h_csr);

// CSR -> BSR on the device from a device CSR: the same row_ptr, col_idx and
// fp16 values as bsr_from_csr_host, built next to the kernels (allocates the
// three arrays; release with bsr_free_device).  Column indices must ascend
// within each row (repeats allowed, adjacent; the last is kept) and
// num_cols <= 4128768.  Errors print and exit, like the reference's wrappers.
BSR bsr_from_csr_device(const CSR& d_csr);

// Fill-in statistics of a device CSR, same contract as bsr_from_csr_device.
BSR_stats bsr_stats_from_csr_device(const CSR& d_csr);

}  // namespace spmm
