#pragma once
// Compressed-sparse-row matrix and its host-side operations.
//
// Drop-in for the reference's src/csr.h (csr.h:6-41): same namespace, same
// struct field order, same function signatures and the same error conventions
// (std::runtime_error on bad input, exit(EXIT_FAILURE) on host OOM or HIP
// failure).  Device copies live in HBM as three flat arrays:
//   row_ptr int32[num_rows + 1], col_idx int32[nnz], values fp32[nnz].

#include <string>
#include <vector>

namespace spmm {

// Plain-old-data view; whether the pointers are host or device memory is a
// convention of the caller (csr.h:7-14).
struct CSR {
    int    num_rows = 0;
    int    num_cols = 0;
    int    nnz      = 0;
    int*   row_ptr  = nullptr;
    int*   col_idx  = nullptr;
    float* values   = nullptr;
};

// malloc-backed host storage; exits the process when malloc fails (csr.cu:19-32).
CSR  csr_alloc_host(int rows, int cols, int nnz);
// Frees host storage and zeroes every field (csr.cu:34-42).
void csr_free_host(CSR& m);

// COO -> CSR.  Entries are ordered by (row, col) with a stable index sort;
// duplicates are KEPT (they are summed by any SpMM), exactly as csr.cu:44-72
// does despite the comment at csr.h:20.  Throws std::runtime_error when the
// three vectors differ in length.
CSR csr_from_coo_host(int rows, int cols,
                      const std::vector<int>&   row_indices,
                      const std::vector<int>&   col_indices,
                      const std::vector<float>& values);

// Bernoulli(density) per cell in row-major order, drawn from std::mt19937(seed)
// with std::uniform_real_distribution<float>(0,1); each hit then draws its value
// from uniform_real_distribution<float>(-1,1) on the same engine (csr.cu:74-103).
// Throws std::runtime_error when density is outside [0, 1].
CSR generate_uniform_random_csr(int rows, int cols, float density, int seed);

// Rows [row_begin, row_end) as a new host CSR with a rebased row_ptr
// (csr.cu:105-123).  Throws std::runtime_error on an invalid range.
CSR csr_row_slice_host(const CSR& m, int row_begin, int row_end);

// Binary file: int32 rows, int32 cols, int32 nnz, row_ptr, col_idx, fp32 values,
// little-endian (csr.h:32-35, csr.cu:125-150).  Throws std::runtime_error when
// the file cannot be opened or is short.
CSR  csr_read_binary_host(const std::string& path);
void csr_write_binary_host(const CSR& m, const std::string& path);

// hipMalloc + three host-to-device copies / hipFree of the three arrays
// (csr.cu:152-178).
CSR  csr_to_device(const CSR& host);
void csr_free_device(CSR& device);

}  // namespace spmm
