#pragma once
// Drop-in for the reference's src/kernels/spmm_tiled_v3.h (spmm_tiled_v3.h:40).
//
// The production CSR kernel (the engine).  Workgroups own nnz-balanced row
// blocks; the block's nonzeros are split evenly over its waves (rows that cross a
// wave boundary are summed in LDS in wave order); each wave streams 64-entry
// (col, value) chunks through VGPRs and issues vector B-row loads (float4 /
// float2 / float per lane, chosen from N and alignment) several rows ahead.
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  The launch goes to the null stream and
// does not synchronise; a launch failure prints and exits like HIP_CHECK.
// N == 0 or M == 0 launches nothing.

#include "../csr.h"

namespace spmm {

void spmm_tiled_v3(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
