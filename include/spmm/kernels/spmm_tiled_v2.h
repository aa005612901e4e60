#pragma once
// Drop-in for the reference's src/kernels/spmm_tiled_v2.h (spmm_tiled_v2.h:38).
//
// Role: the vectorised-B variant.  Served by the row-block engine with float4
// lanes.  Keeps the reference's contract: N must be a multiple of 128 and B/C
// 16-byte aligned, otherwise the launcher prints a message and calls abort()
// (spmm_tiled_v2.cu:99-105).
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  Null stream, no synchronisation.

#include "../csr.h"

namespace spmm {

void spmm_tiled_v2(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
