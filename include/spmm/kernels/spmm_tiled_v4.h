#pragma once
// Drop-in for the reference's src/kernels/spmm_tiled_v4.h (spmm_tiled_v4.h:79).
//
// Role: the 256-column register tile.  Served by the row-block engine with
// float4 lanes (256 columns per pass) whenever N and the pointers allow it.
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  The launch goes to the null stream and
// does not synchronise; a launch failure prints and exits like HIP_CHECK.
// N == 0 or M == 0 launches nothing.

#include "../csr.h"

namespace spmm {

void spmm_tiled_v4(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
