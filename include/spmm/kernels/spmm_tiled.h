#pragma once
// Drop-in for the reference's src/kernels/spmm_tiled.h (spmm_tiled.h:45).
//
// Role: column-tile streaming.  Served by the row-block engine (the kernel behind
// spmm_tiled_v3) with a 64-column tile: one lane per column per pass.
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  The launch goes to the null stream and
// does not synchronise; a launch failure prints and exits like HIP_CHECK.
// N == 0 or M == 0 launches nothing.

#include "../csr.h"

namespace spmm {

void spmm_tiled(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
