#pragma once
// Drop-in for the reference's src/kernels/spmm_baseline.h (spmm_baseline.h:17).
//
// Role: the naive kernel.  One lane per output element C(i, j); a wave covers
// 64 consecutive columns of one row and every lane re-walks the row's CSR entries.
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  The launch goes to the null stream and
// does not synchronise; a launch failure prints and exits like HIP_CHECK.
// N == 0 or M == 0 launches nothing.

#include "../csr.h"

namespace spmm {

void spmm_baseline(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
