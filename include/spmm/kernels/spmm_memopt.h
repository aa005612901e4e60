#pragma once
// Drop-in for the reference's src/kernels/spmm_memopt.h (spmm_memopt.h:18).
//
// Role: wave-per-row without staging.  One wave64 per row; lane l owns columns
// l, l+64, ...; the row's (col, value) pairs are read with wave-uniform scalar loads.
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  The launch goes to the null stream and
// does not synchronise; a launch failure prints and exits like HIP_CHECK.
// N == 0 or M == 0 launches nothing.

#include "../csr.h"

namespace spmm {

void spmm_memopt(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
