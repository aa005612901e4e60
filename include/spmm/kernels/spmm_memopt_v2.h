#pragma once
// Drop-in for the reference's src/kernels/spmm_memopt_v2.h (spmm_memopt_v2.h:26).
//
// Role: the register-capped variant of spmm_memopt.  Same wave-per-row kernel,
// compiled with a tighter launch bound (8 waves per SIMD).
//
// d_A is a device CSR; d_B (K x N) and d_C (M x N) are row-major fp32 device
// buffers with leading dimension N.  The launch goes to the null stream and
// does not synchronise; a launch failure prints and exits like HIP_CHECK.
// N == 0 or M == 0 launches nothing.

#include "../csr.h"

namespace spmm {

void spmm_memopt_v2(const CSR& d_A, const float* d_B, float* d_C, int N);

}  // namespace spmm
