#pragma once
// Drop-in for the reference's src/kernels/spmm_wmma.h (spmm_wmma.h:32,39).
//
// BSR x dense on gfx950 matrix cores: v_mfma_f32_16x16x32_f16, fp16 inputs,
// fp32 accumulation and fp32 C.  Two 16x16 blocks of one block-row make the
// 32-deep K of one MFMA; the matching 32 rows of B are staged through LDS in a
// K-contiguous layout so each lane's B operand is one 16-byte LDS read.
//
// Unlike the reference kernel, B rows at or beyond K are never read (the
// reference has no K bound on its B fragment, spmm_wmma.cu:81-85) and any
// N >= 1 is accepted; callers that follow the reference still pass N % 16 == 0.

#include <hip/hip_fp16.h>

#include "../bsr.h"

namespace spmm {

// fp32 -> fp16, round to nearest even, elementwise over n_elements.
void float_to_half(const float* d_src, half* d_dst, int n_elements);

//   d_bsr    : device BSR of A (fp16 blocks)
//   d_B_fp16 : K x N fp16, row-major
//   d_C      : M x N fp32, row-major (fully overwritten)
void spmm_wmma(const BSR& d_bsr, const half* d_B_fp16, float* d_C, int N);

}  // namespace spmm
