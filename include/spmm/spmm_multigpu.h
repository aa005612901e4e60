#pragma once
// Memory strategies of the reference's src/spmm_multigpu.h (:1-58), single-GPU
// subset: gpu_count() and the unified-memory path spmm_unified().
//
// spmm_multigpu (the reference's per-device row split with one host thread per
// GPU) is not part of this single-GPU engine and is not declared here; a
// caller that uses it fails to compile rather than silently running on one
// device.

#include "csr.h"

namespace spmm {

// Number of HIP devices visible to the process (spmm_multigpu.h:32).
int gpu_count();

// Single-GPU SpMM with A, B and C in HIP managed memory (hipMallocManaged),
// prefetched to the current device, multiplied by the tiled_v3 engine
// (spmm_multigpu.h:54-58, spmm_multigpu.cu:122-182).  Returns the median
// per-launch kernel time in ms over `iters` launches after `warmup`; h_C is
// filled on return.  Unlike the reference, the prefetch status is checked:
// a device without managed memory is an error, and a device that does not
// support prefetching is reported once on stderr (its pages then move on
// first touch).  Errors print and exit, like the reference's wrappers.
float spmm_unified(const CSR& h_A, const float* h_B, float* h_C, int N, int warmup, int iters);

}  // namespace spmm
