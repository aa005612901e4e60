// Allocation-free merge-path launch: spmm_c_tiled_v3_split with its carry
// workspace taken from a file-scope device array instead of the caller.
//
// For callers that cannot call hipMalloc (code under HIP graph capture, tight
// serving loops, harnesses that forbid allocation).  The caller still passes
// the matrix, the split-row table, B and C; the P x N fp32 carries of the
// parts that continue a row live in `scratch`, which each GPU holds from the
// first call on that device until the process ends.
//
// Every carry slot the fix-up kernel reads is written by the engine kernel of
// the same call (a continuation part stores its piece of the row before the
// fix-up adds it), so nothing needs clearing between calls.  All calls on one
// GPU share that GPU's array: calls that overlap on one GPU (concurrent
// streams, or host threads launching together) race on it.

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "engine.h"

namespace spmm {
namespace engine {

namespace {

// Capacity of the carry workspace: parts x N <= kNoAllocScratchFloats (2 MiB;
// e.g. 512 parts up to N = 1024).
constexpr long kNoAllocScratchFloats = 1L << 19;
constexpr int  kMaxDevices           = 64;

__device__ __align__(256) float scratch[kNoAllocScratchFloats];

// Device address of `scratch` per device, looked up once with that device
// current.  In host code `scratch` names a host-side stand-in, never the
// device memory, so only these pointers are handed to kernels.
std::mutex g_scratch_mutex;
float*     g_scratch_ptr[kMaxDevices] = {};

Error scratch_for_current_device(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return Error{kHipError, std::string("hipGetDevice: ") + hipGetErrorString(e)};
    if (dev < 0 || dev >= kMaxDevices) {
        return Error{kUnsupported, "no-alloc launch supports device ids below 64"};
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            return Error{kHipError, std::string("hipGetSymbolAddress(scratch): ") +
                                        (e != hipSuccess ? hipGetErrorString(e) : "null address")};
        }
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return Error{};
}

}  // namespace

long noalloc_scratch_floats() { return kNoAllocScratchFloats; }

Error launch_csr_split_noalloc(const CSR& A, const int* split_rows, int parts, const float* B,
                               float* C, int N, hipStream_t stream) {
    if (parts < 1) return Error{kInvalid, "split partition needs parts >= 1"};
    if (N < 0) return Error{kInvalid, "negative N"};
    if (static_cast<long long>(parts) * N > kNoAllocScratchFloats) {
        return Error{kUnsupported,
                     "no-alloc split launch: parts x N = " +
                         std::to_string(static_cast<long long>(parts) * N) +
                         " exceeds the carry workspace of " + std::to_string(kNoAllocScratchFloats) +
                         " floats (use spmm_c_tiled_v3_split with a workspace)"};
    }
    float* carry = nullptr;
    Error err = scratch_for_current_device(&carry);
    if (err.status != kOk) return err;
    SplitPlan plan;
    plan.rows  = split_rows;
    plan.parts = parts;
    plan.carry = carry;
    return launch_csr_split(A, B, C, N, stream, plan);
}

}  // namespace engine
}  // namespace spmm
