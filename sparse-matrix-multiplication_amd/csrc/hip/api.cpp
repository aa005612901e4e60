// The reference's kernel entry points (src/kernels/*.h) on top of the launch
// layer.  Conventions kept from the reference launchers: null stream, no
// synchronisation, launch errors print and exit(EXIT_FAILURE)
// (e.g. spmm_tiled_v3.cu:108-115), the tiled_v2 shape contract prints and
// abort()s (spmm_tiled_v2.cu:99-105).

#include <cstdio>
#include <cstdlib>

#include "engine.h"
#include "spmm/kernels/spmm_baseline.h"
#include "spmm/kernels/spmm_memopt.h"
#include "spmm/kernels/spmm_memopt_v2.h"
#include "spmm/kernels/spmm_tiled.h"
#include "spmm/kernels/spmm_tiled_v2.h"
#include "spmm/kernels/spmm_tiled_v3.h"
#include "spmm/kernels/spmm_tiled_v4.h"
#include "spmm/kernels/spmm_wmma.h"

namespace spmm {

namespace {

void exit_on_error(const engine::Error& e, const char* who) {
    if (e.status == engine::kOk) return;
    std::fprintf(stderr, "%s: %s\n", who, e.message.c_str());
    if (e.status == engine::kUnsupported) std::abort();
    std::exit(EXIT_FAILURE);
}

void run_csr(engine::CsrRole role, const CSR& d_A, const float* d_B, float* d_C, int N,
             const char* who) {
    exit_on_error(engine::launch_csr(role, d_A, d_B, d_C, N, nullptr), who);
}

}  // namespace

void spmm_baseline(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::Baseline, d_A, d_B, d_C, N, "spmm_baseline");
}
void spmm_memopt(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::Memopt, d_A, d_B, d_C, N, "spmm_memopt");
}
void spmm_memopt_v2(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::MemoptV2, d_A, d_B, d_C, N, "spmm_memopt_v2");
}
void spmm_tiled(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::Tiled, d_A, d_B, d_C, N, "spmm_tiled");
}
void spmm_tiled_v2(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::TiledV2, d_A, d_B, d_C, N, "spmm_tiled_v2");
}
void spmm_tiled_v3(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::TiledV3, d_A, d_B, d_C, N, "spmm_tiled_v3");
}
void spmm_tiled_v4(const CSR& d_A, const float* d_B, float* d_C, int N) {
    run_csr(engine::CsrRole::TiledV4, d_A, d_B, d_C, N, "spmm_tiled_v4");
}

void float_to_half(const float* d_src, half* d_dst, int n_elements) {
    exit_on_error(engine::launch_float_to_half(d_src, d_dst, n_elements, nullptr),
                  "float_to_half");
}

BSR bsr_from_csr_device(const CSR& d_csr) {
    BSR out;
    exit_on_error(engine::build_bsr_device(d_csr, &out, nullptr), "bsr_from_csr_device");
    return out;
}

BSR_stats bsr_stats_from_csr_device(const CSR& d_csr) {
    BSR_stats out{};
    exit_on_error(engine::bsr_stats_device(d_csr, &out, nullptr), "bsr_stats_from_csr_device");
    return out;
}

void spmm_wmma(const BSR& d_bsr, const half* d_B_fp16, float* d_C, int N) {
    exit_on_error(engine::launch_bsr(d_bsr, d_B_fp16, d_C, N, nullptr), "spmm_wmma");
}

}  // namespace spmm
