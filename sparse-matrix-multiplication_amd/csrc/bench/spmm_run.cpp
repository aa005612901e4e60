// spmm_run: the integrated driver with the CLI and output of the reference's
// src/bench/spmm_run.cu (Args :27-41, parse_args :62-97, main :169-238):
// ingest A, choose a back end with hybrid_choose, run it with spmm_hybrid_run,
// verify, print the plan= and run= lines.
//
// Differences: verification uses the host fp64 loop instead of cuSPARSE (the
// [PASS] rule, rel_l2 < 1e-2, is unchanged); --multi-gpu is not part of this
// single-GPU engine and is rejected; --pattern selects the structured inputs
// of the BASELINE configs.

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "common.h"
#include "spmm/csr.h"
#include "spmm/metrics.h"
#include "spmm/patterns.h"
#include "spmm/spmm_hybrid.h"
#include "spmm/spmm_multigpu.h"

namespace {

struct Args {
    drv::MatrixArgs mat;
    int   n = 256;
    int   warmup = 3;
    int   iters = 10;
    float threshold = spmm::kHybridAutoThreshold;  // per-N MI355X crossover
    bool  verify = true;
    bool  unified = false;
    int   cpu_threads = 0;
};

void print_usage(const char* prog) {
    std::fprintf(stderr,
                 "Usage: %s [options]\n"
                 "  --m INT          rows of A and C            (default 4096)\n"
                 "  --k INT          cols of A / rows of B      (default 4096)\n"
                 "  --n INT          cols of B and C            (default 256)\n"
                 "  --density FLOAT  fraction of nonzeros       (default 0.01)\n"
                 "  --seed INT       RNG seed                   (default 42)\n"
                 "  --warmup INT     warmup iterations          (default 3)\n"
                 "  --iters INT      timed iterations           (default 10)\n"
                 "  --threshold FLT  BSR fill-in cut-off for the MFMA path (default: the MI355X\n"
                 "                   crossover for N, 8 at N <= 16 .. %.0f at N >= 256)\n"
                 "  --bin PATH       load CSR from a binary file (overrides --m/--k/--density)\n"
                 "  --no-verify      skip the host fp64 correctness check\n"
                 "  --unified        single-GPU unified-memory path (CSR engine)\n"
                 "  --cpu-threads INT host threads of the verification loop (default: all)\n"
                 "%s",
                 prog, static_cast<double>(spmm::kHybridDefaultThreshold), drv::matrix_usage());
}

Args parse_args(int argc, char** argv) {
    Args a;
    a.mat.m = 4096;
    a.mat.k = 4096;
    for (int i = 1; i < argc; ++i) {
        const std::string opt = argv[i];
        auto need = [&]() -> std::string {
            if (i + 1 >= argc) {
                std::fprintf(stderr, "missing value for %s\n", opt.c_str());
                print_usage(argv[0]);
                std::exit(EXIT_FAILURE);
            }
            return std::string(argv[++i]);
        };
        if (opt == "--m") a.mat.m = std::stoi(need());
        else if (opt == "--k") a.mat.k = std::stoi(need());
        else if (opt == "--n") a.n = std::stoi(need());
        else if (opt == "--density") a.mat.density = std::stof(need());
        else if (opt == "--seed") a.mat.seed = std::stoi(need());
        else if (opt == "--warmup") a.warmup = std::stoi(need());
        else if (opt == "--iters") a.iters = std::stoi(need());
        else if (opt == "--threshold") a.threshold = std::stof(need());
        else if (opt == "--bin") a.mat.bin_path = need();
        else if (opt == "--no-verify") a.verify = false;
        else if (opt == "--cpu-threads") a.cpu_threads = std::stoi(need());
        else if (opt == "--unified") a.unified = true;
        else if (opt == "--multi-gpu" || opt == "--gpus") {
            std::fprintf(stderr, "%s is not part of this single-GPU engine\n", opt.c_str());
            std::exit(EXIT_FAILURE);
        } else if (opt == "-h" || opt == "--help") {
            print_usage(argv[0]);
            std::exit(0);
        } else if (drv::parse_matrix_opt(a.mat, opt, i, argc, argv)) {
        } else {
            std::fprintf(stderr, "unknown option: %s\n", opt.c_str());
            print_usage(argv[0]);
            std::exit(EXIT_FAILURE);
        }
    }
    return a;
}

}  // namespace

int main(int argc, char** argv) {
    Args args = parse_args(argc, argv);
    spmm::CSR h_A = drv::build_matrix(args.mat);
    const int M = args.mat.m, K = args.mat.k, N = args.n;
    const float density = (M > 0 && K > 0)
                              ? static_cast<float>(h_A.nnz) / (static_cast<float>(M) * K)
                              : 0.f;
    std::vector<float> h_B = spmm::generate_dense_row_major(K, N, args.mat.seed + 1);
    if (args.mat.fp16_values) spmm::dense_round_to_fp16(h_B.data(), static_cast<long>(h_B.size()));
    std::vector<float> h_C(static_cast<size_t>(M) * N, 0.f);

    const spmm::HybridPlan plan = spmm::hybrid_choose(h_A, N, args.threshold);
    float ms = 0.f;
    std::string mode;
    if (args.unified) {
        ms   = spmm::spmm_unified(h_A, h_B.data(), h_C.data(), N, args.warmup, args.iters);
        mode = "unified[csr]";
    } else {
        ms   = spmm::spmm_hybrid_run(plan, h_A, h_B.data(), h_C.data(), N, args.warmup,
                                     args.iters);
        mode = std::string("hybrid[") + spmm::backend_name(plan.backend) + "]";
    }
    const double flops = 2.0 * static_cast<double>(h_A.nnz) * N;
    const double gflops = flops / (static_cast<double>(ms) * 1.0e6);

    std::printf("plan backend=%s fill_in=%.2f block_density=%.4f threshold=%.2f n_aligned=%d "
                "reason=\"%s\"\n",
                spmm::backend_name(plan.backend), plan.fill_in_ratio, plan.block_density,
                plan.threshold, plan.n_aligned ? 1 : 0, plan.reason);

    float l2 = -1.f;
    double cpu_ms = 0.0;
    int cpu_threads = 0;
    if (args.verify) {
        const drv::CpuLeg cpu = drv::run_cpu_reference(h_A, h_B.data(), N, args.cpu_threads, 1);
        l2 = spmm::rel_l2(h_C, cpu.C);
        cpu_ms = cpu.ms;
        cpu_threads = cpu.threads;
    }
    std::printf("run mode=%s m=%d k=%d n=%d nnz=%d density=%.6f time_ms=%.4f gflops=%.2f "
                "rel_l2_err=%.3e %s",
                mode.c_str(), M, K, N, h_A.nnz, density, ms, gflops, l2,
                args.verify ? (l2 < 1e-2f ? "[PASS]" : "[FAIL]") : "[unverified]");
    if (args.verify) std::printf(" cpu_ms=%.3f cpu_threads=%d", cpu_ms, cpu_threads);
    std::printf("\n");
    spmm::csr_free_host(h_A);
    return 0;
}
