// spmm_bench: per-kernel benchmark and correctness harness with the CLI and
// output line of the reference's src/bench/harness.cu (Args :41-52,
// parse_args :82-112, the kernel= line :458-464).
//
// Differences from the reference, all additive:
//   * the correctness reference is the host fp64 loop (spmm_host_reference_f64),
//     not cuSPARSE, and its time is printed as cpu_ms= with cpu_threads=;
//   * time_ms= is the median over --iters batches of --batch back-to-back
//     launches divided by the batch size; single_ms= keeps the reference's
//     one-event-pair-per-launch median;
//   * hbm_gbs= / pct_hbm= price the compulsory bytes (roofline.py:177-185)
//     against MI355X's 8 TB/s, and the MFMA path adds pct_mfma=;
//   * cold_ms= is the median of single launches each preceded by a 512 MiB
//     write that evicts L2 (4 MiB per XCD) and the 256 MiB MALL;
//   * cpu_1t_ms= is one run of the same host loop on one thread;
//   * --pattern selects the structured inputs of the BASELINE configs.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../hip/engine.h"
#include "common.h"
#include "spmm/bsr.h"
#include "spmm/csr.h"
#include "spmm/partition.h"
#include "spmm/kernels/spmm_baseline.h"
#include "spmm/kernels/spmm_memopt.h"
#include "spmm/kernels/spmm_memopt_v2.h"
#include "spmm/kernels/spmm_tiled.h"
#include "spmm/kernels/spmm_tiled_v2.h"
#include "spmm/kernels/spmm_tiled_v3.h"
#include "spmm/kernels/spmm_tiled_v4.h"
#include "spmm/kernels/spmm_wmma.h"
#include "spmm/metrics.h"
#include "spmm/patterns.h"
#include "spmm/spmm_hybrid.h"
#include "spmm/spmm_multigpu.h"
#include "spmm/utils.h"

namespace {

struct Args {
    drv::MatrixArgs mat;
    int         n = 256;
    int         warmup = 3;
    int         iters = 10;
    int         batch = 50;
    int         cpu_threads = 0;  // 0: all hardware threads
    int         cpu_reps = 3;
    bool        cpu_1t = true;
    bool        cold = true;
    std::string kernel = "both";
};

void print_usage(const char* prog) {
    std::fprintf(stderr,
                 "Usage: %s [options]\n"
                 "  --m INT          rows of A and C        (default 1024)\n"
                 "  --k INT          cols of A / rows of B  (default 1024)\n"
                 "  --n INT          cols of B and C        (default 256)\n"
                 "  --density FLOAT  fraction of nonzeros   (default 0.01)\n"
                 "  --seed INT       RNG seed               (default 42)\n"
                 "  --warmup INT     warmup iterations      (default 3)\n"
                 "  --iters INT      timed iterations       (default 10)\n"
                 "  --batch INT      launches per timed batch (default 50)\n"
                 "  --bin PATH       load CSR from binary file (overrides --m/--k/--density)\n"
                 "  --kernel STR     baseline | memopt | memopt_v2 | tiled | tiled_v2 | tiled_v3\n"
                 "                   | tiled_v4 | csr_auto | split | khalf | wmma | hybrid | unified\n"
                 "                   | both | all\n"
                 "                   both = baseline + memopt (default); all = every kernel;\n"
                 "                   csr_auto = the CSR form the hybrid picks, timed in batches;\n"
                 "                   split / khalf = the merge-path form / over B-row halves\n"
                 "                   whatever the hybrid would pick\n"
                 "  --cpu-threads INT host threads of the fp64 reference (default: all)\n"
                 "  --cpu-reps INT   timed repetitions of the fp64 reference (default 3)\n"
                 "  --no-cpu-1t      skip the one-thread run of the fp64 reference\n"
                 "  --no-cold        skip the cold-cache (L2 and MALL flushed) timing\n"
                 "%s",
                 prog, drv::matrix_usage());
}

Args parse_args(int argc, char** argv) {
    Args a;
    a.mat.m = 1024;
    a.mat.k = 1024;
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
        else if (opt == "--batch") a.batch = std::max(1, std::stoi(need()));
        else if (opt == "--bin") a.mat.bin_path = need();
        else if (opt == "--kernel") a.kernel = need();
        else if (opt == "--cpu-threads") a.cpu_threads = std::stoi(need());
        else if (opt == "--cpu-reps") a.cpu_reps = std::stoi(need());
        else if (opt == "--no-cpu-1t") a.cpu_1t = false;
        else if (opt == "--no-cold") a.cold = false;
        else if (opt == "-h" || opt == "--help") { print_usage(argv[0]); std::exit(0); }
        else if (drv::parse_matrix_opt(a.mat, opt, i, argc, argv)) {}
        else {
            std::fprintf(stderr, "unknown option: %s\n", opt.c_str());
            print_usage(argv[0]);
            std::exit(EXIT_FAILURE);
        }
    }
    if (a.iters < 1) a.iters = 1;
    return a;
}

struct Result {
    std::string name;
    float time_ms = 0.f, single_ms = 0.f, cold_ms = 0.f, gflops = 0.f;
    spmm::ErrorStats err;
    double bytes = 0.0;
    double mfma_flops = 0.0;  // executed matrix-core FLOPs (0 for CSR kernels)
};

// Scratch written before each cold launch: larger than L2 (8 x 4 MiB) plus
// the 256 MiB MALL, so the launch finds none of its inputs on chip.
constexpr size_t kFlushBytes = size_t(512) << 20;

template <typename Launch>
float time_cold(Launch launch, const Args& a, void* d_flush) {
    GpuTimer t;
    std::vector<float> cold;
    for (int i = 0; i < a.iters; ++i) {
        HIP_CHECK(hipMemsetAsync(d_flush, i & 0xff, kFlushBytes, nullptr));
        t.start();
        launch();
        t.stop();
        cold.push_back(t.elapsed_ms());
    }
    return spmm::median(cold);
}

template <typename Launch>
void time_launches(Launch launch, const Args& a, float* batch_ms, float* single_ms) {
    for (int i = 0; i < a.warmup; ++i) launch();
    HIP_CHECK(hipDeviceSynchronize());
    GpuTimer t;
    std::vector<float> per_launch, batched;
    for (int i = 0; i < a.iters; ++i) {
        t.start();
        launch();
        t.stop();
        per_launch.push_back(t.elapsed_ms());
    }
    for (int i = 0; i < a.iters; ++i) {
        t.start();
        for (int r = 0; r < a.batch; ++r) launch();
        t.stop();
        batched.push_back(t.elapsed_ms() / a.batch);
    }
    *single_ms = spmm::median(per_launch);
    *batch_ms  = spmm::median(batched);
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

    // CPU reference (also the reported CPU baseline)
    const drv::CpuLeg cpu = drv::run_cpu_reference(h_A, h_B.data(), N, args.cpu_threads,
                                                   args.cpu_reps);
    const double cpu_1t_ms =
        args.cpu_1t ? drv::run_cpu_reference(h_A, h_B.data(), N, 1, 1).ms : -1.0;
    void* d_flush = nullptr;
    if (args.cold) HIP_CHECK(hipMalloc(&d_flush, kFlushBytes));
    auto cold = [&](auto launch) { return args.cold ? time_cold(launch, args, d_flush) : -1.f; };

    spmm::CSR d_A = spmm::csr_to_device(h_A);
    float *d_B = nullptr, *d_C = nullptr;
    const size_t b_bytes = sizeof(float) * static_cast<size_t>(K) * N;
    const size_t c_bytes = sizeof(float) * static_cast<size_t>(M) * N;
    HIP_CHECK(hipMalloc(&d_B, b_bytes > 0 ? b_bytes : 4));
    HIP_CHECK(hipMalloc(&d_C, c_bytes > 0 ? c_bytes : 4));
    if (b_bytes > 0) HIP_CHECK(hipMemcpy(d_B, h_B.data(), b_bytes, hipMemcpyHostToDevice));

    auto fetch_compare = [&](Result& r) {
        std::vector<float> h_C(static_cast<size_t>(M) * N);
        if (c_bytes > 0) HIP_CHECK(hipMemcpy(h_C.data(), d_C, c_bytes, hipMemcpyDeviceToHost));
        r.err = spmm::compare(h_C, cpu.C);
    };
    const double flops = 2.0 * static_cast<double>(h_A.nnz) * N;
    auto finish = [&](Result& r) {
        r.gflops = static_cast<float>(flops / (static_cast<double>(r.time_ms) * 1.0e6));
    };

    std::vector<Result> results;
    struct Named { const char* name; void (*fn)(const spmm::CSR&, const float*, float*, int); };
    const Named csr_kernels[] = {
        {"baseline", spmm::spmm_baseline}, {"memopt", spmm::spmm_memopt},
        {"memopt_v2", spmm::spmm_memopt_v2}, {"tiled", spmm::spmm_tiled},
        {"tiled_v2", spmm::spmm_tiled_v2}, {"tiled_v3", spmm::spmm_tiled_v3},
        {"tiled_v4", spmm::spmm_tiled_v4}};
    const std::string& ks = args.kernel;
    for (const Named& k : csr_kernels) {
        const std::string name = k.name;
        const bool in_both = name == "baseline" || name == "memopt";
        if (!(ks == name || ks == "all" || (ks == "both" && in_both))) continue;
        if (name == "tiled_v2" && N % 128 != 0) {
            if (ks == "tiled_v2") {
                std::fprintf(stderr, "tiled_v2 requires --n divisible by 128 (got n=%d). Skipping.\n", N);
            }
            continue;
        }
        Result r;
        r.name = name;
        time_launches([&] { k.fn(d_A, d_B, d_C, N); }, args, &r.time_ms, &r.single_ms);
        r.cold_ms = cold([&] { k.fn(d_A, d_B, d_C, N); });
        fetch_compare(r);
        finish(r);
        r.bytes = drv::csr_bytes(M, K, N, h_A.nnz);
        results.push_back(r);
    }

    if (ks == "csr_auto" || ks == "split" || ks == "khalf" || ks == "all") {
        // The CSR form spmm_hybrid_run's CSR branch picks from the row lengths
        // (row groups, the engine with the longest row as hint, the
        // merge-path partition, or merge-path over B-row halves), timed like
        // the kernels above.
        namespace eng = spmm::engine;
        eng::CsrChoice ch = eng::choose_csr_form(h_A, N);
        if (ks == "split") {
            if (h_A.nnz < 1) {
                std::fprintf(stderr, "split: the matrix has no nonzeros\n");
                std::exit(EXIT_FAILURE);
            }
            ch.form  = eng::CsrForm::Split;
            ch.parts = eng::split_partition_parts(h_A.nnz);
        } else if (ks == "khalf") {
            ch.form = eng::CsrForm::KHalf;
        }
        int* d_rows = nullptr;
        float* d_carry = nullptr;
        eng::SplitPlan plan;
        eng::KHalfPlan khalf;
        if (ch.form == eng::CsrForm::KHalf) {
            const eng::Error e = eng::khalf_plan_build(h_A, N, &khalf);
            if (e.status != eng::kOk) {
                std::fprintf(stderr, "B-row halves plan failed: %s\n", e.message.c_str());
                std::exit(EXIT_FAILURE);
            }
        }
        if (ch.form == eng::CsrForm::Split) {
            const std::vector<int> rows = spmm::nnz_split_rows(h_A, ch.parts);
            HIP_CHECK(hipMalloc(&d_rows, sizeof(int) * rows.size()));
            HIP_CHECK(hipMemcpy(d_rows, rows.data(), sizeof(int) * rows.size(),
                                hipMemcpyHostToDevice));
            HIP_CHECK(hipMalloc(&d_carry, sizeof(float) * static_cast<size_t>(ch.parts) * N));
            plan.rows  = d_rows;
            plan.parts = ch.parts;
            plan.carry = d_carry;
        }
        auto launch = [&] {
            const eng::Error e =
                ch.form == eng::CsrForm::KHalf ? eng::launch_csr_khalf(khalf, d_B, d_C, nullptr)
                : ch.form == eng::CsrForm::Split
                    ? eng::launch_csr_split(d_A, d_B, d_C, N, nullptr, plan)
                    : eng::launch_csr(eng::CsrRole::TiledV3, d_A, d_B, d_C, N, nullptr, nullptr,
                                      0, &ch.opts);
            if (e.status != eng::kOk) {
                std::fprintf(stderr, "csr_auto launch failed: %s\n", e.message.c_str());
                std::exit(EXIT_FAILURE);
            }
        };
        Result r;
        r.name = ks == "split" || ks == "khalf"
                     ? ks
                     : std::string("csr_auto[") + eng::csr_form_name(ch.form) + "]";
        time_launches(launch, args, &r.time_ms, &r.single_ms);
        r.cold_ms = cold(launch);
        fetch_compare(r);
        finish(r);
        r.bytes = drv::csr_bytes(M, K, N, h_A.nnz);
        results.push_back(r);
        if (d_rows != nullptr) HIP_CHECK(hipFree(d_rows));
        if (d_carry != nullptr) HIP_CHECK(hipFree(d_carry));
        eng::khalf_plan_free(&khalf);
    }

    if (ks == "wmma" || ks == "all") {
        const spmm::BSR_host h_bsr = spmm::bsr_from_csr_host(h_A);
        const spmm::BSR_stats st = spmm::bsr_compute_stats(h_bsr);
        std::printf("bsr_stats blocks=%d stored_elems=%ld original_nnz=%d "
                    "fill_in_ratio=%.2f block_density=%.4f\n",
                    st.num_blocks, st.stored_elements, st.original_nnz, st.fill_in_ratio,
                    st.block_density);
        spmm::BSR d_bsr = spmm::bsr_to_device(h_bsr);
        half* d_B16 = nullptr;
        HIP_CHECK(hipMalloc(&d_B16, sizeof(half) * (static_cast<size_t>(K) * N + 1)));
        spmm::float_to_half(d_B, d_B16, K * N);
        HIP_CHECK(hipDeviceSynchronize());
        Result r;
        r.name = "wmma";
        time_launches([&] { spmm::spmm_wmma(d_bsr, d_B16, d_C, N); }, args, &r.time_ms,
                      &r.single_ms);
        r.cold_ms = cold([&] { spmm::spmm_wmma(d_bsr, d_B16, d_C, N); });
        fetch_compare(r);
        finish(r);
        r.bytes = drv::bsr_bytes(M, K, N, h_bsr.num_blocks);
        r.mfma_flops = 2.0 * 256.0 * h_bsr.num_blocks * N;
        results.push_back(r);
        HIP_CHECK(hipFree(d_B16));
        spmm::bsr_free_device(d_bsr);
    }

    if (ks == "hybrid" || ks == "all") {
        const spmm::HybridPlan plan = spmm::hybrid_choose(h_A, N);
        std::printf("hybrid_plan backend=%s fill_in=%.2f block_density=%.4f threshold=%.2f "
                    "n_aligned=%d reason=\"%s\"\n",
                    spmm::backend_name(plan.backend), plan.fill_in_ratio, plan.block_density,
                    plan.threshold, plan.n_aligned ? 1 : 0, plan.reason);
        std::vector<float> h_C(static_cast<size_t>(M) * N);
        Result r;
        r.name = std::string("hybrid[") + spmm::backend_name(plan.backend) + "]";
        r.time_ms = spmm::spmm_hybrid_run(plan, h_A, h_B.data(), h_C.data(), N, args.warmup,
                                          args.iters);
        r.single_ms = r.time_ms;
        r.cold_ms = -1.f;  // host-in/host-out call: not timed cold
        r.err = spmm::compare(h_C, cpu.C);
        finish(r);
        r.bytes = drv::csr_bytes(M, K, N, h_A.nnz);
        results.push_back(r);
    }

    if (ks == "unified") {
        std::vector<float> h_C(static_cast<size_t>(M) * N);
        Result r;
        r.name = "unified";
        r.time_ms = spmm::spmm_unified(h_A, h_B.data(), h_C.data(), N, args.warmup, args.iters);
        r.single_ms = r.time_ms;
        r.cold_ms = -1.f;  // host-in/host-out call: not timed cold
        r.err = spmm::compare(h_C, cpu.C);
        finish(r);
        r.bytes = drv::csr_bytes(M, K, N, h_A.nnz);
        results.push_back(r);
    }

    if (ks == "multigpu") {
        std::fprintf(stderr, "kernel 'multigpu' is not part of this single-GPU engine. "
                             "Skipping.\n");
    }

    for (const Result& r : results) {
        const double gbs = r.bytes / (static_cast<double>(r.time_ms) * 1.0e6);
        std::printf("kernel=%s m=%d k=%d n=%d nnz=%d density=%.6f time_ms=%.4f gflops=%.2f "
                    "max_abs_err=%.3e max_rel_err=%.3e rel_l2_err=%.3e single_ms=%.4f "
                    "hbm_gbs=%.1f pct_hbm=%.2f",
                    r.name.c_str(), M, K, N, h_A.nnz, density, r.time_ms, r.gflops,
                    r.err.max_abs, r.err.max_rel, r.err.rel_l2, r.single_ms, gbs,
                    100.0 * gbs / drv::kHbmPeakGBs);
        if (r.cold_ms > 0) std::printf(" cold_ms=%.4f", r.cold_ms);
        if (r.mfma_flops > 0) {
            const double mf = r.mfma_flops / (static_cast<double>(r.time_ms) * 1.0e6);
            std::printf(" pct_mfma=%.2f", 100.0 * mf / drv::kMfmaF16Peak);
        }
        std::printf(" cpu_ms=%.3f cpu_threads=%d cpu_gflops=%.2f", cpu.ms, cpu.threads,
                    flops / (cpu.ms * 1.0e6));
        if (cpu_1t_ms > 0) std::printf(" cpu_1t_ms=%.3f", cpu_1t_ms);
        std::printf("\n");
    }

    if (d_flush != nullptr) HIP_CHECK(hipFree(d_flush));
    HIP_CHECK(hipFree(d_B));
    HIP_CHECK(hipFree(d_C));
    spmm::csr_free_device(d_A);
    spmm::csr_free_host(h_A);
    return 0;
}
