#pragma once
// Shared pieces of the two drivers: matrix ingestion (synthetic pattern or the
// binary CSR file), the CPU verification leg and byte models.

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <thread>
#include <vector>

#include "spmm/csr.h"
#include "spmm/metrics.h"
#include "spmm/patterns.h"

namespace drv {

struct MatrixArgs {
    int         m = 0, k = 0;
    float       density = 0.01f;
    int         seed = 42;
    std::string pattern = "uniform";  // uniform | banded | block-diagonal | power-law
    int         bandwidth = 64;       // banded half-bandwidth
    int         block = 256;          // block-diagonal block size
    double      mean_deg = 164.0;     // power-law
    double      alpha = 1.5;          // power-law
    int         cap = 4096;           // power-law max row nnz
    bool        fp16_values = false;  // round A and B through fp16
    std::string bin_path;
};

// Returns true when opt was consumed (i advanced past its value).
inline bool parse_matrix_opt(MatrixArgs& a, const std::string& opt, int& i, int argc,
                             char** argv) {
    auto need = [&]() -> std::string {
        if (i + 1 >= argc) {
            std::fprintf(stderr, "missing value for %s\n", opt.c_str());
            std::exit(EXIT_FAILURE);
        }
        return std::string(argv[++i]);
    };
    if (opt == "--pattern") a.pattern = need();
    else if (opt == "--bandwidth") a.bandwidth = std::stoi(need());
    else if (opt == "--block") a.block = std::stoi(need());
    else if (opt == "--mean-deg") a.mean_deg = std::stod(need());
    else if (opt == "--alpha") a.alpha = std::stod(need());
    else if (opt == "--cap") a.cap = std::stoi(need());
    else if (opt == "--fp16-values") a.fp16_values = true;
    else return false;
    return true;
}

inline const char* matrix_usage() {
    return "  --pattern STR    uniform | banded | block-diagonal | power-law (default uniform)\n"
           "  --bandwidth INT  banded half-bandwidth            (default 64)\n"
           "  --block INT      block-diagonal block size        (default 256)\n"
           "  --mean-deg FLT   power-law mean row length        (default 164)\n"
           "  --alpha FLT      power-law Pareto exponent        (default 1.5)\n"
           "  --cap INT        power-law max row length         (default 4096)\n"
           "  --fp16-values    round A and B through fp16 (the fp16 configs)\n";
}

inline spmm::CSR build_matrix(MatrixArgs& a) {
    spmm::CSR h;
    if (!a.bin_path.empty()) {
        h = spmm::csr_read_binary_host(a.bin_path);
    } else if (a.pattern == "uniform") {
        h = spmm::generate_uniform_random_csr(a.m, a.k, a.density, a.seed);
    } else if (a.pattern == "banded") {
        h = spmm::generate_banded_csr(a.m, a.k, a.bandwidth, a.seed);
    } else if (a.pattern == "block-diagonal") {
        h = spmm::generate_block_diagonal_csr(a.m, a.k, a.block, a.seed);
    } else if (a.pattern == "power-law") {
        h = spmm::generate_power_law_csr(a.m, a.k, a.mean_deg, a.alpha, a.cap, a.seed);
    } else {
        std::fprintf(stderr, "unknown pattern: %s\n", a.pattern.c_str());
        std::exit(EXIT_FAILURE);
    }
    a.m = h.num_rows;
    a.k = h.num_cols;
    if (a.fp16_values) spmm::csr_round_values_to_fp16(h);
    return h;
}

inline int hardware_threads() {
    const unsigned hc = std::thread::hardware_concurrency();
    return hc > 0 ? static_cast<int>(hc) : 1;
}

// Median wall time (ms) of `reps` runs of the fp64 host loop.
struct CpuLeg {
    std::vector<float> C;
    double             ms = 0.0;
    int                threads = 1;
};

inline CpuLeg run_cpu_reference(const spmm::CSR& h, const float* B, int N, int threads,
                                int reps) {
    CpuLeg leg;
    leg.threads = threads > 0 ? threads : hardware_threads();
    std::vector<float> times;
    for (int r = 0; r < (reps > 0 ? reps : 1); ++r) {
        const auto t0 = std::chrono::steady_clock::now();
        leg.C = spmm::spmm_host_reference_f64(h, B, N, leg.threads);
        const auto t1 = std::chrono::steady_clock::now();
        times.push_back(std::chrono::duration<float, std::milli>(t1 - t0).count());
    }
    leg.ms = spmm::median(times);
    return leg;
}

// Compulsory bytes of one CSR SpMM (scripts/roofline.py:177-185).
inline double csr_bytes(long m, long k, long n, long nnz) {
    return 8.0 * nnz + 4.0 * (m + 1) + 4.0 * k * n + 4.0 * m * n;
}

// Compulsory bytes of one BSR SpMM with fp16 B and fp32 C.
inline double bsr_bytes(long m, long k, long n, long blocks) {
    return 516.0 * blocks + 4.0 * ((m + 15) / 16 + 1) + 2.0 * k * n + 4.0 * m * n;
}

constexpr double kHbmPeakGBs   = 8000.0;    // MI355X HBM3E
constexpr double kMfmaF16Peak  = 2516.6e3;  // GFLOP/s, dense fp16 MFMA

}  // namespace drv
