// Error statistics (harness.cu:173-201, spmm_run.cu:157-165) and the host
// verification loops used by the drivers.

#include "spmm/metrics.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <thread>

#include "spmm/partition.h"

namespace spmm {

ErrorStats compare(const std::vector<float>& ours, const std::vector<float>& ref) {
    if (ours.size() != ref.size()) throw std::runtime_error("compare: size mismatch");
    ErrorStats s;
    float peak = 0.f;
    for (float v : ref) peak = std::max(peak, std::fabs(v));
    const float floor_rel = 1e-3f * peak;
    double err2 = 0.0, ref2 = 0.0;
    for (size_t i = 0; i < ours.size(); ++i) {
        const float d = std::fabs(ours[i] - ref[i]);
        const float a = std::fabs(ref[i]);
        s.max_abs = std::max(s.max_abs, d);
        if (a > floor_rel) s.max_rel = std::max(s.max_rel, d / a);
        err2 += static_cast<double>(d) * d;
        ref2 += static_cast<double>(a) * a;
    }
    s.rel_l2 = ref2 > 0.0 ? static_cast<float>(std::sqrt(err2 / ref2)) : 0.f;
    return s;
}

float median(std::vector<float> v) {
    if (v.empty()) return 0.f;
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

float rel_l2(const std::vector<float>& ours, const std::vector<float>& ref) {
    if (ours.size() != ref.size()) throw std::runtime_error("rel_l2: size mismatch");
    double err2 = 0.0, ref2 = 0.0;
    for (size_t i = 0; i < ours.size(); ++i) {
        const double d = static_cast<double>(ours[i]) - ref[i];
        err2 += d * d;
        ref2 += static_cast<double>(ref[i]) * ref[i];
    }
    return ref2 > 0.0 ? static_cast<float>(std::sqrt(err2 / ref2)) : 0.f;
}

namespace {

int resolve_threads(int threads) {
    if (threads > 0) return threads;
    const unsigned hc = std::thread::hardware_concurrency();
    return hc > 0 ? static_cast<int>(hc) : 1;
}

template <typename Body>
void run_row_parts(const std::vector<int>& bounds, Body body) {
    const int parts = static_cast<int>(bounds.size()) - 1;
    if (parts == 1) {
        body(bounds[0], bounds[1]);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(parts);
    for (int t = 0; t < parts; ++t) pool.emplace_back(body, bounds[t], bounds[t + 1]);
    for (auto& th : pool) th.join();
}

}  // namespace

std::vector<float> spmm_host_reference_f64(const CSR& A, const float* B, int N, int threads) {
    std::vector<float> C(static_cast<size_t>(A.num_rows) * N, 0.f);
    if (N <= 0 || A.num_rows == 0) return C;
    const std::vector<int> bounds = nnz_balanced_bounds(A, resolve_threads(threads));
    run_row_parts(bounds, [&](int r0, int r1) {
        std::vector<double> acc(static_cast<size_t>(N));
        for (int r = r0; r < r1; ++r) {
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int p = A.row_ptr[r]; p < A.row_ptr[r + 1]; ++p) {
                const double v = A.values[p];
                const float* brow = B + static_cast<size_t>(A.col_idx[p]) * N;
                for (int j = 0; j < N; ++j) acc[j] += v * static_cast<double>(brow[j]);
            }
            float* crow = C.data() + static_cast<size_t>(r) * N;
            for (int j = 0; j < N; ++j) crow[j] = static_cast<float>(acc[j]);
        }
    });
    return C;
}

std::vector<float> spmm_host_reference_bsr_f32(const BSR_host& A, const float* B, int N,
                                               int threads) {
    std::vector<float> C(static_cast<size_t>(A.num_rows) * N, 0.f);
    if (N <= 0 || A.num_rows == 0) return C;
    constexpr int BS = BSR_BLOCK;
    const int nthreads = std::max(1, std::min(resolve_threads(threads), A.block_rows));
    std::vector<int> bounds(static_cast<size_t>(nthreads) + 1);
    for (int t = 0; t <= nthreads; ++t) {
        bounds[t] = static_cast<int>(static_cast<long long>(A.block_rows) * t / nthreads);
    }
    run_row_parts(bounds, [&](int br0, int br1) {
        std::vector<float> acc(static_cast<size_t>(BS) * N);
        for (int br = br0; br < br1; ++br) {
            std::fill(acc.begin(), acc.end(), 0.f);
            for (int b = A.row_ptr[br]; b < A.row_ptr[br + 1]; ++b) {
                const int k0 = A.col_idx[b] * BS;
                const half* blk = A.values.data() + static_cast<size_t>(b) * BS * BS;
                for (int lr = 0; lr < BS; ++lr) {
                    float* arow = acc.data() + static_cast<size_t>(lr) * N;
                    for (int lk = 0; lk < BS && k0 + lk < A.num_cols; ++lk) {
                        const float a = __half2float(blk[lr * BS + lk]);
                        const float* brow = B + static_cast<size_t>(k0 + lk) * N;
                        for (int j = 0; j < N; ++j) {
                            arow[j] += a * __half2float(__float2half(brow[j]));
                        }
                    }
                }
            }
            for (int lr = 0; lr < BS && br * BS + lr < A.num_rows; ++lr) {
                std::copy(acc.begin() + static_cast<size_t>(lr) * N,
                          acc.begin() + static_cast<size_t>(lr + 1) * N,
                          C.begin() + static_cast<size_t>(br * BS + lr) * N);
            }
        }
    });
    return C;
}

}  // namespace spmm
