// B-row halves of the merge-path CSR launch: the host side (plan build and
// release, and the per-row carry runs the fix-up kernel walks).  The kernels
// and the launch are in csr_kernels.hip.
//
// No counterpart in the reference: it is a plan-time layout of the
// spmm_tiled_v3 role (spmm_tiled_v3.cu:108-115) that spmm_hybrid_run's CSR
// branch (spmm_hybrid.cu:103-116) uses when B outgrows one XCD's L2.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <vector>

#include "engine.h"
#include "hip_status.h"
#include "spmm/partition.h"

namespace spmm {
namespace engine {

void khalf_runs(const int* row_ptr, int M, long long nnz, const int* split_rows, int parts,
                int* first, int* last) {
    std::fill(first, first + M, -1);
    std::fill(last, last + M, -1);
    for (int g = 0; g < parts; ++g) {
        // The engine's test for a part whose first row began in an earlier
        // part (its piece of that row goes to carry[g]).
        const long long lo = nnz * g / parts;
        const long long hi = nnz * (g + 1) / parts;
        const int r = split_rows[g];
        if (lo < hi && r >= 0 && r < M && row_ptr[r] < lo) {
            if (first[r] < 0) first[r] = g;
            last[r] = g;
        }
    }
}

namespace {

template <typename T>
Error upload(T** dst, const T* src, size_t n, const char* what) {
    SPMM_TRY_HIP(hipMalloc(reinterpret_cast<void**>(dst), sizeof(T) * std::max<size_t>(n, 1)),
                 what);
    if (n > 0) {
        SPMM_TRY_HIP(hipMemcpy(*dst, src, sizeof(T) * n, hipMemcpyHostToDevice), what);
    }
    return Error{};
}

Error build(const CSR& h_A, int N, KHalfPlan* p) {
    const int M = h_A.num_rows;
    const int K = h_A.num_cols;
    if (M < 0 || K < 0 || N < 0 || h_A.nnz < 0) return Error{kInvalid, "negative matrix dimension"};
    if (M > 0 && h_A.row_ptr == nullptr) return Error{kInvalid, "null host pointer"};
    if (h_A.nnz > 0 && (h_A.col_idx == nullptr || h_A.values == nullptr)) {
        return Error{kInvalid, "null host pointer"};
    }
    if (!khalf_pays(K, N)) {
        return Error{kUnsupported,
                     "B-row halves need N % 4 == 0 and K x N x 4 bytes over 4 MiB with half of "
                     "the rows within it (and within the buffer limits)"};
    }
    const int K0 = K / 2;
    // Entries per row and half; columns must lie in [0, K).
    std::vector<int> rp0(static_cast<size_t>(M) + 1, 0), rp1(static_cast<size_t>(M) + 1, 0);
    for (int r = 0; r < M; ++r) {
        int n0 = 0, n1 = 0;
        for (int e = h_A.row_ptr[r]; e < h_A.row_ptr[r + 1]; ++e) {
            const int c = h_A.col_idx[e];
            if (c < 0 || c >= K) return Error{kInvalid, "column index outside [0, num_cols)"};
            (c < K0 ? n0 : n1) += 1;
        }
        rp0[r + 1] = rp0[r] + n0;
        rp1[r + 1] = rp1[r] + n1;
    }
    if (rp0[M] < kKHalfMinNnz || rp1[M] < kKHalfMinNnz) {
        return Error{kUnsupported, "B-row halves need " + std::to_string(kKHalfMinNnz) +
                                       " entries in each half"};
    }
    // Stable split of every row: entry order inside each half is the row's.
    std::vector<int>   c0(rp0[M]), c1(rp1[M]);
    std::vector<float> v0(rp0[M]), v1(rp1[M]);
    for (int r = 0; r < M; ++r) {
        int i0 = rp0[r], i1 = rp1[r];
        for (int e = h_A.row_ptr[r]; e < h_A.row_ptr[r + 1]; ++e) {
            const int c = h_A.col_idx[e];
            if (c < K0) {
                c0[i0] = c;
                v0[i0++] = h_A.values[e];
            } else {
                c1[i1] = c - K0;
                v1[i1++] = h_A.values[e];
            }
        }
    }
    p->M = M;
    p->K = K;
    p->K0 = K0;
    p->N = N;
    std::vector<int> runs(static_cast<size_t>(M) * 4);
    std::vector<int> first(M), last(M);
    const std::vector<int>*   rps[2]  = {&rp0, &rp1};
    const std::vector<int>*   cols[2] = {&c0, &c1};
    const std::vector<float>* vals[2] = {&v0, &v1};
    for (int h = 0; h < 2; ++h) {
        CSR hv;
        hv.num_rows = M;
        hv.num_cols = h == 0 ? K0 : K - K0;
        hv.nnz      = (*rps[h])[M];
        hv.row_ptr  = const_cast<int*>(rps[h]->data());
        hv.col_idx  = const_cast<int*>(cols[h]->data());
        hv.values   = const_cast<float*>(vals[h]->data());
        const int parts = split_partition_parts(hv.nnz);
        const std::vector<int> rows = nnz_split_rows(hv, parts);
        khalf_runs(hv.row_ptr, M, hv.nnz, rows.data(), parts, first.data(), last.data());
        for (int r = 0; r < M; ++r) {
            runs[static_cast<size_t>(r) * 4 + 2 * h]     = first[r];
            runs[static_cast<size_t>(r) * 4 + 2 * h + 1] = last[r];
        }
        CSR& d = p->half[h];
        d.num_rows = M;
        d.num_cols = hv.num_cols;
        d.nnz      = hv.nnz;
        SPMM_TRY(upload(&d.row_ptr, hv.row_ptr, static_cast<size_t>(M) + 1, "hipMalloc"));
        SPMM_TRY(upload(&d.col_idx, hv.col_idx, static_cast<size_t>(hv.nnz), "hipMalloc"));
        SPMM_TRY(upload(&d.values, hv.values, static_cast<size_t>(hv.nnz), "hipMalloc"));
        SPMM_TRY(upload(&p->rows[h], rows.data(), rows.size(), "hipMalloc"));
        p->parts[h] = parts;
        SPMM_TRY_HIP(hipMalloc(&p->carry[h], sizeof(float) * static_cast<size_t>(parts) * N),
                     "hipMalloc");
    }
    SPMM_TRY(upload(&p->runs, runs.data(), runs.size(), "hipMalloc"));
    SPMM_TRY_HIP(hipMalloc(&p->partial, sizeof(float) * std::max<size_t>(
                                            static_cast<size_t>(M) * N, 1)),
                 "hipMalloc");
    return Error{};
}

}  // namespace

void khalf_plan_free(KHalfPlan* p) {
    if (p == nullptr) return;
    for (int h = 0; h < 2; ++h) {
        (void)hipFree(p->half[h].row_ptr);
        (void)hipFree(p->half[h].col_idx);
        (void)hipFree(p->half[h].values);
        (void)hipFree(p->rows[h]);
        (void)hipFree(p->carry[h]);
    }
    (void)hipFree(p->partial);
    (void)hipFree(p->runs);
    *p = KHalfPlan{};
}

Error khalf_plan_build(const CSR& h_A, int N, KHalfPlan* out) {
    if (out == nullptr) return Error{kInvalid, "null plan"};
    *out = KHalfPlan{};
    Error e = build(h_A, N, out);
    if (e.status != kOk) khalf_plan_free(out);
    return e;
}

}  // namespace engine
}  // namespace spmm
