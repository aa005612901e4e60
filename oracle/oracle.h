/*
 * CPU ORACLE FOR THE SpMM HOT PATH -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of what the reference computes on this path, written
 * to check the engine (libspmm_amd.so).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only as the checker or as
 * the timed CPU baseline.  No engine entry point calls into it.
 *
 * Each function cites the reference file:line it restates.  The reference has
 * no CPU SpMM (it checks against cuSPARSE, harness.cu:123-171); the SpMM loops
 * below are the host loops its north star asks for: fp64 accumulation for CSR,
 * fp32 accumulation of fp16-rounded operands for BSR.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   mt19937 / canonical float  numpy's MT19937 (legacy seeding) raw stream, the
 *                              C++ standard's 10000th-output value, and the
 *                              reference's committed nnz counts
 *   uniform generator          nnz known answers from reports/data/sweep.csv and
 *                              scripts/roofline.py EMBEDDED (12 cells)
 *   coo_to_csr                 numpy lexsort on random triplets with duplicates
 *   csr_spmm_f64               scipy.sparse CSR @ dense in float64, identity,
 *                              empty rows, single entries, brute force
 *   csr_spmm_f32_fma           an fp64 restatement of each fused step on random
 *                              inputs, exact integer cases, and a case where the
 *                              fused and the unfused chain round differently
 *   f32_to_f16 / f16_to_f32    numpy float16 conversion (RNE) over edge cases
 *   bsr_build / bsr_stats      brute-force densification, known block counts and
 *                              fill-in from reports/tensor_core_wmma.md:43-56,
 *                              closed forms (banded, block-diagonal)
 *   bsr_spmm_f32               numpy float64 product of the fp16-rounded dense
 *                              operands (error bound), and exact small cases
 *   hybrid_rule                closed-form table of spmm_hybrid.cu:35-54
 *   nnz_balanced_bounds        brute-force definition and invariants
 *   compare / rel_l2 / median  hand-computed vectors
 */
#ifndef SPMM_ORACLE_H
#define SPMM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- RNG: std::mt19937 and libstdc++ uniform_real_distribution<float> ---- */
typedef struct oracle_mt19937 {
    uint32_t state[624];
    int      index;
} oracle_mt19937;

/* csr.cu:79 (std::mt19937 rng(seed)) */
void     oracle_mt_seed(oracle_mt19937* g, uint32_t seed);
uint32_t oracle_mt_next(oracle_mt19937* g);
void     oracle_mt_raw(uint32_t seed, uint32_t* out, long n);
/* generate_canonical<float, 24> over one 32-bit draw, then a + u * (b - a)
 * (csr.cu:80-81 uni/vals, harness.cu:116) */
float    oracle_canonical_f32(uint32_t draw);
float    oracle_uniform_f32(oracle_mt19937* g, float a, float b);

/* ---- generators ------------------------------------------------------ */
/* csr.cu:74-103.  Writes row_ptr[rows+1], col_idx / values up to capacity;
 * returns nnz, or -1 when nnz exceeds capacity (arrays may be NULL with
 * capacity 0 to count only). */
long oracle_generate_uniform_csr(int rows, int cols, float density, int seed,
                                 int* row_ptr, int* col_idx, float* values,
                                 long capacity);
/* harness.cu:114-120 */
void oracle_generate_dense(int rows, int cols, int seed, float* out);

/* csr.cu:44-72: stable order by (row, col), duplicates kept.  Returns 0, or -1
 * on a row index outside [0, rows). */
int oracle_coo_to_csr(int rows, long n, const int* r, const int* c, const float* v,
                      int* row_ptr, int* col_idx, float* values);

/* ---- CSR SpMM, fp64 accumulation (north star host loop) ---------------
 * C[r][j] = sum_p (double)values[p] * (double)B[col_idx[p]][j] in CSR order.
 * abs_c (nullable) receives sum_p |values[p]| * |B[col_idx[p]][j]|, the scale
 * of the fp32 rounding error of any summation order.  Rows are split over
 * `threads` pthreads by oracle_nnz_balanced_bounds. */
void oracle_csr_spmm_f64(int M, int N, const int* row_ptr, const int* col_idx,
                         const float* values, const float* B, double* C, double* abs_c,
                         int threads);

/* ---- CSR SpMM, fp32 fused chain (spmm_baseline.cu:11-25) --------------
 * C[r][j] = fmaf(values[p], B[col_idx[p]][j], ...) from 0.f in CSR order: the
 * reference's baseline kernel bit for bit (nvcc contracts its a*b + sum). */
void oracle_csr_spmm_f32_fma(int M, int N, const int* row_ptr, const int* col_idx,
                             const float* values, const float* B, float* C);

/* ---- fp16 ------------------------------------------------------------ */
/* __float2half round-to-nearest-even (bsr.cu:94-96, spmm_wmma.cu:22) */
uint16_t oracle_f32_to_f16(float x);
float    oracle_f16_to_f32(uint16_t h);
void     oracle_f32_to_f16_array(const float* in, uint16_t* out, long n);

/* ---- BSR 16x16 (bsr.cu:30-109, :149-162) -----------------------------
 * Pass 1: block_row_ptr[M/16 + 1] (ceil) from sorted unique block-columns;
 * returns the number of blocks.  Pass 2 (oracle_bsr_fill): block_col_idx and
 * row-major fp16 block values; a repeated (row, col) keeps the last one in
 * CSR order.  Returns 0, or -1 on a column outside [0, K). */
long oracle_bsr_count(int M, int K, const int* row_ptr, const int* col_idx,
                      int* block_row_ptr);
int  oracle_bsr_fill(int M, int K, const int* row_ptr, const int* col_idx,
                     const float* values, const int* block_row_ptr, int* block_col_idx,
                     uint16_t* block_values);
void oracle_bsr_stats(int M, int K, long num_blocks, long nnz, double* fill_in_ratio,
                      double* block_density, long* stored_elements);

/* BSR SpMM: C = A_bsr * B16, fp32 accumulation, block order then k order.
 * B16 holds fp16 bits (K x N row-major). */
void oracle_bsr_spmm_f32(int M, int K, int N, const int* block_row_ptr,
                         const int* block_col_idx, const uint16_t* block_values,
                         const uint16_t* B16, float* C, int threads);

/* ---- dispatch, partition, metrics ------------------------------------ */
/* spmm_hybrid.cu:35-54.  Returns 1 for the matrix-core path, 0 for CSR;
 * reason_id: 0 "low fill-in", 1 "N not aligned", 2 "high fill-in". */
int  oracle_hybrid_rule(double fill_in_ratio, int N, float threshold, int* reason_id);
/* spmm_multigpu.cu:26-40 */
void oracle_nnz_balanced_bounds(int M, const int* row_ptr, int parts, int* bounds);
/* harness.cu:179-196 */
void oracle_compare(const float* ours, const float* ref, long n, float* max_abs,
                    float* max_rel, float* rel_l2);
/* spmm_run.cu:157-165 */
float oracle_rel_l2(const float* ours, const float* ref, long n);
/* harness.cu:198-201: sorts v in place, returns v[n/2] */
float oracle_median(float* v, int n);

#ifdef __cplusplus
}
#endif

#endif /* SPMM_ORACLE_H */
