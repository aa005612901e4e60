/*
 * CPU ORACLE -- TEST INFRASTRUCTURE (see oracle.h for scope and pins).
 * Plain C11 + pthreads; built by oracle/Makefile into oracle/build/liboracle.so.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * mt19937 (Matsumoto & Nishimura 1998; the engine behind std::mt19937,
 * csr.cu:79, harness.cu:115)
 * ==================================================================== */
void oracle_mt_seed(oracle_mt19937* g, uint32_t seed) {
    g->state[0] = seed;
    for (int i = 1; i < 624; ++i) {
        const uint32_t prev = g->state[i - 1];
        g->state[i] = 1812433253u * (prev ^ (prev >> 30)) + (uint32_t)i;
    }
    g->index = 624;
}

static void mt_twist(oracle_mt19937* g) {
    for (int i = 0; i < 624; ++i) {
        const uint32_t y = (g->state[i] & 0x80000000u) | (g->state[(i + 1) % 624] & 0x7fffffffu);
        uint32_t next = g->state[(i + 397) % 624] ^ (y >> 1);
        if (y & 1u) next ^= 0x9908b0dfu;
        g->state[i] = next;
    }
    g->index = 0;
}

uint32_t oracle_mt_next(oracle_mt19937* g) {
    if (g->index >= 624) mt_twist(g);
    uint32_t y = g->state[g->index++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

void oracle_mt_raw(uint32_t seed, uint32_t* out, long n) {
    oracle_mt19937 g;
    oracle_mt_seed(&g, seed);
    for (long i = 0; i < n; ++i) out[i] = oracle_mt_next(&g);
}

/* libstdc++ generate_canonical<float, 24>: the engine range is 2^32 >= 2^24,
 * so one draw is used: u = float(draw) / 2^32, pulled below 1 when the float
 * rounding of the draw reaches 2^32. */
float oracle_canonical_f32(uint32_t draw) {
    float u = (float)draw / 4294967296.0f;
    if (u >= 1.0f) u = nextafterf(1.0f, 0.0f);
    return u;
}

/* uniform_real_distribution<float>(a, b): canonical * (b - a) + a, in float. */
float oracle_uniform_f32(oracle_mt19937* g, float a, float b) {
    const float u = oracle_canonical_f32(oracle_mt_next(g));
    const float span = b - a;
    volatile float prod = u * span; /* two roundings, as in the library (no FMA) */
    return prod + a;
}

/* ======================================================================
 * Generators
 * ==================================================================== */
long oracle_generate_uniform_csr(int rows, int cols, float density, int seed, int* row_ptr,
                                 int* col_idx, float* values, long capacity) {
    oracle_mt19937 g;
    oracle_mt_seed(&g, (uint32_t)seed);
    long nnz = 0;
    if (row_ptr) row_ptr[0] = 0;
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) {
            const float u = oracle_uniform_f32(&g, 0.0f, 1.0f);
            if (u < density) {
                const float v = oracle_uniform_f32(&g, -1.0f, 1.0f);
                if (nnz < capacity && col_idx && values) {
                    col_idx[nnz] = c;
                    values[nnz] = v;
                }
                ++nnz;
            }
        }
        if (row_ptr) row_ptr[r + 1] = (int)nnz;
    }
    return (nnz <= capacity || capacity == 0) ? nnz : -1;
}

void oracle_generate_dense(int rows, int cols, int seed, float* out) {
    oracle_mt19937 g;
    oracle_mt_seed(&g, (uint32_t)seed);
    const long n = (long)rows * cols;
    for (long i = 0; i < n; ++i) out[i] = oracle_uniform_f32(&g, -1.0f, 1.0f);
}

/* ======================================================================
 * COO -> CSR: stable merge sort of indices by (row, col)
 * ==================================================================== */
typedef struct { const int* r; const int* c; } coo_keys;

static int key_less(const coo_keys* k, long a, long b) {
    if (k->r[a] != k->r[b]) return k->r[a] < k->r[b];
    return k->c[a] < k->c[b];
}

static void merge_sort(const coo_keys* k, long* idx, long* tmp, long n) {
    if (n < 2) return;
    const long h = n / 2;
    merge_sort(k, idx, tmp, h);
    merge_sort(k, idx + h, tmp, n - h);
    long i = 0, j = h, o = 0;
    while (i < h && j < n) {
        /* take from the right only when strictly smaller: stability */
        if (key_less(k, idx[j], idx[i])) tmp[o++] = idx[j++];
        else tmp[o++] = idx[i++];
    }
    while (i < h) tmp[o++] = idx[i++];
    while (j < n) tmp[o++] = idx[j++];
    memcpy(idx, tmp, sizeof(long) * (size_t)n);
}

int oracle_coo_to_csr(int rows, long n, const int* r, const int* c, const float* v, int* row_ptr,
                      int* col_idx, float* values) {
    for (long i = 0; i < n; ++i) {
        if (r[i] < 0 || r[i] >= rows) return -1;
    }
    long* idx = (long*)malloc(sizeof(long) * (size_t)(n > 0 ? n : 1));
    long* tmp = (long*)malloc(sizeof(long) * (size_t)(n > 0 ? n : 1));
    if (!idx || !tmp) {
        free(idx);
        free(tmp);
        return -2;
    }
    for (long i = 0; i < n; ++i) idx[i] = i;
    coo_keys keys = {r, c};
    merge_sort(&keys, idx, tmp, n);
    for (int i = 0; i <= rows; ++i) row_ptr[i] = 0;
    for (long i = 0; i < n; ++i) {
        col_idx[i] = c[idx[i]];
        values[i] = v[idx[i]];
        row_ptr[r[idx[i]] + 1] += 1;
    }
    for (int i = 0; i < rows; ++i) row_ptr[i + 1] += row_ptr[i];
    free(idx);
    free(tmp);
    return 0;
}

/* ======================================================================
 * Partition (spmm_multigpu.cu:26-40)
 * ==================================================================== */
void oracle_nnz_balanced_bounds(int M, const int* row_ptr, int parts, int* bounds) {
    const long long total = row_ptr[M];
    bounds[0] = 0;
    bounds[parts] = M;
    int r = 0;
    for (int g = 1; g < parts; ++g) {
        const long long target = total * g / parts;
        while (r < M && row_ptr[r] < target) ++r;
        bounds[g] = r;
    }
    for (int g = 1; g <= parts; ++g) {
        if (bounds[g] < bounds[g - 1]) bounds[g] = bounds[g - 1];
    }
}

/* ======================================================================
 * CSR SpMM, fp64 accumulation
 * ==================================================================== */
typedef struct {
    int r0, r1, N;
    const int* row_ptr;
    const int* col_idx;
    const float* values;
    const float* B;
    double* C;
    double* abs_c;
} csr_job;

static void* csr_rows(void* arg) {
    const csr_job* j = (const csr_job*)arg;
    const int N = j->N;
    for (int r = j->r0; r < j->r1; ++r) {
        double* crow = j->C + (size_t)r * N;
        double* arow = j->abs_c ? j->abs_c + (size_t)r * N : NULL;
        for (int n = 0; n < N; ++n) crow[n] = 0.0;
        if (arow) for (int n = 0; n < N; ++n) arow[n] = 0.0;
        for (int p = j->row_ptr[r]; p < j->row_ptr[r + 1]; ++p) {
            const double v = (double)j->values[p];
            const float* brow = j->B + (size_t)j->col_idx[p] * N;
            for (int n = 0; n < N; ++n) crow[n] += v * (double)brow[n];
            if (arow) {
                const double av = fabs(v);
                for (int n = 0; n < N; ++n) arow[n] += av * fabs((double)brow[n]);
            }
        }
    }
    return NULL;
}

void oracle_csr_spmm_f64(int M, int N, const int* row_ptr, const int* col_idx,
                         const float* values, const float* B, double* C, double* abs_c,
                         int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    int bounds[257];
    oracle_nnz_balanced_bounds(M, row_ptr, threads, bounds);
    csr_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        csr_job j = {bounds[t], bounds[t + 1], N, row_ptr, col_idx, values, B, C, abs_c};
        jobs[t] = j;
    }
    if (threads == 1) {
        csr_rows(&jobs[0]);
        return;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, csr_rows, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
}

/* ======================================================================
 * CSR SpMM as the reference's baseline kernel computes it
 * (src/kernels/spmm_baseline.cu:11-25): per output, sum = 0.f, then
 * sum += values[p] * B[col_idx[p]][j] for p in CSR order, which nvcc's default
 * contraction makes one fused multiply-add per entry.  fmaf is the correctly
 * rounded fused operation; this file is built with -ffp-contract=off, so no
 * other expression is fused.
 * ====================================================================== */

void oracle_csr_spmm_f32_fma(int M, int N, const int* row_ptr, const int* col_idx,
                             const float* values, const float* B, float* C) {
    for (int r = 0; r < M; ++r) {
        float* crow = C + (size_t)r * N;
        for (int n = 0; n < N; ++n) {
            float sum = 0.f;
            for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
                sum = fmaf(values[p], B[(size_t)col_idx[p] * N + n], sum);
            }
            crow[n] = sum;
        }
    }
}

/* ======================================================================
 * fp16, round to nearest even (IEEE 754 binary16)
 * ==================================================================== */
uint16_t oracle_f32_to_f16(float x) {
    uint32_t bits;
    memcpy(&bits, &x, sizeof bits);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t exp = (bits >> 23) & 0xffu;
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan: keep the top payload bits, force a quiet NaN */
        if (mant == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (mant >> 13));
    }
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* may carry into inf */
        return (uint16_t)(sign | h);
    }
    /* binary16 subnormal or zero: value = full * 2^(exp-150), half = m * 2^-24 */
    if (exp == 0) return sign; /* fp32 subnormals are far below half's range */
    const uint32_t full = mant | 0x800000u;
    const int shift = 14 - e; /* >= 14 */
    if (shift > 24) return sign;
    uint32_t m = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return (uint16_t)(sign | m);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else if (exp != 0) {
        bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    } else if (mant == 0) {
        bits = sign;
    } else {
        /* subnormal: mant * 2^-24 */
        const float f = (float)mant * (1.0f / 16777216.0f);
        memcpy(&bits, &f, sizeof bits);
        bits |= sign;
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

/* ======================================================================
 * BSR build: the reference's three passes (bsr.cu:30-109)
 * ==================================================================== */
static int cmp_int(const void* a, const void* b) {
    const int x = *(const int*)a, y = *(const int*)b;
    return (x > y) - (x < y);
}

/* Sorted unique block-columns of block-row br into buf; returns their count. */
static int block_cols_of_row(int br, int M, const int* row_ptr, const int* col_idx, int* buf) {
    int n = 0;
    const int r_end = (br + 1) * 16 < M ? (br + 1) * 16 : M;
    for (int r = br * 16; r < r_end; ++r) {
        for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p) buf[n++] = col_idx[p] / 16;
    }
    qsort(buf, (size_t)n, sizeof(int), cmp_int);
    int u = 0;
    for (int i = 0; i < n; ++i) {
        if (u == 0 || buf[u - 1] != buf[i]) buf[u++] = buf[i];
    }
    return u;
}

static int max_block_row_nnz(int M, const int* row_ptr) {
    int best = 0;
    for (int br = 0; br * 16 < M; ++br) {
        const int r_end = (br + 1) * 16 < M ? (br + 1) * 16 : M;
        const int n = row_ptr[r_end] - row_ptr[br * 16];
        if (n > best) best = n;
    }
    return best;
}

long oracle_bsr_count(int M, int K, const int* row_ptr, const int* col_idx, int* block_row_ptr) {
    (void)K;
    const int block_rows = (M + 15) / 16;
    int* buf = (int*)malloc(sizeof(int) * (size_t)(max_block_row_nnz(M, row_ptr) + 1));
    block_row_ptr[0] = 0;
    for (int br = 0; br < block_rows; ++br) {
        block_row_ptr[br + 1] = block_row_ptr[br] + block_cols_of_row(br, M, row_ptr, col_idx, buf);
    }
    free(buf);
    return block_rows > 0 ? block_row_ptr[block_rows] : 0;
}

int oracle_bsr_fill(int M, int K, const int* row_ptr, const int* col_idx, const float* values,
                    const int* block_row_ptr, int* block_col_idx, uint16_t* block_values) {
    const int block_rows = (M + 15) / 16;
    const int nnz = row_ptr[M];
    for (int p = 0; p < nnz; ++p) {
        if (col_idx[p] < 0 || col_idx[p] >= K) return -1;
    }
    int* buf = (int*)malloc(sizeof(int) * (size_t)(max_block_row_nnz(M, row_ptr) + 1));
    const long nb = block_rows > 0 ? block_row_ptr[block_rows] : 0;
    float* staging = (float*)calloc((size_t)(nb > 0 ? nb : 1) * 256, sizeof(float));
    for (int br = 0; br < block_rows; ++br) {
        const int cnt = block_cols_of_row(br, M, row_ptr, col_idx, buf);
        const int base = block_row_ptr[br];
        for (int i = 0; i < cnt; ++i) block_col_idx[base + i] = buf[i];
        const int r_end = (br + 1) * 16 < M ? (br + 1) * 16 : M;
        for (int r = br * 16; r < r_end; ++r) {
            for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
                const int bc = col_idx[p] / 16;
                /* binary search for bc among this block-row's columns */
                int lo = 0, hi = cnt;
                while (lo < hi) {
                    const int mid = (lo + hi) / 2;
                    if (buf[mid] < bc) lo = mid + 1; else hi = mid;
                }
                staging[(size_t)(base + lo) * 256 + (r % 16) * 16 + col_idx[p] % 16] = values[p];
            }
        }
    }
    for (long i = 0; i < nb * 256; ++i) block_values[i] = oracle_f32_to_f16(staging[i]);
    free(staging);
    free(buf);
    return 0;
}

void oracle_bsr_stats(int M, int K, long num_blocks, long nnz, double* fill_in_ratio,
                      double* block_density, long* stored_elements) {
    const long stored = num_blocks * 256;
    const long all = (long)((M + 15) / 16) * ((K + 15) / 16);
    if (stored_elements) *stored_elements = stored;
    if (fill_in_ratio) *fill_in_ratio = nnz > 0 ? (double)stored / (double)nnz : 0.0;
    if (block_density) *block_density = all > 0 ? (double)num_blocks / (double)all : 0.0;
}

/* ======================================================================
 * BSR SpMM, fp32 accumulation over fp16 operands
 * ==================================================================== */
typedef struct {
    int br0, br1, M, K, N;
    const int* brp;
    const int* bci;
    const uint16_t* bv;
    const uint16_t* B16;
    float* C;
} bsr_job;

static void* bsr_rows(void* arg) {
    const bsr_job* j = (const bsr_job*)arg;
    const int N = j->N;
    for (int br = j->br0; br < j->br1; ++br) {
        for (int lr = 0; lr < 16; ++lr) {
            const int r = br * 16 + lr;
            if (r >= j->M) break;
            float* crow = j->C + (size_t)r * N;
            for (int n = 0; n < N; ++n) crow[n] = 0.0f;
            for (int b = j->brp[br]; b < j->brp[br + 1]; ++b) {
                const int k0 = j->bci[b] * 16;
                for (int lk = 0; lk < 16; ++lk) {
                    const int k = k0 + lk;
                    if (k >= j->K) break;
                    const float a = oracle_f16_to_f32(j->bv[(size_t)b * 256 + lr * 16 + lk]);
                    const uint16_t* brow = j->B16 + (size_t)k * N;
                    for (int n = 0; n < N; ++n) {
                        const float prod = a * oracle_f16_to_f32(brow[n]); /* exact */
                        crow[n] = crow[n] + prod;
                    }
                }
            }
        }
    }
    return NULL;
}

void oracle_bsr_spmm_f32(int M, int K, int N, const int* block_row_ptr, const int* block_col_idx,
                         const uint16_t* block_values, const uint16_t* B16, float* C,
                         int threads) {
    const int block_rows = (M + 15) / 16;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads > block_rows) threads = block_rows > 0 ? block_rows : 1;
    bsr_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        bsr_job j = {(int)((long long)block_rows * t / threads),
                     (int)((long long)block_rows * (t + 1) / threads),
                     M, K, N, block_row_ptr, block_col_idx, block_values, B16, C};
        jobs[t] = j;
    }
    if (threads == 1) {
        bsr_rows(&jobs[0]);
        return;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, bsr_rows, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
}

/* ======================================================================
 * Dispatch rule and metrics
 * ==================================================================== */
int oracle_hybrid_rule(double fill_in_ratio, int N, float threshold, int* reason_id) {
    const int aligned = (N > 0) && (N % 16 == 0);
    const int dense_blocks = fill_in_ratio <= (double)threshold;
    int use_mfma = 0, why;
    if (aligned && dense_blocks) {
        use_mfma = 1;
        why = 0;
    } else if (!aligned) {
        why = 1;
    } else {
        why = 2;
    }
    if (reason_id) *reason_id = why;
    return use_mfma;
}

void oracle_compare(const float* ours, const float* ref, long n, float* max_abs, float* max_rel,
                    float* rel_l2) {
    float peak = 0.0f, mabs = 0.0f, mrel = 0.0f;
    for (long i = 0; i < n; ++i) {
        const float a = fabsf(ref[i]);
        if (a > peak) peak = a;
    }
    const float floor_rel = 1e-3f * peak;
    double e2 = 0.0, r2 = 0.0;
    for (long i = 0; i < n; ++i) {
        const float d = fabsf(ours[i] - ref[i]);
        const float a = fabsf(ref[i]);
        if (d > mabs) mabs = d;
        if (a > floor_rel && d / a > mrel) mrel = d / a;
        e2 += (double)d * (double)d;
        r2 += (double)a * (double)a;
    }
    if (max_abs) *max_abs = mabs;
    if (max_rel) *max_rel = mrel;
    if (rel_l2) *rel_l2 = r2 > 0.0 ? (float)sqrt(e2 / r2) : 0.0f;
}

float oracle_rel_l2(const float* ours, const float* ref, long n) {
    double e2 = 0.0, r2 = 0.0;
    for (long i = 0; i < n; ++i) {
        const double d = (double)ours[i] - (double)ref[i];
        e2 += d * d;
        r2 += (double)ref[i] * (double)ref[i];
    }
    return r2 > 0.0 ? (float)sqrt(e2 / r2) : 0.0f;
}

static int cmp_float(const void* a, const void* b) {
    const float x = *(const float*)a, y = *(const float*)b;
    return (x > y) - (x < y);
}

float oracle_median(float* v, int n) {
    if (n <= 0) return 0.0f;
    qsort(v, (size_t)n, sizeof(float), cmp_float);
    return v[n / 2];
}
