/*
 * C ABI of the MI355X SpMM engine (libspmm_amd.so).
 *
 * The reference exposes a C++ API only (namespace spmm, the src/ headers); this header
 * is the flat binding an FFI (ctypes, cgo, JNI, N-API) would load.  Each entry
 * point names the reference declaration it stands for.  The same library also
 * exports that C++ API itself (the include/spmm/ headers).
 *
 * Conventions
 *   - Plain pointers and sizes only.  spmm_csr_t / spmm_bsr_t have the field
 *     order and layout of spmm::CSR / spmm::BSR (csr.h:7-14, bsr.h:45-56);
 *     fp16 data is passed as uint16_t bit patterns.
 *   - "d_" pointers are device (HBM) pointers, "h_" pointers host pointers.
 *   - Every function returns SPMM_OK (0) or an error code and never exits the
 *     process; spmm_c_last_error() gives the message of the calling thread's
 *     last failure.  (The C++ API keeps the reference's exit/abort behaviour.)
 *   - stream: a hipStream_t passed as void*; NULL is the null stream, which is
 *     what the reference launchers use.  Launchers enqueue and return without
 *     synchronising.
 *   - Host structs filled by this library (spmm_c_generate_*, *_from_*_host,
 *     *_read_binary_host) own malloc'd arrays: release them with
 *     spmm_c_csr_free_host / spmm_c_bsr_free_host.
 */
#ifndef SPMM_CAPI_H
#define SPMM_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SPMM_OK          = 0,
    SPMM_INVALID     = 1, /* bad argument */
    SPMM_UNSUPPORTED = 2, /* shape contract of the entry point violated */
    SPMM_HIP_ERROR   = 3, /* HIP runtime error */
    SPMM_IO_ERROR    = 4, /* file missing or short */
    SPMM_NO_MEMORY   = 5  /* host allocation failed */
};

/* Backend ids of spmm_hybrid_plan_t.backend (spmm_hybrid.h:26-29). */
enum { SPMM_BACKEND_CSR = 0, SPMM_BACKEND_WMMA = 1 };

typedef struct spmm_csr_t {
    int    num_rows;
    int    num_cols;
    int    nnz;
    int*   row_ptr;
    int*   col_idx;
    float* values;
} spmm_csr_t;

typedef struct spmm_bsr_t {
    int       num_rows;
    int       num_cols;
    int       block_rows;
    int       block_cols;
    int       num_blocks;
    int       nnz;
    int*      row_ptr;
    int*      col_idx;
    uint16_t* values; /* fp16 bits, 256 per block, row-major inside a block */
} spmm_bsr_t;

typedef struct spmm_bsr_stats_t {
    int    num_blocks;
    long   stored_elements;
    int    original_nnz;
    double fill_in_ratio;
    double block_density;
} spmm_bsr_stats_t;

typedef struct spmm_hybrid_plan_t {
    int         backend; /* SPMM_BACKEND_* */
    double      fill_in_ratio;
    double      block_density;
    float       threshold;
    int         n_aligned;
    const char* reason; /* static string */
} spmm_hybrid_plan_t;

/* Engine tuning (0 = automatic).  No counterpart in the reference: exposes the
 * row-block engine's compile-time variants for measurement sweeps. */
typedef struct spmm_engine_opts_t {
    int vec;            /* floats per lane per B load: 1, 2, 4 */
    int waves;          /* waves per workgroup: 2, 4, 8 */
    int unroll;         /* B row segments per lane per step (two steps in flight): 4, 8 */
    int rows_per_block; /* implicit partition granularity */
    int groups;         /* lane groups per wave, entries interleaved: 1, 2, 4 */
    int slices;         /* XCD-tied column slices of B and C: 1, 2, 4, 8 */
    int global_loads;   /* 1: 64-bit address loads of B instead of buffer loads
                           (automatic when B exceeds 2 GiB or N > 4095) */
    int row_groups;     /* sub-wave row groups instead of the row-block engine:
                           one row per group of column lanes x entry lanes, no
                           partition, buffer loads only (N <= 4095, B < 2 GiB);
                           vec as above, unroll 2 or 4.  1: index-load form
                           chosen from the shape, 2: per-lane index loads,
                           3: cooperative index loads.  0: the engine, except
                           that default launches of tiled_v3 / tiled_v4 with
                           N <= 16 (at most four 16-byte column lanes), or
                           N <= 32 on up to 4 M nonzeros, take the
                           row groups */
    int entry_lanes;    /* row groups: entry lanes per row, power of two <= 64 */
    int max_row_hint;   /* longest row's entries if known (0 = unknown).
                           row_groups != 0: lets the kernel drop its long-row
                           pass when no row needs it (a hint below the true
                           longest row is still correct: each group then sums
                           its long row itself, which only costs time).
                           row_groups == 0: the row-block engine (also for the
                           narrow B that takes row groups by default); rows
                           within 2 x average + 32 entries give it a grid of
                           whole rounds of 4-wave workgroups; a wrong hint only
                           costs time */
} spmm_engine_opts_t;

/* BSR matrix-core kernel tuning (0 = automatic).  No counterpart in the
 * reference: exposes the kernels' variants for measurement sweeps.  Default:
 * the shared-panel kernel on wide B with long structured block-rows (N >= 256,
 * 24 - 64 blocks per block-row on average, K <= 131072), else the wave kernel. */
typedef struct spmm_bsr_opts_t {
    int row_group;  /* 0: automatic; 1: wave kernel (one wave per block-row);
                       4, 8: shared-panel kernel with that many block-rows per
                       workgroup sharing staged B tiles */
    int tiles;      /* wave kernel: 16-column MFMA tiles per wave, 1, 2, 4;
                       panel kernel: 16-column tiles per workgroup, 4 or 8 */
    int per_wave;   /* 1: wave kernel whatever row_group says */
    int depth;      /* wave kernel: block pairs in flight per wave, 1, 2, 4;
                       panel kernel: LDS stages in flight, 2 or 4.
                       tiles / depth 0: the kernel's default.  Values no
                       kernel has, or (row_group 1 / 4 / 8, per_wave) values
                       the named kernel lacks, are SPMM_INVALID; under the
                       automatic choice the chosen kernel's default replaces
                       a value it lacks. */
    int xcd_order;  /* 0, 1 XCD-grouped workgroup order; 2 dispatch order */
    int reserved0;  /* must be 0: held the removed multi-row wave variant's
                       block-rows per wave; nonzero is SPMM_INVALID */
    int reserved1;  /* must be 0: held the removed split-K wave variant;
                       nonzero is SPMM_INVALID */
    int addressing; /* 0: B rows / A blocks as buffer records where they fit
                       (N % 8 == 0, 16-byte aligned B); 1: pointer-arithmetic
                       wave kernel */
} spmm_bsr_opts_t;

const char* spmm_c_last_error(void);
const char* spmm_c_version(void);

/* ---- host CSR (csr.h:17-39) ------------------------------------------- */
int spmm_c_csr_alloc_host(int rows, int cols, int nnz, spmm_csr_t* out);   /* csr.h:17 */
void spmm_c_csr_free_host(spmm_csr_t* m);                                  /* csr.h:18 */
int spmm_c_csr_from_coo_host(int rows, int cols, int n, const int* row_indices,
                             const int* col_indices, const float* values,
                             spmm_csr_t* out);                             /* csr.h:21 */
int spmm_c_generate_uniform_random_csr(int rows, int cols, float density, int seed,
                                       spmm_csr_t* out);                   /* csr.h:25 */
int spmm_c_csr_row_slice_host(const spmm_csr_t* m, int row_begin, int row_end,
                              spmm_csr_t* out);                            /* csr.h:30 */
int spmm_c_csr_read_binary_host(const char* path, spmm_csr_t* out);        /* csr.h:34 */
int spmm_c_csr_write_binary_host(const spmm_csr_t* m, const char* path);   /* csr.h:35 */
int spmm_c_csr_to_device(const spmm_csr_t* h, spmm_csr_t* d_out);          /* csr.h:38 */
int spmm_c_csr_free_device(spmm_csr_t* d);                                 /* csr.h:39 */

/* ---- BSR (bsr.h:71-80) ------------------------------------------------ */
int spmm_c_bsr_from_csr_host(const spmm_csr_t* h, spmm_bsr_t* out);       /* bsr.h:71 */
void spmm_c_bsr_free_host(spmm_bsr_t* h);                                  /* BSR_host dtor */
int spmm_c_bsr_to_device(const spmm_bsr_t* h, spmm_bsr_t* d_out);          /* bsr.h:74 */
int spmm_c_bsr_free_device(spmm_bsr_t* d);                                 /* bsr.h:77 */
int spmm_c_bsr_compute_stats(const spmm_bsr_t* h, spmm_bsr_stats_t* out);  /* bsr.h:80 */
/* Additions with no reference counterpart (the reference builds BSR on the host
 * only, bsr.cu:30-109): stats of a host CSR without building the blocks; CSR ->
 * BSR and its stats on the device from a device CSR (column indices ascending
 * within each row, num_cols <= 4128768; SPMM_UNSUPPORTED otherwise; the device
 * BSR is released with spmm_c_bsr_free_device); device BSR -> host copy
 * (release with spmm_c_bsr_free_host). */
int spmm_c_bsr_stats_from_csr_host(const spmm_csr_t* h, spmm_bsr_stats_t* out);
int spmm_c_bsr_from_csr_device(const spmm_csr_t* d_A, spmm_bsr_t* d_out, void* stream);
int spmm_c_bsr_stats_from_csr_device(const spmm_csr_t* d_A, spmm_bsr_stats_t* out,
                                     void* stream);
int spmm_c_bsr_to_host(const spmm_bsr_t* d, spmm_bsr_t* h_out);

/* ---- synthetic inputs (harness.cu:114-120, gen_matrices.py:37-81) ----- */
int spmm_c_generate_dense_row_major(int rows, int cols, int seed, float* h_out);
int spmm_c_generate_banded_csr(int rows, int cols, int half_bandwidth, int seed,
                               spmm_csr_t* out);
int spmm_c_generate_block_diagonal_csr(int rows, int cols, int block, int seed,
                                       float value_scale, spmm_csr_t* out);
/* same structure, values U[-1,1) as gen_matrices.py:62 */
int spmm_c_generate_block_diagonal_uniform_csr(int rows, int cols, int block, int seed,
                                               spmm_csr_t* out);
int spmm_c_generate_power_law_csr(int rows, int cols, double mean_deg, double alpha,
                                  int max_row_nnz, int seed, spmm_csr_t* out);
int spmm_c_round_to_fp16(float* h_values, long n); /* values := fp32(fp16_rne(values)) */

/* ---- partition and metrics (spmm_multigpu.cu:26-40, harness.cu:179-201) */
int spmm_c_nnz_balanced_bounds(const spmm_csr_t* h, int parts, int* h_bounds_out);
int spmm_c_compare(const float* ours, const float* ref, long n, float* max_abs,
                   float* max_rel, float* rel_l2);
int spmm_c_host_reference_f64(const spmm_csr_t* h_A, const float* h_B, int N, int threads,
                              float* h_C);
int spmm_c_host_reference_bsr_f32(const spmm_bsr_t* h_A, const float* h_B, int N,
                                  int threads, float* h_C);

/* ---- kernel entry points (the src/kernels/ headers); d_A is a device CSR -------- */
int spmm_c_baseline(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                    void* stream);                               /* spmm_baseline.h:17  */
int spmm_c_memopt(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                  void* stream);                                 /* spmm_memopt.h:18    */
int spmm_c_memopt_v2(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                     void* stream);                              /* spmm_memopt_v2.h:26 */
int spmm_c_tiled(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                 void* stream);                                  /* spmm_tiled.h:45     */
int spmm_c_tiled_v2(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                    void* stream);                               /* spmm_tiled_v2.h:38  */
int spmm_c_tiled_v3(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                    void* stream);                               /* spmm_tiled_v3.h:40  */
int spmm_c_tiled_v4(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                    void* stream);                               /* spmm_tiled_v4.h:79  */
/* spmm_tiled_v3 with an explicit nnz-balanced row partition: d_bounds holds
 * parts+1 row bounds (spmm_c_nnz_balanced_bounds, the reference's split of
 * spmm_multigpu.cu:26-40 applied to workgroups). */
int spmm_c_tiled_v3_partitioned(const spmm_csr_t* d_A, const int* d_bounds, int parts,
                                const float* d_B, float* d_C, int N, void* stream);
/* Default number of parts for spmm_c_tiled_v3_partitioned. */
int spmm_c_default_partition_parts(int num_rows, int nnz);
/* Merge-path partition (no counterpart in the reference; used by spmm_hybrid_run):
 * part g multiplies nonzeros [nnz*g/parts, nnz*(g+1)/parts), cutting long rows
 * between workgroups (1 <= parts <= max(nnz, 1), else SPMM_INVALID).
 * d_split_rows: parts+1 ints from spmm_c_nnz_split_rows;
 * d_carry: a workspace of parts * N floats.  Two launches (the engine, then
 * the carry fix-up); results are deterministic. */
int spmm_c_nnz_split_rows(const spmm_csr_t* h, int parts, int* h_rows_out);
int spmm_c_split_partition_parts(int nnz);
int spmm_c_tiled_v3_split(const spmm_csr_t* d_A, const int* d_split_rows, int parts,
                          const float* d_B, float* d_C, int N, float* d_carry, void* stream);
/* spmm_c_tiled_v3_split without the caller's workspace: the carries live in a
 * file-scope device array of 2^19 floats (2 MiB) that each GPU holds from the
 * first call on it until the process ends.  No counterpart in the reference:
 * it is for callers that cannot allocate (HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc); it calls no allocating routine.  parts x
 * N above 2^19 returns SPMM_UNSUPPORTED.  All calls on one GPU share its array:
 * calls that overlap on one GPU race. */
int spmm_c_tiled_v3_split_noalloc(const spmm_csr_t* d_A, const int* d_split_rows, int parts,
                                  const float* d_B, float* d_C, int N, void* stream);
/* The CSR form spmm_hybrid_run's CSR branch picks for host CSR h and a B of N
 * columns (no counterpart in the reference): *form_out = 0 the row-block
 * engine, 1 sub-wave row groups, 2 the merge-path partition, 3 the merge-path
 * partition over B-row halves (spmm_c_khalf_*); *opts_out the launch options
 * for spmm_c_tiled_v3_opts (forms 0 and 1: the longest row as max_row_hint,
 * row_groups = 1 for form 1); *parts_out the merge-path parts (form 2, else
 * 0).  Host only. */
int spmm_c_csr_auto_form(const spmm_csr_t* h, int N, int* form_out,
                         spmm_engine_opts_t* opts_out, int* parts_out);
/* Merge-path partition over B-row halves (no counterpart in the reference;
 * spmm_hybrid_run's CSR form when B is over one XCD's 4 MiB L2 at full width
 * and half of its rows fit, form 3 above).  A's entries with column < K/2 and
 * the rest each get their own merge-path partition; XCDs 0-3 multiply the
 * first half by B rows [0, K/2) and XCDs 4-7 the second by rows [K/2, K), each
 * over all N columns; a second kernel adds the halves' carries and the second
 * half's partial rows to C in a fixed order (deterministic).
 * create: h_A is a host CSR with columns in [0, num_cols); uploads both halves
 *   and allocates the plan's workspaces (an M x N partial, parts x N carries
 *   per half).  SPMM_UNSUPPORTED unless N % 4 == 0, num_cols x N x 4 bytes is
 *   over 4 MiB with half of the rows within it (and N x 4 <= 16383, B within
 *   2 GiB), and each half holds at least 512 entries.
 * launch: d_B (num_cols x N, the N given to create) and d_C (M x N), fp32,
 *   16-byte aligned; two kernels on `stream`; the plan's workspaces are shared by its launches, so
 *   launches of one plan must not overlap.
 * runs: host helper behind the fix-up's per-row carry table -- for the
 *   merge-path partition of row_ptr (M rows, nnz entries) into parts with row
 *   table split_rows, first[r] / last[r] = the first and last part continuing
 *   row r (whose first nonzero lies in an earlier part), -1 when none. */
typedef struct spmm_khalf_plan spmm_khalf_plan_t;
int  spmm_c_khalf_plan_create(const spmm_csr_t* h_A, int N, spmm_khalf_plan_t** plan_out);
int  spmm_c_khalf_launch(const spmm_khalf_plan_t* plan, const float* d_B, float* d_C,
                         void* stream);
void spmm_c_khalf_plan_destroy(spmm_khalf_plan_t* plan);
int  spmm_c_khalf_runs(const int* row_ptr, int M, long long nnz, const int* split_rows,
                       int parts, int* first_out, int* last_out);
/* spmm_tiled_v3 with explicit engine options (no reference counterpart). */
int spmm_c_tiled_v3_opts(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                         const spmm_engine_opts_t* opts, void* stream);

int spmm_c_float_to_half(const float* d_src, uint16_t* d_dst, long n_elements,
                         void* stream);                          /* spmm_wmma.h:32 */
int spmm_c_wmma(const spmm_bsr_t* d_bsr, const uint16_t* d_B_fp16, float* d_C, int N,
                void* stream);                                   /* spmm_wmma.h:39 */
/* spmm_wmma with explicit kernel options (no reference counterpart). */
int spmm_c_wmma_opts(const spmm_bsr_t* d_bsr, const uint16_t* d_B_fp16, float* d_C, int N,
                     const spmm_bsr_opts_t* opts, void* stream);

/* Run-panel form of spmm_wmma (no counterpart in the reference; the form
 * spmm_c_hybrid_run runs when every block-row of the BSR is a run of
 * consecutive block-columns and each panel's runs cover their union without a
 * gap, as in banded and block-diagonal matrices).  The plan holds one record
 * per panel of rows_per_panel (4 or 8) block-rows; the kernel then reads no
 * row_ptr / col_idx.
 * create: reads the device BSR's row_ptr and col_idx back (synchronises
 *   `stream`) and uploads the records; SPMM_UNSUPPORTED when the structure is
 *   not runs as above (use spmm_c_wmma then).
 * launch: d_A must carry the row_ptr / col_idx arrays the plan was created
 *   from (SPMM_INVALID otherwise; its values may change between launches);
 *   d_B (num_cols x N fp16 bits) and d_C (num_rows x N fp32) 16-byte
 *   aligned, N % 8 == 0, N * 2 <= 16383; shape < 0 picks the default kernel
 *   shape (spmm_c_bsr_tile_shape lists them); the result equals spmm_c_wmma's
 *   within fp32 rounding (same products, same pairwise K order).
 * records: the host part of create, for callers with a host copy of the
 *   block structure: panels x 32 ints into records_out (room for
 *   ceil(block_rows / rows_per_panel) x 32), *max_union_out the widest union. */
typedef struct spmm_bsr_tile_plan spmm_bsr_tile_plan_t;
int  spmm_c_bsr_tile_plan_create(const spmm_bsr_t* d_A, int rows_per_panel, void* stream,
                                 spmm_bsr_tile_plan_t** plan_out);
int  spmm_c_bsr_tile_launch(const spmm_bsr_tile_plan_t* plan, const spmm_bsr_t* d_A,
                            const uint16_t* d_B_fp16, float* d_C, int N, int shape,
                            void* stream);
void spmm_c_bsr_tile_plan_destroy(spmm_bsr_tile_plan_t* plan);
int  spmm_c_bsr_tile_plan_info(const spmm_bsr_tile_plan_t* plan, int* panels_out,
                               int* rows_per_panel_out, int* max_union_out);
int  spmm_c_bsr_tile_records(const int* row_ptr, const int* col_idx, int block_rows,
                             int block_cols, int rows_per_panel, int* records_out,
                             int* max_union_out);
/* Kernel shapes: count, and shape id's (rows per panel, columns per
 * workgroup, wave columns, slots per chunk, chunk buffers, kind: 0 ring with
 * A in VGPRs, 1 whole union with A in VGPRs, 2 producer / consumer waves);
 * the default shape for a plan and N columns. */
int  spmm_c_bsr_tile_shape_count(void);
int  spmm_c_bsr_tile_shape(int id, int* fields_out /* 6 ints */);
int  spmm_c_bsr_tile_default_shape(const spmm_bsr_tile_plan_t* plan, int N);

/* ---- hybrid dispatch (spmm_hybrid.h:48-64) ---------------------------- */
/* The wide-B cut-off (N >= 256) and the per-N MI355X crossover; no
 * counterpart in the reference (its default is the constant 2.0). */
float spmm_c_hybrid_default_threshold(void);
float spmm_c_hybrid_default_threshold_for(int N);
/* fill_in_threshold < 0 selects spmm_c_hybrid_default_threshold_for(N).
 * The host-in calls (choose, run, unified) return SPMM_INVALID for a host CSR
 * with negative sizes, no row_ptr, or entries without col_idx (or, to run,
 * without values), before reading it or touching the device. */
int spmm_c_hybrid_choose(const spmm_csr_t* h_A, int N, float fill_in_threshold,
                         spmm_hybrid_plan_t* out);               /* spmm_hybrid.h:48 */
const char* spmm_c_backend_name(int backend);                    /* spmm_hybrid.h:51 */
/* ---- unified memory on one GPU (spmm_multigpu.h:32, :54-58) ----------- */
int spmm_c_gpu_count(void);                                                /* spmm_multigpu.h:32 */
/* A, B, C in managed memory, prefetched, tiled_v3 engine.  *prefetched_out:
 * 1 prefetched; 0 the device could not prefetch (pages then move on first
 * touch); -1 the device has no managed memory (MI355X with XNACK off): device
 * allocations filled by explicit copies stand in for the managed ranges, the
 * state a prefetch reaches, and the GPU never touches host memory. */
int spmm_c_unified(const spmm_csr_t* h_A, const float* h_B, float* h_C, int N, int warmup,
                   int iters, float* ms_out, int* prefetched_out);     /* spmm_multigpu.h:57 */

int spmm_c_hybrid_run(const spmm_hybrid_plan_t* plan, const spmm_csr_t* h_A,
                      const float* h_B, float* h_C, int N, int warmup, int iters,
                      float* ms_out);                            /* spmm_hybrid.h:62 */

/* ---- measurement helpers (no reference counterpart) -------------------
 * Launch one entry point `reps` times back to back on `stream` without
 * synchronising, so a caller's events can bracket a batch.  kernel ids:
 * 0 baseline, 1 memopt, 2 memopt_v2, 3 tiled, 4 tiled_v2, 5 tiled_v3,
 * 6 tiled_v4 (d_A_any is a spmm_csr_t*), 7 wmma (d_A_any is a spmm_bsr_t*,
 * d_B a uint16_t* of fp16 bits). */
int spmm_c_launch_repeat(int kernel_id, const void* d_A_any, const void* d_B, float* d_C,
                         int N, int reps, void* stream);
/* Same with explicit engine options for kernel id 5 (tiled_v3). */
int spmm_c_launch_repeat_split(const spmm_csr_t* d_A, const int* d_split_rows, int parts,
                               const float* d_B, float* d_C, int N, float* d_carry, int reps,
                               void* stream);
int spmm_c_launch_repeat_opts(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                              const spmm_engine_opts_t* opts, int reps, void* stream);
int spmm_c_launch_repeat_khalf(const spmm_khalf_plan_t* plan, const float* d_B, float* d_C,
                               int reps, void* stream);
/* Same for the matrix-core kernel with explicit options. */
int spmm_c_launch_repeat_wmma_opts(const spmm_bsr_t* d_bsr, const uint16_t* d_B_fp16,
                                   float* d_C, int N, const spmm_bsr_opts_t* opts, int reps,
                                   void* stream);
int spmm_c_launch_repeat_bsr_tile(const spmm_bsr_tile_plan_t* plan, const spmm_bsr_t* d_A,
                                  const uint16_t* d_B_fp16, float* d_C, int N, int shape,
                                  int reps, void* stream);
/* Times `reps` back-to-back launches between two hipEvents recorded on
 * `stream`; writes the elapsed milliseconds of the whole batch. */
int spmm_c_time_repeat(int kernel_id, const void* d_A_any, const void* d_B, float* d_C,
                       int N, int reps, void* stream, float* ms_out);
int spmm_c_device_synchronize(void);
/* Shader-clock trace (no reference counterpart; a timing diagnostic): one
 * wave enqueued on `stream` writes the shader-cycle count and the 100 MHz
 * real-time tick count `samples` (2 .. 2^20) times, `interval_ticks`
 * (1 .. 1e8) ticks apart, to d_out[2i] and d_out[2i + 1] (d_out: 2 * samples
 * uint64), and ends after at most 60 s.  Launched on a second stream beside
 * a workload, 100 * dcycles / dticks is the shader clock in MHz that the
 * workload ran at during interval i. */
int spmm_c_shader_clock_trace(uint64_t* d_out, int samples, int interval_ticks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPMM_CAPI_H */
