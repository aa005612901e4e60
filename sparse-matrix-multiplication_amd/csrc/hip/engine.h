#pragma once
// Internal launch layer shared by the C++ drop-in API, the C ABI and the
// hybrid dispatcher.  Every launcher validates its arguments, enqueues on the
// given stream and returns a status; the public wrappers turn a status into
// the reference's conventions (exit / abort) or into a C error code.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "spmm/bsr.h"
#include "spmm/csr.h"
#include "spmm/spmm_hybrid.h"

namespace spmm {
namespace engine {

enum Status : int {
    kOk          = 0,
    kInvalid     = 1,  // bad argument (negative size, null pointer, misaligned)
    kUnsupported = 2,  // a shape contract of the entry point is violated
    kHipError    = 3,  // the HIP runtime reported an error
};

// Which reference entry point is being served.
enum class CsrRole : int {
    Baseline = 0,
    Memopt   = 1,
    MemoptV2 = 2,
    Tiled    = 3,
    TiledV2  = 4,
    TiledV3  = 5,
    TiledV4  = 6,
};

// Tuning of the row-block engine.  Zero fields mean "choose automatically".
struct EngineOpts {
    int vec            = 0;  // floats per lane per B load: 1, 2 or 4
    int waves          = 0;  // waves per workgroup: 2, 4 or 8
    int unroll         = 0;  // B-row loads per lane per step (two steps in flight): 4 or 8
    int rows_per_block = 0;  // implicit partition: rows per workgroup
    int groups         = 0;  // lane groups per wave (entries interleaved): 1, 2 or 4
    int slices         = 0;  // XCD-tied column slices of B and C: 1, 2, 4 or 8
    int global_loads   = 0;  // 1: 64-bit address loads of B instead of buffer loads
    // Sub-wave row groups instead of the row-block engine (one row per group
    // of column lanes x entry lanes; no partition, buffer loads only; unroll
    // 2 or 4 entries per entry lane per iteration, vec as above): 1 with the
    // index-load form chosen from the shape, 2 per-lane index loads, 3
    // cooperative index loads handed out by shuffles.  0: the engine, except
    // that default launches of spmm_tiled_v3 / _v4 with at most four column
    // lanes (N <= 16 with 16-byte lanes), or eight (N <= 32) on up to 4 M
    // nonzeros, take the row groups.
    int row_groups     = 0;
    int entry_lanes    = 0;  // row groups: entry lanes per row, a power of two up to 64
    // The longest row's entries when the caller knows it (0 = unknown).
    // row_groups != 0: with no row longer than the long-row cut, the kernel
    // is built without its workgroup-wide pass; with a hint below the true
    // longest row each group sums its long row itself (correct, slower).
    // row_groups == 0: the
    // row-block engine (a hint also keeps narrow B off the default row
    // groups); rows within 2 x average + 32 entries give its implicit
    // partition a grid of whole rounds of 4-wave workgroups instead of ~160
    // entries per wave; a wrong hint only costs time.
    int max_row_hint   = 0;
};

struct Error {
    int         status = kOk;
    std::string message;
};

// d_bounds (nullable) is a device array of parts+1 row bounds produced by
// nnz_balanced_bounds; when given, workgroup g owns rows [bounds[g], bounds[g+1]).
Error launch_csr(CsrRole role, const CSR& d_A, const float* d_B, float* d_C, int N,
                 hipStream_t stream, const int* d_bounds = nullptr, int parts = 0,
                 const EngineOpts* opts = nullptr);

Error launch_float_to_half(const float* d_src, half* d_dst, long n, hipStream_t stream);

// Shader-clock trace (clock.hip): one wave writes (shader cycles, 100 MHz
// ticks) `samples` times, `interval_ticks` apart, to d_out[2i], d_out[2i+1];
// the delivered MHz of interval i is 100 * dcycles / dticks.
Error launch_shader_clock_trace(unsigned long long* d_out, int samples, int interval_ticks,
                                hipStream_t stream);

// Tuning of the BSR matrix-core kernels.  All zero selects the default: the
// shared-panel kernel on wide B with long structured block-rows (N >= 256, 24
// - 64 blocks per block-row), else the wave kernel, with shapes from N.
struct BsrOpts {
    int row_group  = 0;  // 0: automatic; 1: wave kernel; 4, 8: panel kernel with that many
                         // block-rows per workgroup sharing staged B tiles
    int tiles      = 0;  // wave kernel: 16-column tiles per wave, 1, 2, 4;
                         // panel kernel: 16-column tiles per workgroup, 4 or 8
    int per_wave   = 0;  // 1: wave kernel whatever row_group says
    int depth      = 0;  // wave kernel: block pairs in flight per wave, 1, 2 or 4;
                         // panel kernel: LDS stages in flight, 2 or 4
    int xcd_order  = 0;  // 0, 1 XCD-grouped workgroup order; 2 dispatch order
    int addressing = 0;  // 0 buffer records where they fit, 1 pointer arithmetic (wave kernel)
};

Error launch_bsr(const BSR& d_A, const half* d_B, float* d_C, int N, hipStream_t stream,
                 const BsrOpts* opts = nullptr);

// Run-panel plan of a BSR whose block-rows are runs of consecutive
// block-columns (bsr_tile.hip).  Panel p = block-rows [pR, pR + R); its
// record of kTileDescInts ints holds the union of the runs (first
// block-column, width) and per block-row the run as union slots [lo, hi) and
// the A block of slot lo.  Device memory is owned by the plan.
constexpr int kTileDescInts = 32;
struct BsrTilePlan {
    int* desc       = nullptr;  // device, panels x kTileDescInts
    int  R          = 0;        // block-rows per panel, 4 or 8
    int  panels     = 0;
    int  num_rows   = 0;        // the matrix the plan describes (checked at launch)
    int  num_cols   = 0;
    int  block_rows = 0;
    int  num_blocks = 0;
    int  max_union  = 0;        // widest panel union, in block-columns
    const int* row_ptr = nullptr;  // the structure arrays it was built from (checked at
    const int* col_idx = nullptr;  // launch; the values may change between launches)
};
// Kernel shapes (id, R, NT columns per workgroup, WC wave columns, CS slots
// per staged chunk, NB chunk buffers, KIND).  KIND 0: A operands in VGPRs, a
// ring of NB B buffers with NB - 1 chunks in flight (any union width); 1: A
// in VGPRs, the whole union in flight (widest union <= NB * CS); 2: producer
// and consumer waves, A and B staged in LDS, the whole union in flight; 3: as
// 2 with the consumers loading their A operands straight into VGPRs.
struct TileShape {
    int R, NT, WC, CS, NB, KIND;
};
#define SPMM_TILE_SHAPES(X)      \
    X(0, 8, 64, 1, 4, 4, 2)      \
    X(1, 4, 64, 1, 4, 3, 2)      \
    X(2, 4, 128, 2, 4, 4, 2)     \
    X(3, 4, 64, 1, 4, 4, 2)      \
    X(4, 4, 128, 1, 4, 4, 2)     \
    X(5, 4, 32, 1, 4, 3, 2)      \
    X(6, 8, 64, 1, 4, 3, 2)      \
    X(7, 4, 64, 1, 4, 4, 1)      \
    X(8, 4, 32, 1, 4, 3, 1)      \
    X(9, 4, 128, 2, 4, 5, 0)     \
    X(10, 4, 64, 1, 4, 4, 0)     \
    X(11, 8, 64, 1, 4, 5, 0)     \
    X(12, 4, 32, 1, 4, 4, 2)     \
    X(13, 4, 64, 1, 4, 4, 3)     \
    X(14, 4, 32, 1, 4, 3, 3)     \
    X(15, 4, 32, 1, 4, 4, 3)     \
    X(16, 8, 64, 1, 4, 4, 3)
#define SPMM_TILE_ENTRY(ID, R_, NT_, WC_, CS_, NB_, KIND_) TileShape{R_, NT_, WC_, CS_, NB_, KIND_},
constexpr TileShape kTileShapes[] = {SPMM_TILE_SHAPES(SPMM_TILE_ENTRY)};
#undef SPMM_TILE_ENTRY
int tile_shape_count();
// The shape the hybrid and the C ABI use when none is given, for an M-row
// matrix times N columns and a plan of R block-rows per panel whose widest
// union is max_union block-columns.
int default_tile_shape(int R, int max_union, int M, int N);
// Block-rows per panel of the default shape for M rows and N columns.
int default_tile_rows(int M, int N);
// Host part of the plan build: the records, or kUnsupported when a block-row
// is not a run or a panel's runs leave a gap.
Error bsr_tile_plan_from_host(const int* row_ptr, const int* col_idx, int block_rows,
                              int block_cols, int R, std::vector<int>* desc, int* max_union);
// Reads the device BSR's row_ptr and col_idx back (synchronises `stream`) and
// uploads the records.
Error bsr_tile_plan_build(const BSR& d_A, int R, BsrTilePlan* out, hipStream_t stream);
void  bsr_tile_plan_free(BsrTilePlan* p);
// shape < 0: default_tile_shape.  kUnsupported unless N % 8 == 0, B, C and
// the values are 16-byte aligned and the operands fit the buffer records.
Error launch_bsr_tile(const BsrTilePlan& plan, const BSR& d_A, const half* d_B, float* d_C,
                      int N, hipStream_t stream, int shape = -1);

// CSR -> BSR on the device: allocates the BSR's three arrays (release with
// bsr_free_device) and fills them exactly as bsr_from_csr_host would.  The
// CSR's column indices must ascend within each row (repeats adjacent).
Error build_bsr_device(const CSR& d_A, BSR* out, hipStream_t stream);

// Fill-in statistics of a device CSR (the numbers bsr_compute_stats gives
// for bsr_from_csr_host of the same matrix), without building the values.
Error bsr_stats_device(const CSR& d_A, BSR_stats* out, hipStream_t stream);

// Host-in/host-out execution of a hybrid plan (spmm_hybrid_run): *ms is the
// median per-launch kernel time.
Error run_hybrid(const HybridPlan& plan, const CSR& h_A, const float* h_B, float* h_C, int N,
                 int warmup, int iters, float* ms);

// Unified-memory execution (spmm_unified).  *residency: how A, B and C
// reached the device — managed and prefetched, managed and moved on first
// touch (the device could not prefetch), or, on a device without managed
// memory, device allocations filled by explicit copies.
enum UnifiedResidency : int {
    kUnifiedPrefetched   = 1,
    kUnifiedFirstTouch   = 0,
    kUnifiedDeviceCopies = -1,
};
Error run_unified(const CSR& h_A, const float* h_B, float* h_C, int N, int warmup, int iters,
                  float* ms, int* residency);

// Merge-path partition of the row-block engine: part g takes nonzeros
// [nnz*g/P, nnz*(g+1)/P) whatever rows they belong to, so a long row is shared
// by several workgroups.  rows (P+1 device ints, nnz_split_rows) holds the row
// of each part's first nonzero; carry is a device workspace of P x N floats.
// The part where a row starts stores it; later parts holding pieces of it
// write their partial to carry, and a second kernel adds those to C in part
// order (deterministic).
struct SplitPlan {
    const int* rows  = nullptr;
    int        parts = 0;
    float*     carry = nullptr;
};
Error launch_csr_split(const CSR& d_A, const float* d_B, float* d_C, int N, hipStream_t stream,
                       const SplitPlan& plan, const EngineOpts* opts = nullptr);
// The same launch with the carry workspace taken from a file-scope device
// array (noalloc.hip) instead of the caller: allocates nothing, shares one
// workspace per GPU (overlapping calls on a GPU race), and refuses parts x N
// beyond noalloc_scratch_floats() floats.
Error launch_csr_split_noalloc(const CSR& d_A, const int* d_split_rows, int parts,
                               const float* d_B, float* d_C, int N, hipStream_t stream);
long noalloc_scratch_floats();

// B-row halves of the merge-path launch, for a B over one XCD's 4 MiB L2 at
// full width whose half fits (khalf_pays).  A's entries with column < K0 =
// K/2 form half 0, the rest (columns rebased by K0) half 1, each with its own
// merge-path partition.  One launch runs half 0 on XCDs 0-3 into C and half 1
// on XCDs 4-7 into `partial`, all N columns each, so every XCD's L2 holds
// half of B's rows at full width; a second kernel adds, row by row, half 0's
// carries to C and half 1's to the partial, then the partial to C (a fixed
// order: deterministic).  Built once from the host matrix, reused for any B
// of N columns; device memory is owned by the plan (khalf_plan_free).
struct KHalfPlan {
    CSR    half[2]  = {};       // device
    int*   rows[2]  = {};       // merge-path row tables, parts + 1 ints each
    int    parts[2] = {};
    float* carry[2] = {};       // parts x N floats each
    float* partial  = nullptr;  // M x N floats: half 1's rows
    int*   runs     = nullptr;  // M x 4 ints: (first, last) carry part of each row in
                                // half 0, then in half 1; -1 for none
    int    M = 0, K = 0, K0 = 0, N = 0;
};
bool  khalf_pays(int K, int N);
// Host CSR in (columns in [0, K)); kUnsupported unless khalf_pays(K, N) and
// each half holds at least kKHalfMinNnz entries.
constexpr int kKHalfMinNnz = 512;
Error khalf_plan_build(const CSR& h_A, int N, KHalfPlan* out);
void  khalf_plan_free(KHalfPlan* p);
Error launch_csr_khalf(const KHalfPlan& p, const float* d_B, float* d_C, hipStream_t stream);
// For a merge-path partition (row_ptr of M rows, nnz entries, split_rows of
// parts + 1): first[r] / last[r] = the first and last part that continues row
// r (its first nonzero lies in an earlier part), -1 when none.
void khalf_runs(const int* row_ptr, int M, long long nnz, const int* split_rows, int parts,
                int* first, int* last);
// Parts of the merge-path partition for nnz nonzeros, and whether it beats
// the row partition for a matrix whose longest row has max_row_nnz entries.
int split_partition_parts(int nnz);
bool split_pays(int max_row_nnz);

// Whether sub-wave row groups beat the row-block engine for an M-row CSR with
// rows of avg_row entries on average and at most max_row, times a K x N B.
bool row_groups_pay(int M, int N, int K, double avg_row, int max_row);

// Number of workgroups the engine uses for an explicit partition of this CSR.
int default_partition_parts(int num_rows, int nnz);

// The CSR form spmm_hybrid_run's CSR branch runs for a host CSR and a B of N
// columns, decided from its row lengths: sub-wave row groups when
// row_groups_pay, the merge-path partition when split_pays (parts from
// split_partition_parts) -- split over B-row halves when khalf_pays and each
// half holds at least kKHalfMinNnz entries -- the row-block engine
// otherwise.  opts carries the longest row as max_row_hint (and row_groups =
// 1 for row groups).
enum class CsrForm { RowGroups, Engine, Split, KHalf };
struct CsrChoice {
    CsrForm    form    = CsrForm::Engine;
    EngineOpts opts;
    int        parts   = 0;  // merge-path parts (Split only; KHalf plans choose their own)
    int        max_row = 0;
};
CsrChoice choose_csr_form(const CSR& h_A, int N);
const char* csr_form_name(CsrForm f);  // "rowgroups", "engine", "split", "khalf"

}  // namespace engine
}  // namespace spmm
