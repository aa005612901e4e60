// CSR -> BSR (16x16 fp16 blocks) on the device, and the fill-in statistics of
// a device CSR.  The reference builds BSR on the host only (bsr.cu:30-109,
// stats :149-162); this produces the identical BSR (same block order, same
// fp16 rounding, the last of repeated (row, col) entries kept) from a CSR that
// is already in HBM, so the dispatcher can upload the smaller CSR and build
// the BSR next to the kernel.
//
// Work decomposition: one workgroup (4 waves) per block-row of 16 CSR rows.
//   count:  mark the block-columns of the block-row in an LDS bitmap
//           (ds_or), popcount -> blocks of the block-row; also flags column
//           indices out of range or not ascending within a row.
//   scan:   exclusive scan of the counts -> BSR row_ptr (two-level).
//   fill:   rebuild the bitmap, exclusive prefix of word popcounts -> the
//           slot of every block-column; write col_idx in ascending order,
//           zero the block-row's values, then scatter each entry as fp16.
// Rows are walked one wave per row with lanes striding over its entries.
// Within a row, column indices must ascend (repeats adjacent): an entry
// followed by one with the same column is skipped, so the last one is the
// only writer of its element and the result does not depend on scheduling.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "engine.h"
#include "spmm/utils.h"

namespace spmm {
namespace engine {

namespace {

constexpr int kBuildThreads  = 256;   // 4 waves per workgroup
// Bitmap words per block-row; the fill kernel holds the bitmap and its word
// prefix (2 x 4 bytes per word) plus 16 bytes of static LDS within 64 KiB:
// block_cols <= 258048, i.e. K <= 4128768.
constexpr int kMaxBuildWords = 8064;
constexpr int kScanTile      = 2048;  // elements per workgroup of the scan (8 per thread)
constexpr int kFlagRange     = 1;     // a column index outside [0, K)
constexpr int kFlagOrder     = 2;     // column indices descending inside a row

struct BuildArgs {
    const int*   row_ptr;
    const int*   col_idx;
    const float* values;
    int          M;
    int          K;
    int          block_rows;
    int          words;      // ceil(block_cols / 32)
    int*         brp;        // BSR row_ptr (block_rows + 1): counts, then offsets
    int*         flags;      // kFlag* bits, OR-ed over the matrix
    int*         bcol;       // BSR col_idx
    _Float16*    bval;       // BSR values
};

// Exclusive scan of one value per thread over the 256-thread workgroup.
// s_tmp holds 4 ints; every thread of the workgroup must call it.
__device__ int wg_exclusive_scan(int v, int* total, int* s_tmp) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) s_tmp[wave] = x;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kBuildThreads / 64; ++w) {
        const int t = s_tmp[w];
        if (w < wave) before += t;
        all += t;
    }
    __syncthreads();  // s_tmp may be reused by the caller
    *total = all;
    return before + x - v;
}

// Marks the block-columns of block-row br in bitmap; returns kFlag* bits
// found by this thread.
__device__ int mark_block_row(const BuildArgs& a, int br, unsigned* bitmap, bool check) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r0 = br * 16;
    const int r1 = min(a.M, r0 + 16);
    int bad = 0;
    for (int r = r0 + wave; r < r1; r += kBuildThreads / 64) {
        const int p1 = a.row_ptr[r + 1];
        for (int p = a.row_ptr[r] + lane; p < p1; p += 64) {
            const int c = a.col_idx[p];
            if (check) {
                if (static_cast<unsigned>(c) >= static_cast<unsigned>(a.K)) {
                    bad |= kFlagRange;
                    continue;
                }
                if (p + 1 < p1 && a.col_idx[p + 1] < c) bad |= kFlagOrder;
            }
            const int bc = c >> 4;
            atomicOr(&bitmap[bc >> 5], 1u << (bc & 31));
        }
    }
    return bad;
}

__global__ __launch_bounds__(kBuildThreads) void bsr_count_kernel(BuildArgs a) {
    extern __shared__ unsigned s_dyn[];
    __shared__ int s_tmp[kBuildThreads / 64];
    unsigned* bitmap = s_dyn;
    const int br = blockIdx.x;
    for (int w = threadIdx.x; w < a.words; w += kBuildThreads) bitmap[w] = 0u;
    __syncthreads();
    const int bad = mark_block_row(a, br, bitmap, true);
    if (bad != 0) atomicOr(a.flags, bad);
    __syncthreads();
    int cnt = 0;
    for (int w = threadIdx.x; w < a.words; w += kBuildThreads) cnt += __popc(bitmap[w]);
    int total;
    (void)wg_exclusive_scan(cnt, &total, s_tmp);
    if (threadIdx.x == 0) a.brp[br] = total;
}

// Level 1: each workgroup scans kScanTile elements of data[0..n) in place
// (exclusive) and records its tile total.
__global__ __launch_bounds__(kBuildThreads) void scan_tiles_kernel(int* data, int n, int* tile_sums) {
    __shared__ int s_tmp[kBuildThreads / 64];
    const long base = static_cast<long>(blockIdx.x) * kScanTile + threadIdx.x * 8;
    int v[8];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = base + i < n ? data[base + i] : 0;
        sum += v[i];
    }
    int total;
    int run = wg_exclusive_scan(sum, &total, s_tmp);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (base + i < n) data[base + i] = run;
        run += v[i];
    }
    if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

// Level 2 (one workgroup): exclusive scan of the tile totals in place; the
// grand total goes to data[n].
__global__ __launch_bounds__(kBuildThreads) void scan_tile_sums_kernel(int* tile_sums, int tiles,
                                                                     int* data, int n) {
    __shared__ int s_tmp[kBuildThreads / 64];
    const int base = threadIdx.x * 8;
    int v[8];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = base + i < tiles ? tile_sums[base + i] : 0;
        sum += v[i];
    }
    int total;
    int run = wg_exclusive_scan(sum, &total, s_tmp);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (base + i < tiles) tile_sums[base + i] = run;
        run += v[i];
    }
    if (threadIdx.x == 0) data[n] = total;
}

// Level 3: add each tile's offset.
__global__ __launch_bounds__(kBuildThreads) void scan_add_kernel(int* data, int n,
                                                               const int* tile_sums) {
    const int off = tile_sums[blockIdx.x];
    const long base = static_cast<long>(blockIdx.x) * kScanTile;
    for (int i = threadIdx.x; i < kScanTile; i += kBuildThreads) {
        if (base + i < n) data[base + i] += off;
    }
}

__global__ __launch_bounds__(kBuildThreads) void bsr_fill_kernel(BuildArgs a) {
    extern __shared__ unsigned s_dyn[];
    __shared__ int s_tmp[kBuildThreads / 64];
    unsigned* bitmap = s_dyn;
    int* prefix = reinterpret_cast<int*>(s_dyn + a.words);
    const int br = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    for (int w = threadIdx.x; w < a.words; w += kBuildThreads) bitmap[w] = 0u;
    __syncthreads();
    (void)mark_block_row(a, br, bitmap, false);
    __syncthreads();

    // Exclusive prefix of popcounts: thread t owns words [t*per, (t+1)*per).
    const int per = (a.words + kBuildThreads - 1) / kBuildThreads;
    const int w0 = min(a.words, threadIdx.x * per);
    const int w1 = min(a.words, w0 + per);
    int mine = 0;
    for (int w = w0; w < w1; ++w) mine += __popc(bitmap[w]);
    int total;
    int run = wg_exclusive_scan(mine, &total, s_tmp);
    for (int w = w0; w < w1; ++w) {
        prefix[w] = run;
        run += __popc(bitmap[w]);
    }
    __syncthreads();

    const int first = a.brp[br];  // slot 0 of this block-row
    // Block-columns in ascending order.
    for (int w = threadIdx.x; w < a.words; w += kBuildThreads) {
        unsigned bits = bitmap[w];
        int pos = first + prefix[w];
        while (bits != 0u) {
            const int b = __builtin_ctz(bits);
            a.bcol[pos++] = w * 32 + b;
            bits &= bits - 1u;
        }
    }
    // Zero the block-row's values (16-byte stores; every block is 512 bytes).
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    i32x4* vz = reinterpret_cast<i32x4*>(a.bval + static_cast<size_t>(first) * 256);
    const long chunks = static_cast<long>(total) * 256 / 8;
    for (long i = threadIdx.x; i < chunks; i += kBuildThreads) vz[i] = i32x4(0);
    __syncthreads();  // zeros are stored before any entry lands on them

    const int r0 = br * 16;
    const int r1 = min(a.M, r0 + 16);
    for (int r = r0 + wave; r < r1; r += kBuildThreads / 64) {
        const int p1 = a.row_ptr[r + 1];
        for (int p = a.row_ptr[r] + lane; p < p1; p += 64) {
            const int c = a.col_idx[p];
            if (p + 1 < p1 && a.col_idx[p + 1] == c) continue;  // a later repeat wins
            const int bc = c >> 4;
            const int w = bc >> 5;
            const int slot = prefix[w] + __popc(bitmap[w] & ((1u << (bc & 31)) - 1u));
            a.bval[static_cast<size_t>(first + slot) * 256 + (r - r0) * 16 + (c & 15)] =
                static_cast<_Float16>(a.values[p]);
        }
    }
}

Error fail(int status, std::string msg) { return Error{status, std::move(msg)}; }

Error from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return Error{};
    return fail(kHipError, std::string(what) + ": " + hipGetErrorString(e));
}

Error check_build_args(const CSR& d_A) {
    if (d_A.num_rows < 0 || d_A.num_cols < 0 || d_A.nnz < 0) {
        return fail(kInvalid, "negative matrix dimension");
    }
    if (d_A.num_rows > 0 && d_A.row_ptr == nullptr) return fail(kInvalid, "null device pointer");
    if (d_A.nnz > 0 && (d_A.col_idx == nullptr || d_A.values == nullptr)) {
        return fail(kInvalid, "null device pointer");
    }
    const int block_cols = (d_A.num_cols + 15) / 16;
    if ((block_cols + 31) / 32 > kMaxBuildWords) {
        return fail(kUnsupported, "device BSR build supports num_cols <= " +
                                      std::to_string(kMaxBuildWords * 32 * 16));
    }
    const int block_rows = (d_A.num_rows + 15) / 16;
    if ((block_rows + kScanTile - 1) / kScanTile > kScanTile) {
        return fail(kUnsupported, "device BSR build supports num_rows <= " +
                                      std::to_string(16L * kScanTile * kScanTile));
    }
    return Error{};
}

// Counts blocks per block-row into d_brp and scans them into the BSR row_ptr.
// On return h_info = {num_blocks, flags}.
Error count_and_scan(const CSR& d_A, int* d_brp, int* d_work, int h_info[2], hipStream_t stream) {
    const int block_rows = (d_A.num_rows + 15) / 16;
    const int words = ((d_A.num_cols + 15) / 16 + 31) / 32;
    const int tiles = (block_rows + kScanTile - 1) / kScanTile;
    int* d_flags = d_work;
    int* d_tiles = d_work + 1;
    hipError_t e = hipMemsetAsync(d_flags, 0, sizeof(int), stream);
    if (e != hipSuccess) return from_hip(e, "device BSR build");
    BuildArgs a{d_A.row_ptr, d_A.col_idx, d_A.values, d_A.num_rows, d_A.num_cols,
                block_rows, words, d_brp, d_flags, nullptr, nullptr};
    const size_t lds = sizeof(unsigned) * std::max(words, 1);
    hipLaunchKernelGGL(bsr_count_kernel, dim3(block_rows), dim3(kBuildThreads), lds, stream, a);
    hipLaunchKernelGGL(scan_tiles_kernel, dim3(tiles), dim3(kBuildThreads), 0, stream, d_brp,
                       block_rows, d_tiles);
    hipLaunchKernelGGL(scan_tile_sums_kernel, dim3(1), dim3(kBuildThreads), 0, stream, d_tiles,
                       tiles, d_brp, block_rows);
    hipLaunchKernelGGL(scan_add_kernel, dim3(tiles), dim3(kBuildThreads), 0, stream, d_brp,
                       block_rows, d_tiles);
    e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e, "device BSR build launch");
    e = hipMemcpyAsync(&h_info[0], d_brp + block_rows, sizeof(int), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) {
        e = hipMemcpyAsync(&h_info[1], d_flags, sizeof(int), hipMemcpyDeviceToHost, stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return from_hip(e, "device BSR build");
    if (h_info[1] & kFlagRange) return fail(kInvalid, "column index out of range");
    if (h_info[1] & kFlagOrder) {
        return fail(kUnsupported,
                    "device BSR build needs column indices ascending within each row");
    }
    return Error{};
}

}  // namespace

Error build_bsr_device(const CSR& d_A, BSR* out, hipStream_t stream) {
    Error err = check_build_args(d_A);
    if (err.status != kOk) return err;
    BSR d;
    d.num_rows   = d_A.num_rows;
    d.num_cols   = d_A.num_cols;
    d.block_rows = (d_A.num_rows + 15) / 16;
    d.block_cols = (d_A.num_cols + 15) / 16;
    d.nnz        = d_A.nnz;
    const int tiles = (d.block_rows + kScanTile - 1) / kScanTile;
    int* d_work = nullptr;
    hipError_t e = hipMalloc(&d.row_ptr, sizeof(int) * (static_cast<size_t>(d.block_rows) + 1));
    if (e == hipSuccess) e = hipMalloc(&d_work, sizeof(int) * (static_cast<size_t>(tiles) + 2));
    if (e != hipSuccess) {
        (void)hipFree(d.row_ptr);
        return from_hip(e, "device BSR build allocation");
    }
    auto release = [&] {
        (void)hipFree(d_work);
        (void)hipFree(d.row_ptr);
        (void)hipFree(d.col_idx);
        (void)hipFree(d.values);
    };
    int info[2] = {0, 0};
    if (d.block_rows == 0) {
        e = hipMemsetAsync(d.row_ptr, 0, sizeof(int), stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) {
            release();
            return from_hip(e, "device BSR build");
        }
    } else {
        err = count_and_scan(d_A, d.row_ptr, d_work, info, stream);
        if (err.status != kOk) {
            release();
            return err;
        }
    }
    d.num_blocks = info[0];
    const size_t nb = static_cast<size_t>(d.num_blocks);
    e = hipMalloc(&d.col_idx, sizeof(int) * std::max<size_t>(nb, 1));
    if (e == hipSuccess) e = hipMalloc(&d.values, sizeof(half) * std::max<size_t>(nb * 256, 1));
    if (e != hipSuccess) {
        release();
        return from_hip(e, "device BSR build allocation");
    }
    if (d.block_rows > 0) {
        const int words = (d.block_cols + 31) / 32;
        BuildArgs a{d_A.row_ptr, d_A.col_idx, d_A.values, d_A.num_rows, d_A.num_cols,
                    d.block_rows, words, d.row_ptr, d_work, d.col_idx,
                    reinterpret_cast<_Float16*>(d.values)};
        const size_t lds = 2 * sizeof(unsigned) * std::max(words, 1);
        hipLaunchKernelGGL(bsr_fill_kernel, dim3(d.block_rows), dim3(kBuildThreads), lds, stream,
                           a);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) {
            release();
            return from_hip(e, "device BSR fill");
        }
    }
    (void)hipFree(d_work);
    *out = d;
    return Error{};
}

Error bsr_stats_device(const CSR& d_A, BSR_stats* out, hipStream_t stream) {
    Error err = check_build_args(d_A);
    if (err.status != kOk) return err;
    const int block_rows = (d_A.num_rows + 15) / 16;
    const int block_cols = (d_A.num_cols + 15) / 16;
    int info[2] = {0, 0};
    if (block_rows > 0) {
        const int tiles = (block_rows + kScanTile - 1) / kScanTile;
        int* d_brp = nullptr;
        int* d_work = nullptr;
        hipError_t e = hipMalloc(&d_brp, sizeof(int) * (static_cast<size_t>(block_rows) + 1));
        if (e == hipSuccess) e = hipMalloc(&d_work, sizeof(int) * (static_cast<size_t>(tiles) + 2));
        if (e != hipSuccess) {
            (void)hipFree(d_brp);
            return from_hip(e, "device BSR stats allocation");
        }
        err = count_and_scan(d_A, d_brp, d_work, info, stream);
        (void)hipFree(d_brp);
        (void)hipFree(d_work);
        if (err.status != kOk) return err;
    }
    BSR_stats s;
    s.num_blocks      = info[0];
    s.stored_elements = static_cast<long>(info[0]) * 256;
    s.original_nnz    = d_A.nnz;
    s.fill_in_ratio   = d_A.nnz > 0 ? static_cast<double>(s.stored_elements) / d_A.nnz : 0.0;
    const long all    = static_cast<long>(block_rows) * block_cols;
    s.block_density   = all > 0 ? static_cast<double>(info[0]) / all : 0.0;
    *out = s;
    return Error{};
}

}  // namespace engine
}  // namespace spmm
