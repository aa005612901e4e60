// CSR x dense kernels for gfx950 (wave64, 256 CUs in 8 XCDs).
//
//   csr_lane_per_output   role of spmm_baseline   (spmm_baseline.cu:11-25)
//   csr_wave_per_row      role of spmm_memopt/_v2 (spmm_memopt.cu:11-38)
//   csr_rowblock          role of spmm_tiled*     (spmm_tiled_v3.cu:21-104), the engine
//
// All three accumulate in fp32 with fused multiply-adds.  C is fully written
// (rows without nonzeros get zeros), so callers never clear it.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "engine.h"
#include "spmm/utils.h"

typedef float spmm_f32x2 __attribute__((ext_vector_type(2)));
typedef float spmm_f32x4 __attribute__((ext_vector_type(4)));

// Structured buffer loads (LLVM's AMDGPU intrinsics; index = record, offset =
// byte offset inside the record).  The intrinsic names are fixed by LLVM.
__device__ spmm_f32x4 sbuf_load_x4(__amdgpu_buffer_rsrc_t rsrc, int index, int offset,
                                   int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4f32");
__device__ spmm_f32x2 sbuf_load_x2(__amdgpu_buffer_rsrc_t rsrc, int index, int offset,
                                   int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v2f32");
__device__ float sbuf_load_x1(__amdgpu_buffer_rsrc_t rsrc, int index, int offset, int soffset,
                              int aux) __asm("llvm.amdgcn.struct.ptr.buffer.load.f32");

namespace spmm {
namespace engine {

namespace {

constexpr int kWave = 64;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int VEC> struct Vec;
template <> struct Vec<1> { using T = float; };
template <> struct Vec<2> { using T = f32x2; };
template <> struct Vec<4> { using T = f32x4; };

template <int VEC>
__device__ __forceinline__ typename Vec<VEC>::T vzero() {
    return typename Vec<VEC>::T(0.0f);
}

// ---------------------------------------------------------------------------
// Role: spmm_baseline.  One lane per C(i, j); a wave spans 64 columns of one
// row, so the row's (col, value) reads are wave-uniform and the B reads are
// one coalesced 256-byte segment per nonzero.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void csr_lane_per_output(
    int M, int N, const int* __restrict__ row_ptr, const int* __restrict__ col_idx,
    const float* __restrict__ vals, const float* __restrict__ B, float* __restrict__ C) {
    const int j = blockIdx.x * kWave + threadIdx.x;
    const int i = blockIdx.y * 4 + threadIdx.y;
    if (i >= M || j >= N) return;
    const int p0 = row_ptr[i];
    const int p1 = row_ptr[i + 1];
    float sum = 0.f;
    for (int p = p0; p < p1; ++p) {
        sum = __builtin_fmaf(vals[p], B[static_cast<size_t>(col_idx[p]) * N + j], sum);
    }
    C[static_cast<size_t>(i) * N + j] = sum;
}

// ---------------------------------------------------------------------------
// Role: spmm_memopt / spmm_memopt_v2.  One wave per row; lane l owns columns
// c0 + l + 64*t (t < CPL) of each column pass, every nonzero is read once per
// pass with a wave-uniform (scalar) load.
// ---------------------------------------------------------------------------
template <int CPL, int MIN_WAVES_PER_EU>
__global__ __launch_bounds__(256, MIN_WAVES_PER_EU) void csr_wave_per_row(
    int M, int N, const int* __restrict__ row_ptr, const int* __restrict__ col_idx,
    const float* __restrict__ vals, const float* __restrict__ B, float* __restrict__ C) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & (kWave - 1);
    if (row >= M) return;
    const int p0 = row_ptr[row];
    const int p1 = row_ptr[row + 1];
    float* crow = C + static_cast<size_t>(row) * N;
    for (int c0 = 0; c0 < N; c0 += kWave * CPL) {
        float acc[CPL];
#pragma unroll
        for (int t = 0; t < CPL; ++t) acc[t] = 0.f;
        for (int p = p0; p < p1; ++p) {
            const float v = vals[p];
            const float* brow = B + static_cast<size_t>(col_idx[p]) * N;
#pragma unroll
            for (int t = 0; t < CPL; ++t) {
                const int c = c0 + lane + kWave * t;
                if (c < N) acc[t] = __builtin_fmaf(v, brow[c], acc[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            const int c = c0 + lane + kWave * t;
            if (c < N) crow[c] = acc[t];
        }
    }
}

// ---------------------------------------------------------------------------
// The engine (role: spmm_tiled / _v2 / _v3 / _v4).
//
// Partition.  Workgroup g owns rows [r_begin, r_end): either g*R .. g*R+R
// (implicit, R chosen from the average row length) or bounds[g] .. bounds[g+1]
// (an explicit nnz-balanced partition).  Inside the workgroup the nonzeros of
// those rows are cut into WAVES equal contiguous ranges, one per wave, so a
// long row is shared by several waves and many short rows by one wave.
// Merge-path mode (split_rows) cuts at the workgroup level too: workgroup g
// takes nonzeros [nnz*g/P, nnz*(g+1)/P) whatever rows they belong to; a row
// that began in an earlier workgroup is summed into carry[g] instead of C, and
// csr_split_fixup adds the carries to C in part order afterwards.
//
// Lane groups.  A wave is split into G groups of 64/G lanes; each group covers
// one column tile of COLS = (64/G) * VEC columns with VEC-float (up to 16-byte)
// loads, and the groups take interleaved entries of the wave's range (group h
// takes entries h, h+G, h+2G, ...).  One load instruction therefore fetches G
// different B row segments: for N = 128 fp32, G = 2 and each half-wave reads
// one 512-byte row with dwordx4 loads.
//
// Per wave.  The wave copies (col, value) pairs of its range into its own LDS
// window (kWCap entries, all loads issued at once); every lane then reads the
// entry of its group with one broadcast ds_read_b64 and gathers its B segment
// with a bounds-checked buffer load (one record per B row, so the row index is
// the load's index operand and needs no address arithmetic).  The range is
// walked in steps of U*G entries with the next step's loads in flight while
// the current step is accumulated.  A scalar test per step sends only the
// steps that cross a row end to the slow path, so row bookkeeping costs per
// row, not per entry (measured on MI355X: per-entry scalar tests made the
// kernel issue-bound on the shared scalar unit).  At a row end the groups'
// tiles are summed with cross-lane shuffles and the row is flushed:
//   - a row that lies wholly inside the wave's range is stored to C;
//   - the first row of a range that started in an earlier wave goes to an LDS
//     slot (s_part[wave]);
//   - the last row of a range that continues in a later wave stays in the
//     registers of its owner, which after a barrier adds the LDS slots of the
//     following waves in wave order and stores it.
// The sum order is fixed by the partition and the launch shape, so results
// are deterministic run to run.
//
// Rows of the workgroup without nonzeros are zero-filled up front.  Row
// pointers are staged in LDS in windows of kRpCap rows.
// ---------------------------------------------------------------------------
struct RowblockArgs {
    const int*   row_ptr;
    const int*   col_idx;
    const float* vals;
    const float* B;
    float*       C;
    const int*   bounds;  // nullable
    int          M;
    int          N;
    int          K;            // rows of B (records of the B buffer)
    int          rows_per_block;
    int          nblocks;      // row blocks (workgroups of one column slice)
    int          slices;       // column slices: 1, 2, 4 or 8
    int          slice_cols;   // columns per slice (a multiple of VEC)
    // Merge-path partition (nullable split_rows): part g = nonzeros
    // [nnz*g/nblocks, nnz*(g+1)/nblocks); split_rows[g] is the row holding the
    // first of them (split_rows[0] = 0, split_rows[nblocks] = M); carry is a
    // nblocks x N workspace for the partial of a part's first row when that
    // row began in an earlier part.
    const int*   split_rows;
    float*       carry;
    long long    nnz;
    // B-row halves (merge-path only): workgroups on XCDs 4-7 take this second
    // descriptor -- the entries of A whose columns lie in B's upper rows, with
    // rebased columns, those B rows, their own output and merge-path table --
    // and XCDs 0-3 the first, so each XCD's L2 holds half of B at full width.
    int          halves = 0;
    const int*   row_ptr1 = nullptr;
    const int*   col_idx1 = nullptr;
    const float* vals1 = nullptr;
    const float* B1 = nullptr;
    float*       C1 = nullptr;
    int          K1 = 0;
    const int*   split_rows1 = nullptr;
    float*       carry1 = nullptr;
    long long    nnz1 = 0;
    int          nblocks1 = 0;
};

constexpr int kRpCap = 1024;  // row pointers staged per window
constexpr int kWCap  = 256;   // (col, value) entries a wave stages at a time

// Third dword of a gfx9 buffer resource: 32-bit data format, no swizzle.
constexpr int kBufWord3 = 0x00020000;

// VEC floats of B row k at byte offset colb: a structured-buffer load (record
// k of N*4 bytes; rows outside [0, K) read as zeros), or a plain 64-bit
// address when B is too large for the buffer form.
template <int VEC, bool SBUF>
__device__ __forceinline__ typename Vec<VEC>::T load_b(__amdgpu_buffer_rsrc_t rsrc,
                                                       const float* bcol, int k, int colb,
                                                       int N) {
    if constexpr (SBUF) {
        if constexpr (VEC == 4) return sbuf_load_x4(rsrc, k, colb, 0, 0);
        else if constexpr (VEC == 2) return sbuf_load_x2(rsrc, k, colb, 0, 0);
        else return sbuf_load_x1(rsrc, k, colb, 0, 0);
    } else {
        return *reinterpret_cast<const typename Vec<VEC>::T*>(bcol + static_cast<size_t>(k) * N);
    }
}

template <int VEC>
__device__ __forceinline__ void store_vec(float* p, typename Vec<VEC>::T v) {
    __builtin_nontemporal_store(v, reinterpret_cast<typename Vec<VEC>::T*>(p));
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m); }

// Sum of the G groups' tiles, returned to every lane.
template <int VEC, int G>
__device__ __forceinline__ typename Vec<VEC>::T reduce_groups(typename Vec<VEC>::T v) {
    if constexpr (G == 1) {
        return v;
    } else {
        using VT = typename Vec<VEC>::T;
#pragma unroll
        for (int m = kWave / G; m < kWave; m <<= 1) {
            VT o;
            if constexpr (VEC == 1) {
                o = shfl_xor_f(v, m);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) o[e] = shfl_xor_f(v[e], m);
            }
            v += o;
        }
        return v;
    }
}

// Orders a wave's LDS writes before its own lanes' reads of them.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int VEC, int G, int WAVES, int U, bool SBUF>
__global__ __launch_bounds__(WAVES * 64) void csr_rowblock(RowblockArgs a) {
    using VT = typename Vec<VEC>::T;
    constexpr int LPG  = kWave / G;   // lanes per group
    constexpr int COLS = LPG * VEC;   // columns per pass
    constexpr int STEP = U * G;       // entries per step
    static_assert(kWave % STEP == 0 && kWCap % kWave == 0, "U * G must divide the wave size");

    __shared__ int  s_rp[kRpCap + 1];
    __shared__ VT   s_part[WAVES][LPG];
    __shared__ int  s_first[WAVES];
    __shared__ int2 s_kv[WAVES][kWCap + STEP];

    const int lane  = threadIdx.x & (kWave - 1);
    const int wave  = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp   = lane / LPG;
    const int glane = lane % LPG;
    const int N     = a.N;

    // Column slices are tied to XCDs: workgroups are dispatched round-robin
    // over the 8 XCDs, so workgroup g runs on XCD g % 8.  With S slices, XCDs
    // s*8/S .. (s+1)*8/S - 1 compute columns [s*SC, (s+1)*SC) of every row
    // block, so each XCD's L2 holds only 1/S of B.  With B-row halves, XCDs
    // 0-3 work through the parts of the first descriptor and XCDs 4-7 through
    // those of the second (all columns each).
    int rb = blockIdx.x, slice = 0;
    if (a.halves) {
        const int x = blockIdx.x & 7;
        rb = (blockIdx.x >> 3) * 4 + (x & 3);
        if (x >= 4) {
            a.row_ptr    = a.row_ptr1;
            a.col_idx    = a.col_idx1;
            a.vals       = a.vals1;
            a.B          = a.B1;
            a.C          = a.C1;
            a.K          = a.K1;
            a.split_rows = a.split_rows1;
            a.carry      = a.carry1;
            a.nnz        = a.nnz1;
            a.nblocks    = a.nblocks1;
        }
    } else if (a.slices > 1) {
        const int per = 8 / a.slices;  // XCDs per slice
        const int x   = blockIdx.x & 7;
        rb    = (blockIdx.x >> 3) * per + x % per;
        slice = x / per;
    }
    if (rb >= a.nblocks) return;  // whole workgroup, before any barrier
    const int cbeg = slice * a.slice_cols;
    const int cend = min(N, cbeg + a.slice_cols);

    int r_begin, r_end, zero_end;
    const bool split = a.split_rows != nullptr;
    long long nz_lo = 0, nz_hi = 0;
    int wg_head = -1;  // first row, when it began in an earlier part (merge-path only)
    if (split) {
        nz_lo    = a.nnz * rb / a.nblocks;
        nz_hi    = a.nnz * (rb + 1) / a.nblocks;
        r_begin  = a.split_rows[rb];
        zero_end = a.split_rows[rb + 1];          // empty rows [r_begin, zero_end) are ours
        r_end    = min(a.M, zero_end + 1);         // + the row our last nonzeros start
        if (nz_lo < nz_hi && r_begin < a.M && a.row_ptr[r_begin] < nz_lo) wg_head = r_begin;
    } else if (a.bounds != nullptr) {
        r_begin  = a.bounds[rb];
        r_end    = a.bounds[rb + 1];
        zero_end = r_end;
    } else {
        r_begin  = rb * a.rows_per_block;
        r_end    = min(a.M, r_begin + a.rows_per_block);
        zero_end = r_end;
    }

    __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a.B), static_cast<short>(SBUF ? N * 4 : 0), SBUF ? a.K : 0, kBufWord3);
    // Entries past a window's end read by the masked lanes of its last step.
    for (int i = lane; i < STEP; i += kWave) s_kv[wave][kWCap + i] = make_int2(0, 0);

    // Copies entries [lo, hi) (hi - lo <= kWCap) into the wave's LDS window;
    // the rest of the window holds (0, 0).  All loads are issued before the
    // first LDS write.
    auto stage = [&](int lo, int hi) {
        constexpr int NL = kWCap / kWave;
        int   kk[NL];
        float vx[NL];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = min(lo + i * kWave + lane, hi - 1);
            kk[i] = a.col_idx[e];
            vx[i] = a.vals[e];
        }
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const bool in = lo + i * kWave + lane < hi;
            s_kv[wave][i * kWave + lane] =
                make_int2(in ? kk[i] : 0, in ? __builtin_bit_cast(int, vx[i]) : 0);
        }
        wave_lds_sync();
    };

    for (int w0 = r_begin; w0 < r_end; w0 += kRpCap) {
        const int nr = min(r_end - w0, kRpCap);
        __syncthreads();  // the previous window is no longer read
        for (int i = threadIdx.x; i <= nr; i += WAVES * kWave) s_rp[i] = a.row_ptr[w0 + i];
        __syncthreads();

        // Zero-fill the rows of this window that hold no nonzeros.
        for (int base = wave * kWave; base < nr; base += WAVES * kWave) {
            const int i = base + lane;
            uint64_t empty = __ballot(i < nr && w0 + i < zero_end && s_rp[i] == s_rp[i + 1]);
            while (empty) {
                const int b = __builtin_ctzll(empty);
                empty &= empty - 1;
                float* crow = a.C + static_cast<size_t>(w0 + base + b) * N;
                for (int c = cbeg + lane * VEC; c < cend; c += kWave * VEC) {
                    store_vec<VEC>(crow + c, vzero<VEC>());
                }
            }
        }

        int nz0 = s_rp[0];
        int nz_end = s_rp[nr];
        if (split) {
            nz0    = static_cast<int>(max(static_cast<long long>(nz0), nz_lo));
            nz_end = static_cast<int>(min(static_cast<long long>(nz_end), nz_hi));
        }
        const int total = nz_end - nz0;
        if (total <= 0) continue;  // uniform across the workgroup
        const int pa = nz0 + static_cast<int>((static_cast<long long>(total) * wave) / WAVES);
        const int pb = nz0 + static_cast<int>((static_cast<long long>(total) * (wave + 1)) / WAVES);

        // First local row: the last i in [0, nr) with s_rp[i] <= pa.
        int first = 0;
        {
            int lo = 0, hi = nr - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_rp[mid] <= pa) lo = mid; else hi = mid - 1;
            }
            first = lo;
        }

        // A range that fits one window is staged once for all column passes.
        const bool one_window = pb - pa <= kWCap;
        if (one_window && pa < pb) stage(pa, pb);

        for (int c0 = cbeg; c0 < cend; c0 += COLS) {
            const int  col    = c0 + glane * VEC;
            const bool col_ok = col < cend;
            const int  col_ld = col_ok ? col : 0;  // loads stay in bounds; never stored
            const bool writer = grp == 0 && col_ok;
            const float* bcol = a.B + col_ld;
            if (lane == 0) s_first[wave] = (pa < pb) ? -1 : -2;

            int owner_row = -1;  // local row this wave finishes after the barrier
            VT acc = vzero<VEC>();
            if (pa < pb) {
                int  row     = first;
                int  row_end = s_rp[row + 1];
                bool head    = s_rp[row] < pa;  // row began in an earlier wave

                auto flush = [&]() {
                    const VT t = reduce_groups<VEC, G>(acc);
                    if (head) {
                        if (grp == 0) s_part[wave][glane] = t;
                        if (lane == 0) s_first[wave] = row;
                        head = false;
                    } else if (writer) {
                        store_vec<VEC>(a.C + static_cast<size_t>(w0 + row) * N + col, t);
                    }
                    acc = vzero<VEC>();
                };

                for (int win = pa; win < pb; win += kWCap) {
                    const int win_end = min(pb, win + kWCap);
                    if (!one_window) stage(win, win_end);

                    VT    bA[U], bB[U];
                    float vA[U], vB[U];
                    // Loads of the step starting at entry q.
                    auto issue = [&](VT (&bv)[U], float (&vv)[U], int q) {
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const int2 kv = s_kv[wave][q - win + u * G + grp];
                            vv[u] = __builtin_bit_cast(float, kv.y);
                            bv[u] = load_b<VEC, SBUF>(rsrc, bcol, kv.x, col_ld * 4, N);
                        }
                    };
                    // Accumulates the step starting at entry q.
                    auto consume = [&](VT (&bv)[U], float (&vv)[U], int q) {
                        if (q + STEP <= row_end && q + STEP <= win_end) {
#pragma unroll
                            for (int u = 0; u < U; ++u) acc = vv[u] * bv[u] + acc;
                        } else {
#pragma unroll
                            for (int u = 0; u < U; ++u) {
#pragma unroll
                                for (int h = 0; h < G; ++h) {
                                    const int P = q + u * G + h;
                                    if (P < win_end) {
                                        if (P >= row_end) {
                                            flush();
                                            // bounded by the window even for a malformed row_ptr
                                            do {
                                                ++row;
                                                row_end = s_rp[row + 1];
                                            } while (row_end <= P && row < nr - 1);
                                        }
                                        if (grp == h) acc = vv[u] * bv[u] + acc;
                                    }
                                }
                            }
                        }
                    };
                    issue(bA, vA, win);
                    for (int q = win; q < win_end; q += 2 * STEP) {
                        if (q + STEP < win_end) issue(bB, vB, q + STEP);
                        consume(bA, vA, q);
                        if (q + STEP >= win_end) break;
                        if (q + 2 * STEP < win_end) issue(bA, vA, q + 2 * STEP);
                        consume(bB, vB, q + STEP);
                    }
                }
                // The row being accumulated when the range ends.
                acc = reduce_groups<VEC, G>(acc);
                if (row_end == pb && !head) {
                    if (writer) store_vec<VEC>(a.C + static_cast<size_t>(w0 + row) * N + col, acc);
                } else if (head) {
                    if (grp == 0) s_part[wave][glane] = acc;
                    if (lane == 0) s_first[wave] = row;
                } else {
                    owner_row = row;
                }
            }
            __syncthreads();
            if (owner_row >= 0) {
                for (int w = wave + 1; w < WAVES; ++w) {
                    const int f = s_first[w];
                    if (f == -2) continue;
                    if (f != owner_row) break;
                    acc += s_part[w][glane];
                }
                if (writer) store_vec<VEC>(a.C + static_cast<size_t>(w0 + owner_row) * N + col, acc);
            }
            if (wg_head >= 0 && w0 == r_begin && wave == 0) {
                // The part's first row began in an earlier part: the waves that
                // hold pieces of it (local row 0, leading waves) go to the carry.
                VT sum = vzero<VEC>();
                for (int w = 0; w < WAVES; ++w) {
                    const int f = s_first[w];
                    if (f == -2) continue;
                    if (f != 0) break;
                    sum += s_part[w][glane];
                }
                if (writer) store_vec<VEC>(a.carry + static_cast<size_t>(rb) * N + col, sum);
            }
            __syncthreads();  // s_part / s_first are rewritten by the next column pass
        }
    }
}

// Merge-path fix-up: row r that continues into parts g0+1 .. g1 was stored by
// the part where it starts; the first continuation part adds the carries of
// parts g0+1 .. g1 in part order (deterministic) to C[r].  Every part holds at
// least one nonzero (the launcher requires parts <= nnz), so part q > g
// continues row r exactly when split_rows[q] == r.  One wave per part, and
// the loads are arranged in three dependent rounds: the part's row; that
// row's first nonzero together with the rows of the next 64 parts (a ballot
// finds where the run ends); the carries together with C.
constexpr int kFixupCols = 4;  // columns per lane in flight

__global__ __launch_bounds__(64) void csr_split_fixup(const int* __restrict__ row_ptr,
                                                      const int* __restrict__ split_rows,
                                                      const float* __restrict__ carry,
                                                      float* __restrict__ C, int M, int N,
                                                      long long nnz, int parts) {
    const int g    = blockIdx.x;
    const int lane = threadIdx.x;
    const long long lo = nnz * g / parts;
    const long long hi = nnz * (g + 1) / parts;
    const int r  = split_rows[g];
    const int rp = g > 0 ? split_rows[g - 1] : -1;
    if (!(lo < hi && r >= 0 && r < M)) return;
    int base = g + 1;
    int q    = base + lane;
    int w    = q < parts ? split_rows[q] : -1;  // issued before row_ptr[r] returns
    const int rs = row_ptr[r];
    if (rs >= lo) return;  // part g starts row r and stored it
    // part g continues row r; the previous part also continues it when it
    // holds row r and r began before that part's first nonzero
    if (g > 0 && rp == r && rs < nnz * (g - 1) / parts) return;
    int last;
    for (;;) {
        const unsigned long long stop = __ballot(!(q < parts && w == r));
        if (stop != 0ull) {
            last = base + __ffsll(static_cast<long long>(stop)) - 2;
            break;
        }
        base += 64;
        q = base + lane;
        w = q < parts ? split_rows[q] : -1;
    }
    float* crow = C + static_cast<size_t>(r) * N;
    for (int c0 = 0; c0 < N; c0 += 64 * kFixupCols) {
        float cv[kFixupCols], s[kFixupCols];
#pragma unroll
        for (int j = 0; j < kFixupCols; ++j) {
            const int c = c0 + lane + 64 * j;
            cv[j] = c < N ? crow[c] : 0.f;
            s[j]  = 0.f;
        }
        for (int p = g; p <= last; ++p) {
            const float* cr = carry + static_cast<size_t>(p) * N;
#pragma unroll
            for (int j = 0; j < kFixupCols; ++j) {
                const int c = c0 + lane + 64 * j;
                if (c < N) s[j] += cr[c];
            }
        }
#pragma unroll
        for (int j = 0; j < kFixupCols; ++j) {
            const int c = c0 + lane + 64 * j;
            if (c < N) crow[c] = cv[j] + s[j];
        }
    }
}

// Fix-up of the B-row halves: C = (C + carries of half 0) + (partial +
// carries of half 1), row by row, each sum of carries in part order --
// the same order on every launch.  runs[r] = (first, last) continuation part
// of row r in half 0, then in half 1, -1 for none.  One 16-byte chunk of C and
// of the partial per thread (N % 4 == 0); both are read once, so the loads
// stream (measured on c5: 61.4 -> 60.2 us per launch against cached loads
// two chunks per thread).
__global__ __launch_bounds__(256) void csr_khalf_fixup(float* __restrict__ C,
                                                       const float* __restrict__ partial,
                                                       const float* __restrict__ carry0,
                                                       const float* __restrict__ carry1,
                                                       const int4* __restrict__ runs, int N,
                                                       long long chunks) {
    const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= chunks) return;
    const int4 ru = runs[t * 4 / N];
    f32x4 cv = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(C) + t);
    f32x4 pv = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(partial) + t);
    const int c = static_cast<int>(t * 4 % N);
    if (ru.x >= 0) {
        f32x4 s = f32x4(0.f);
        for (int p = ru.x; p <= ru.y; ++p) {
            s += *reinterpret_cast<const f32x4*>(carry0 + static_cast<size_t>(p) * N + c);
        }
        cv += s;
    }
    if (ru.z >= 0) {
        f32x4 s = f32x4(0.f);
        for (int p = ru.z; p <= ru.w; ++p) {
            s += *reinterpret_cast<const f32x4*>(carry1 + static_cast<size_t>(p) * N + c);
        }
        pv += s;
    }
    __builtin_nontemporal_store(cv + pv, reinterpret_cast<f32x4*>(C) + t);
}

// ---------------------------------------------------------------------------
// Sub-wave row groups (the short-row / narrow-N form of spmm_tiled_v3).
//
// A group of L = LC * LE lanes owns one row: LC column lanes cover LC * VEC
// contiguous columns (one pass; more passes when N is wider) and LE entry
// lanes take the row's entries e, e + LE, e + 2*LE, ... so each lane gathers
// whole VEC-float segments of B rows for its own entries.  A wave holds
// 64 / L rows, a 256-thread workgroup four waves; rows never cross groups, so
// there is no row bookkeeping in the loop, and the group phase needs no LDS
// and no barrier.  At the end of a row the entry lanes' partials are summed
// with xor shuffles (fixed order) and entry lane 0 stores the row.
//
// For N of a few columns the row-block engine leaves most lanes idle (its
// groups cover columns, at most 8 per wave) and pays its per-step row tests on
// every entry; here a wave gathers 64 / LC entries per load instruction.
// Measured on MI355X: 1.5 - 4x faster than the engine for N <= 32 on uniform
// rows of 1 .. 300 entries, up to 2x at N = 64, and for N = 128 / 256 on rows
// of a few entries.
//
// A row longer than 8 iterations of its group (8 * LE * U entries) and than
// 4x the average row is not taken by the group but by the whole workgroup
// afterwards (4 * 64 / LC entry lanes, partials added through LDS), so it is
// taken by 256 / L times the lanes.  (Rows of about average length stay in
// their groups: moving them would only serialise the workgroup's rows.)  Rows far longer than that belong
// to the engine or the merge-path partition, which share a row between waves
// and workgroups; the dispatch rule below keeps them there.
// ---------------------------------------------------------------------------
struct RowGroupArgs {
    const int*   row_ptr;
    const int*   col_idx;
    const float* vals;
    const float* B;
    float*       C;
    int          M;
    int          N;
    int          K;
    int          lc_log;    // column lanes per row: 1 << lc_log
    int          le_log;    // entry lanes per row: 1 << le_log
    int          long_len;  // rows with more entries go to the workgroup-wide pass
    int          slices;    // XCD-tied column slices: 1, 2, 4 or 8
    int          slice_cols;
    int          nblocks;   // row blocks (workgroups of one column slice)
};

template <int VEC>
__device__ __forceinline__ typename Vec<VEC>::T xor_add(typename Vec<VEC>::T v, int m) {
    if constexpr (VEC == 1) {
        return v + shfl_xor_f(v, m);
    } else {
        typename Vec<VEC>::T o;
#pragma unroll
        for (int i = 0; i < VEC; ++i) o[i] = shfl_xor_f(v[i], m);
        return v + o;
    }
}

// Sum over the entries p0, p0 + stride, ... (< p1) of the row: U entries per
// iteration, their column indices and values loaded before their B segments.
template <int VEC, int U>
__device__ __forceinline__ typename Vec<VEC>::T row_segment_sum(
    const RowGroupArgs& a, __amdgpu_buffer_rsrc_t rb, int p0, int p1, int stride, int colb) {
    using VT = typename Vec<VEC>::T;
    VT acc = vzero<VEC>();
    for (int p = p0; p < p1; p += stride * U) {
        int   ks[U];
        float vs[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = p + u * stride;
            const bool in = q < p1;
            ks[u] = in ? a.col_idx[q] : -1;  // -1: outside the buffer, reads zeros
            vs[u] = in ? a.vals[q] : 0.0f;
        }
        VT bs[U];
#pragma unroll
        for (int u = 0; u < U; ++u) bs[u] = load_b<VEC, true>(rb, nullptr, ks[u], colb, a.N);
#pragma unroll
        for (int u = 0; u < U; ++u) acc += vs[u] * bs[u];
    }
    return acc;
}

// Cooperative form of a group's pass over entries [p0, p1): the L lanes of
// the group (lanes g0 .. g0+L-1, this lane gl) load L consecutive entries with
// one coalesced load for the columns and one for the values, and sub-step j
// hands entry j*LE + e to lane (e, c) with a shuffle -- one load per L entries
// instead of one per entry lane and entry.
template <int VEC, int U>
__device__ __forceinline__ typename Vec<VEC>::T row_chunks_sum(
    const RowGroupArgs& a, __amdgpu_buffer_rsrc_t rb, int p0, int p1, int g0, int gl, int e,
    int L, int LE, int colb, int chunk_stride) {
    using VT = typename Vec<VEC>::T;
    VT acc = vzero<VEC>();
    const int sub = L / LE;  // sub-steps per chunk (= column lanes)
    for (int base = p0; base < p1; base += chunk_stride) {
        const int   q   = base + gl;
        const int   kc  = q < p1 ? a.col_idx[q] : -1;
        const float vc  = q < p1 ? a.vals[q] : 0.0f;
        const int   cnt = min(L, p1 - base);
        for (int j0 = 0; j0 < sub && j0 * LE < cnt; j0 += U) {
            int   ks[U];
            float vs[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int src = g0 + (((j0 + u) * LE + e) & (L - 1));
                ks[u] = __shfl(kc, src);
                vs[u] = __shfl(vc, src);
                if (j0 + u >= sub) {
                    ks[u] = -1;
                    vs[u] = 0.0f;
                }
            }
            VT bs[U];
#pragma unroll
            for (int u = 0; u < U; ++u) bs[u] = load_b<VEC, true>(rb, nullptr, ks[u], colb, a.N);
#pragma unroll
            for (int u = 0; u < U; ++u) acc += vs[u] * bs[u];
        }
    }
    return acc;
}

template <int VEC, int U, bool COOP, bool LONG_ROWS>
__global__ __launch_bounds__(256) void csr_row_groups(RowGroupArgs a) {
    using VT = typename Vec<VEC>::T;
    const int LC   = 1 << a.lc_log;
    const int LE   = 1 << a.le_log;
    const int L    = LC * LE;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int gl   = lane & (L - 1);
    const int c    = gl & (LC - 1);
    const int e    = gl >> a.lc_log;
    // Column slices tied to XCDs as in the engine: workgroup g runs on XCD
    // g % 8, and with S slices XCDs s*8/S .. (s+1)*8/S - 1 compute columns
    // [s*SC, (s+1)*SC) of every row block, so each XCD's L2 holds 1/S of B.
    int rblk = blockIdx.x, slice = 0;
    if (a.slices > 1) {
        const int per = 8 / a.slices;
        const int x   = blockIdx.x & 7;
        rblk  = (blockIdx.x >> 3) * per + x % per;
        slice = x / per;
    }
    if (rblk >= a.nblocks) return;  // whole workgroup, before any barrier
    const int cbeg = slice * a.slice_cols;
    const int cend = min(a.N, cbeg + a.slice_cols);
    const int row  = (rblk * 4 + wave) * (kWave / L) + (lane >> (a.lc_log + a.le_log));
    const bool live = row < a.M;
    int start = 0, end = 0;
    if (live) {
        start = a.row_ptr[row];
        end   = a.row_ptr[row + 1];
    }
    // LONG_ROWS = false: the caller knows no row exceeds long_len.
    const bool is_long = LONG_ROWS && end - start > a.long_len;
    const int  g_end   = is_long ? start : end;
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a.B), static_cast<short>(a.N * 4), a.K, kBufWord3);

    for (int n0 = cbeg; n0 < cend; n0 += LC * VEC) {
        const int  n    = n0 + c * VEC;
        const bool col  = n < cend;  // lanes past the slice read column 0 and store nothing
        VT acc;
        if constexpr (COOP) {
            acc = row_chunks_sum<VEC, U>(a, rb, start, g_end, lane & ~(L - 1), gl, e, L, LE,
                                         col ? n * 4 : 0, L);
        } else {
            acc = row_segment_sum<VEC, U>(a, rb, start + e, g_end, LE, col ? n * 4 : 0);
        }
        for (int m = LC; m < L; m <<= 1) acc = xor_add<VEC>(acc, m);
        if (live && !is_long && e == 0 && col) {
            store_vec<VEC>(a.C + static_cast<size_t>(row) * a.N + n, acc);
        }
    }

    if constexpr (!LONG_ROWS) return;
    // Long rows of this workgroup, one at a time with all four waves: wave w
    // takes the entries of lanes w*WE .. w*WE+WE-1 of every 4*WE (per-lane
    // loads) or every fourth 64-entry chunk (cooperative loads), and wave 0
    // adds the four waves' partials in wave order (deterministic).
    __shared__ int s_long_rows[4][kWave];
    __shared__ int s_long_cnt[4];
    __shared__ VT  s_part[4][kWave];
    const unsigned long long longs = __ballot(live && is_long && gl == 0);
    if (lane == 0) s_long_cnt[wave] = __popcll(longs);
    if (live && is_long && gl == 0) {
        s_long_rows[wave][__popcll(longs & ((1ull << lane) - 1))] = row;
    }
    __syncthreads();
    const int WE = kWave / LC;  // entry lanes per wave
    const int we = lane >> a.lc_log;
    for (int w2 = 0; w2 < 4; ++w2) {
        const int cnt = s_long_cnt[w2];
        for (int i = 0; i < cnt; ++i) {
            const int r  = s_long_rows[w2][i];
            const int rs = a.row_ptr[r];
            const int re = a.row_ptr[r + 1];
            for (int n0 = cbeg; n0 < cend; n0 += LC * VEC) {
                const int  n   = n0 + c * VEC;
                const bool col = n < cend;
                VT acc;
                // One row at a time: four entries per lane in flight.
                if constexpr (COOP) {
                    acc = row_chunks_sum<VEC, 4>(a, rb, rs + wave * kWave, re, 0, lane, we, kWave,
                                                 WE, col ? n * 4 : 0, 4 * kWave);
                } else {
                    acc = row_segment_sum<VEC, 4>(a, rb, rs + wave * WE + we, re, 4 * WE,
                                                  col ? n * 4 : 0);
                }
                for (int m = LC; m < kWave; m <<= 1) acc = xor_add<VEC>(acc, m);
                if (we == 0) s_part[wave][c] = acc;
                __syncthreads();
                if (wave == 0 && we == 0 && col) {
                    const VT sum = ((s_part[0][c] + s_part[1][c]) + s_part[2][c]) + s_part[3][c];
                    store_vec<VEC>(a.C + static_cast<size_t>(r) * a.N + n, sum);
                }
                __syncthreads();
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Launch helpers
// ---------------------------------------------------------------------------

Error ok() { return Error{}; }

Error fail(int status, std::string msg) { return Error{status, std::move(msg)}; }

Error from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    return fail(kHipError, std::string(what) + ": " + hipGetErrorString(e));
}

bool aligned(const void* p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// Widest VEC (<= want, 4 when want == 0) that keeps every lane's VEC floats
// inside one row and naturally aligned.
int pick_vec(int N, const float* B, float* C, int want) {
    if (want == 0) want = 4;
    for (int v = want; v > 1; v >>= 1) {
        if (N % v == 0 && aligned(B, sizeof(float) * v) && aligned(C, sizeof(float) * v)) return v;
    }
    return 1;
}


// Groups per wave: enough lanes per group to cover N in one pass, at most 8
// groups (8 lanes of 16 bytes) and at least 1 (64 lanes, several passes for
// wide N).
int pick_groups(int N, int vec, int want) {
    if (want == 1 || want == 2 || want == 4 || (want == 8 && vec == 4)) return want;
    const int lanes = (N + vec - 1) / vec;
    if (lanes <= 8 && vec == 4) return 8;
    if (lanes <= 16) return 4;
    if (lanes <= 32) return 2;
    return 1;
}

template <int VEC, int G, int WAVES, int U, bool SBUF>
hipError_t run_rowblock(const RowblockArgs& args, int grid, hipStream_t stream) {
    hipLaunchKernelGGL((csr_rowblock<VEC, G, WAVES, U, SBUF>), dim3(grid), dim3(WAVES * kWave), 0,
                       stream, args);
    return hipGetLastError();
}

// Launch shapes: waves per workgroup (2, 4, 8) x entries in flight per lane
// per step (4, 8).  B loads through a structured buffer unless B is too large
// for one (then only the default shape, 8 waves x 4, is built).
template <int VEC, int G>
hipError_t dispatch_shape(int waves, int unroll, bool sbuf, const RowblockArgs& args, int grid,
                          hipStream_t stream) {
    if (!sbuf) return run_rowblock<VEC, G, 8, 4, false>(args, grid, stream);
    if (waves == 8) {
        return unroll == 8 ? run_rowblock<VEC, G, 8, 8, true>(args, grid, stream)
                           : run_rowblock<VEC, G, 8, 4, true>(args, grid, stream);
    }
    if (waves == 2) {
        return unroll == 8 ? run_rowblock<VEC, G, 2, 8, true>(args, grid, stream)
                           : run_rowblock<VEC, G, 2, 4, true>(args, grid, stream);
    }
    return unroll == 8 ? run_rowblock<VEC, G, 4, 8, true>(args, grid, stream)
                       : run_rowblock<VEC, G, 4, 4, true>(args, grid, stream);
}

template <int VEC>
hipError_t dispatch_groups(int groups, int waves, int unroll, bool sbuf, const RowblockArgs& args,
                           int grid, hipStream_t stream) {
    if constexpr (VEC == 4) {
        if (groups == 8) return dispatch_shape<VEC, 8>(waves, unroll, sbuf, args, grid, stream);
    }
    if (groups == 4) return dispatch_shape<VEC, 4>(waves, unroll, sbuf, args, grid, stream);
    if (groups == 2) return dispatch_shape<VEC, 2>(waves, unroll, sbuf, args, grid, stream);
    return dispatch_shape<VEC, 1>(waves, unroll, sbuf, args, grid, stream);
}

// Column slices for a K x N fp32 B: the fewest (a power of two, at most 8,
// each slice at least 64 columns wide) that bring one XCD's share of B down
// to its 4 MiB L2.  Measured on MI355X: B of 8 MiB (16384 x 128, 8192 x 256)
// 1.2-1.7x faster with 2 slices; B of 4 MiB or less is fastest unsliced.
int auto_slices(int K, int N) {
    const long long b_bytes = static_cast<long long>(K) * N * 4;
    int s = 1;
    while (s < 8 && b_bytes > (4LL << 20) * s && N / (2 * s) >= 64) s *= 2;
    return s;
}

int default_waves(int slices) { return slices == 1 ? 8 : 4; }

// Waves of the engine resident at once on the chip: 16 per CU (four 4-wave
// workgroups) on 256 CUs.
constexpr long kRoundWaves = 4096;

// Rows whose lengths stay within twice the average (plus a constant for
// short rows): uniform random rows qualify, power-law rows do not.
bool rows_even(int M, long long nnz, int max_row) {
    return max_row > 0 && M > 0 &&
           max_row <= 2.0 * static_cast<double>(nnz) / M + 32.0;
}

// Rows per workgroup of the 4-wave row-block launch for even rows: the grid
// is a whole number of rounds of kRoundWaves waves, one round per ~2 M entry
// visits (nnz x slices, ~512 entries per wave).  A partial last round leaves
// CUs idle while it runs.  Measured on MI355X over uniform rows (M 2048 ..
// 32768, 8 .. 164 entries per row, N 64 .. 256), whole rounds gain up to
// 1.35x over ~160 entries per wave (1.2 - 1.6 rounds at M = 12288 .. 16384).
// Skewed rows need the many small workgroups of the default instead: a
// static one-round partition loses up to 1.5x on power-law rows.
int round_rows_per_block(int M, long long nnz, int slices, int waves) {
    const double visits = static_cast<double>(nnz) * slices;
    const long rounds = std::max(1L, std::lround(visits / (kRoundWaves * 512.0)));
    const long blocks = std::max(1L, rounds * kRoundWaves / (static_cast<long>(waves) * slices));
    return static_cast<int>(std::min<long>(kRpCap, std::max(1L, (M + blocks - 1) / blocks)));
}

// B rows as buffer records: the record stride field holds at most 16383
// bytes and the buffer's byte range must fit a signed 32-bit offset.
bool b_fits_buffer(int K, int N) {
    return static_cast<long long>(N) * 4 <= 16383 &&
           static_cast<long long>(K) * N * 4 <= 0x7fffffffLL;
}
}  // namespace

int default_partition_parts(int num_rows, int nnz) {
    // About 1280 nonzeros per workgroup (160 per wave of the default 8-wave
    // shape), at least two workgroups per CU and at most one per row.
    long parts = (static_cast<long>(nnz) + 1279) / 1280;
    parts = std::max<long>(parts, 512);
    parts = std::min<long>(parts, std::max(num_rows, 1));
    return static_cast<int>(std::max<long>(parts, 1));
}

namespace {

int pow2_log_at_least(int x) {
    int l = 0;
    while ((1 << l) < x && l < 6) ++l;
    return l;
}

// Column lanes (log2) of a row group: enough to cover N in one pass, at most
// 64; 32 or 64 drop to 16 (two or four column passes) while the matrix would
// still give >= 16384 waves.
constexpr long kRowGroupTargetWaves = 8192;
int row_group_lc_log(int M, int N, int vec) {
    int lc_log = pow2_log_at_least(ceil_div(N, vec));
    while (lc_log > 4 && (static_cast<long>(M) << lc_log) / kWave >= 2 * kRowGroupTargetWaves) {
        --lc_log;
    }
    return lc_log;
}

// XCD-tied column slices of the row groups: on rows of up to 24 entries with
// a B larger than one XCD's 4 MiB L2, the fewest slices (a power of two, at
// most 8, each at least 32 columns wide) that bring an XCD's share of B under
// 4 MiB (measured on MI355X: M = 16384, N = 256, 16 per row 28.4 -> 20.2 us
// with 4 slices; M = 32768, N = 128: 28.5 -> 25.0 us).  Longer rows keep one
// slice: every slice re-reads the rows' column indices, which then costs more
// than the L2 misses it saves.
int row_group_slices(int K, int N, double avg_row) {
    if (avg_row > 24.0) return 1;
    const long long b_bytes = static_cast<long long>(K) * N * 4;
    int s = 1;
    while (s < 8 && b_bytes > (4LL << 20) * s && N / (2 * s) >= 32) s *= 2;
    return s;
}

template <int VEC, bool COOP, bool LONG_ROWS>
hipError_t run_row_groups(const RowGroupArgs& args, int unroll, int grid, hipStream_t stream) {
    if (unroll == 4) {
        hipLaunchKernelGGL((csr_row_groups<VEC, 4, COOP, LONG_ROWS>), dim3(grid), dim3(256), 0,
                           stream, args);
    } else {
        hipLaunchKernelGGL((csr_row_groups<VEC, 2, COOP, LONG_ROWS>), dim3(grid), dim3(256), 0,
                           stream, args);
    }
    return hipGetLastError();
}

template <int VEC>
hipError_t run_row_groups(const RowGroupArgs& args, bool coop, bool long_rows, int unroll,
                          int grid, hipStream_t stream) {
    if (long_rows) {
        return coop ? run_row_groups<VEC, true, true>(args, unroll, grid, stream)
                    : run_row_groups<VEC, false, true>(args, unroll, grid, stream);
    }
    return coop ? run_row_groups<VEC, true, false>(args, unroll, grid, stream)
                : run_row_groups<VEC, false, false>(args, unroll, grid, stream);
}

// Shape of the sub-wave row groups, measured on MI355X over uniform rows of
// 1 .. 300 entries, M = 2048 .. 65536 and N = 1 .. 256:
//  - column lanes cover N in one pass (up to 64 lanes), except that 32 or 64
//    column lanes drop to 16 (two or four passes) while the matrix would
//    still give >= 16384 waves (e.g. M = 32768, N = 128: 96 -> 89 us);
//  - entry lanes ~1.5 * sqrt(average row) as a power of two, but no more than
//    keep the grid near 8192 waves (32 per CU): beyond that, more rows per
//    wave beat more lanes per row;
//  - 4 entries per entry lane per iteration from 32 entries per row on while
//    B is at most 2 MiB (latency-bound: few, long rows), else 2 -- with B
//    beyond one XCD's L2, fewer gathers in flight keep more of it cached
//    (M = 32768, N = 128, 82 entries per row: 123 -> 88 us);
//  - the cooperative loads (one column/value load per L entries, handed out
//    by shuffles) from 4 column lanes on when rows average >= 32 entries or
//    column lanes x rows >= 2^18: redundant per-lane index loads then cost
//    more than the shuffles (M = 8192, N = 64, 82 per row: 11.4 -> 9.1 us;
//    M = 32768, N = 128: 119 -> 87 us); on short rows of a smaller matrix the
//    per-lane loads are 5-15% ahead.
// row_groups: 1 picks the load form by that rule, 2 forces per-lane loads,
// 3 forces the cooperative loads.
Error launch_row_groups(const CSR& A, const float* B, float* C, int N, hipStream_t stream,
                        int vec, const EngineOpts& o) {
    constexpr long kTargetWaves = kRowGroupTargetWaves;
    const int M = A.num_rows;
    const double avg = A.nnz > 0 ? static_cast<double>(A.nnz) / M : 0.0;
    int slices = o.slices;
    if (slices == 0) slices = row_group_slices(A.num_cols, N, avg);
    if (slices != 1 && slices != 2 && slices != 4 && slices != 8) slices = 1;
    const int slice_cols = ceil_div(ceil_div(N, slices), vec) * vec;
    const int lc_log = row_group_lc_log(M, slice_cols, vec);
    int le_log;
    if (o.entry_lanes != 0) {
        if (o.entry_lanes < 0 || o.entry_lanes > 64 || (o.entry_lanes & (o.entry_lanes - 1)) != 0) {
            return fail(kInvalid, "entry_lanes must be a power of two up to 64");
        }
        le_log = pow2_log_at_least(o.entry_lanes);
    } else {
        const double want = 1.5 * std::sqrt(std::max(avg, 1.0));
        le_log = static_cast<int>(std::lround(std::log2(want)));
        const long cap =
            kTargetWaves * kWave / std::max(1L, (static_cast<long>(M) << lc_log) * slices);
        int cap_log = 0;
        while ((2L << cap_log) <= cap) ++cap_log;
        le_log = std::min(le_log, cap_log);
    }
    le_log = std::max(0, std::min(le_log, 6 - lc_log));
    const bool b_small = static_cast<long long>(A.num_cols) * N * 4 <= (2LL << 20);
    const int unroll = (o.unroll == 2 || o.unroll == 4) ? o.unroll
                                                        : ((avg >= 32.0 && b_small) ? 4 : 2);
    bool coop;
    if (o.row_groups == 2) coop = false;
    else if (o.row_groups == 3) coop = true;
    else coop = lc_log >= 2 && (avg >= 32.0 || (static_cast<long>(M) << lc_log) >= (1L << 18));
    const int rows_per_wg = 4 * (kWave >> (lc_log + le_log));
    const int nblocks = ceil_div(M, rows_per_wg);
    const int grid = slices == 1 ? nblocks : ceil_div(nblocks, 8 / slices) * 8;
    const int long_len = std::max(8 << le_log << (unroll == 4 ? 2 : 1),
                                  static_cast<int>(std::ceil(std::min(4.0 * avg, 1.0e9))));
    RowGroupArgs args{A.row_ptr, A.col_idx,  A.values,   B,          C,
                      M,         N,          A.num_cols, lc_log,     le_log,
                      long_len,  slices,     slice_cols, nblocks};
    // Without a longest-row hint any row may be long: the workgroup-wide pass
    // (one barrier even when no row needs it) is compiled in.
    const bool long_rows = o.max_row_hint <= 0 || o.max_row_hint > long_len;
    hipError_t e;
    if (vec == 4) e = run_row_groups<4>(args, coop, long_rows, unroll, grid, stream);
    else if (vec == 2) e = run_row_groups<2>(args, coop, long_rows, unroll, grid, stream);
    else e = run_row_groups<1>(args, coop, long_rows, unroll, grid, stream);
    return from_hip(e, "csr row groups launch");
}

Error launch_csr_impl(CsrRole role, const CSR& A, const float* B, float* C, int N,
                      hipStream_t stream, const int* bounds, int parts, const EngineOpts* opts,
                      const SplitPlan* split) {
    if (A.num_rows < 0 || A.num_cols < 0 || A.nnz < 0 || N < 0) {
        return fail(kInvalid, "negative matrix dimension");
    }
    if (A.num_rows == 0 || N == 0) return ok();
    if (A.row_ptr == nullptr || B == nullptr || C == nullptr) {
        return fail(kInvalid, "null device pointer");
    }
    if (A.nnz > 0 && (A.col_idx == nullptr || A.values == nullptr)) {
        return fail(kInvalid, "null device pointer");
    }
    if (bounds != nullptr && parts < 1) return fail(kInvalid, "partition needs parts >= 1");

    const int M = A.num_rows;
    switch (role) {
        case CsrRole::Baseline: {
            dim3 block(kWave, 4);
            dim3 grid(ceil_div(N, kWave), ceil_div(M, 4));
            hipLaunchKernelGGL(csr_lane_per_output, grid, block, 0, stream, M, N, A.row_ptr,
                               A.col_idx, A.values, B, C);
            return from_hip(hipGetLastError(), "spmm_baseline launch");
        }
        case CsrRole::Memopt:
            hipLaunchKernelGGL((csr_wave_per_row<2, 1>), dim3(ceil_div(M, 4)), dim3(256), 0, stream,
                               M, N, A.row_ptr, A.col_idx, A.values, B, C);
            return from_hip(hipGetLastError(), "spmm_memopt launch");
        case CsrRole::MemoptV2:
            hipLaunchKernelGGL((csr_wave_per_row<2, 8>), dim3(ceil_div(M, 4)), dim3(256), 0, stream,
                               M, N, A.row_ptr, A.col_idx, A.values, B, C);
            return from_hip(hipGetLastError(), "spmm_memopt_v2 launch");
        default:
            break;
    }

    EngineOpts o = opts ? *opts : EngineOpts{};
    int want_vec = o.vec;
    int want_groups = o.groups;
    if (role == CsrRole::Tiled && want_vec == 0) {
        want_vec = 1;  // one lane per column, 64 columns per pass
        if (want_groups == 0) want_groups = 1;
    }
    if ((role == CsrRole::TiledV2 || role == CsrRole::TiledV4) && want_vec == 0) want_vec = 4;
    if (role == CsrRole::TiledV2) {
        if (N % 128 != 0) {
            return fail(kUnsupported, "spmm_tiled_v2 requires N % 128 == 0 (got N=" +
                                          std::to_string(N) + ")");
        }
        if (!aligned(B, 16) || !aligned(C, 16)) {
            return fail(kUnsupported, "spmm_tiled_v2 requires 16-byte aligned B and C");
        }
    }
    if (want_vec != 0 && want_vec != 1 && want_vec != 2 && want_vec != 4) {
        return fail(kInvalid, "engine vec must be 1, 2 or 4");
    }
    const int vec = pick_vec(N, B, C, want_vec);
    // Default launches of the production roles at N of a few columns (at most
    // four column lanes of VEC floats, e.g. N <= 16 with 16-byte lanes) take
    // the sub-wave row groups: the engine keeps half or more of its lanes idle
    // there, and with 64 .. 256 entry lanes the row groups' workgroup-wide
    // pass shares a long row among many lanes.  Measured on MI355X without
    // row-length knowledge: 1.6 - 3.4x faster on uniform rows at N <= 8 and
    // 2.5 - 3.6x on power-law rows of up to 4096 entries; at N = 12 - 16 over
    // 32 uniform and power-law inputs (M 2048 .. 65536) 2.0x on average, never
    // slower (1.18x at worst).  Up to eight lanes (N <= 32) they win 1.07 -
    // 1.75x on the inputs of up to 2.5 M nonzeros but lose 0.79 - 0.97x on
    // power-law inputs of 4.6 M nonzeros and more, so five to eight lanes take
    // them only up to 4 M nonzeros.  Any explicit engine option keeps the
    // engine, and so does a longest-row hint: a caller that knows its rows
    // (spmm_hybrid_run) chooses the form itself.
    const bool engine_defaults = o.vec == 0 && o.waves == 0 && o.unroll == 0 &&
                                 o.rows_per_block == 0 && o.groups == 0 && o.slices == 0 &&
                                 o.global_loads == 0 && o.entry_lanes == 0 &&
                                 o.max_row_hint == 0;
    if (o.row_groups == 0 && engine_defaults && bounds == nullptr && split == nullptr &&
        (role == CsrRole::TiledV3 || role == CsrRole::TiledV4) &&
        b_fits_buffer(A.num_cols, N) &&
        (pow2_log_at_least(ceil_div(N, vec)) <= 2 ||
         (pow2_log_at_least(ceil_div(N, vec)) <= 3 && A.nnz <= (1 << 22)))) {
        EngineOpts rg = o;
        rg.row_groups = 1;
        return launch_row_groups(A, B, C, N, stream, vec, rg);
    }
    if (o.row_groups != 0) {
        if (o.row_groups < 0 || o.row_groups > 3) {
            return fail(kInvalid, "row_groups must be 0 (engine), 1 (auto), 2 or 3");
        }
        if (bounds != nullptr || split != nullptr) {
            return fail(kInvalid, "row groups take no explicit partition");
        }
        if (!b_fits_buffer(A.num_cols, N)) {
            return fail(kUnsupported, "row groups need N <= 4095 and B within 2 GiB");
        }
        return launch_row_groups(A, B, C, N, stream, vec, o);
    }
    // Column slices (XCD-aware, see the kernel): 1, 2, 4 or 8.
    int slices = o.slices;
    if (slices == 0) slices = role == CsrRole::Tiled ? 1 : auto_slices(A.num_cols, N);
    if (slices != 1 && slices != 2 && slices != 4 && slices != 8) slices = 1;
    int slice_cols = ceil_div(N, slices);
    slice_cols = ceil_div(slice_cols, vec) * vec;
    const int groups = pick_groups(slice_cols, vec, want_groups);
    // Defaults measured on MI355X (c1 / c2 / c5 and uniform / power-law
    // sweeps): 8 waves per workgroup without column slices (a workgroup's
    // nonzeros are split over its waves, so a long row is shared by eight),
    // 4 with them (the sliced launch has twice the workgroups per row block),
    // 4 entries per group in flight per step (two steps in flight), about 160
    // nonzeros per wave and at least 512 workgroups (two per CU) when the
    // matrix allows it: many small workgroups keep skewed rows balanced.
    // Rows known to be even (max_row_hint): the whole-round grid of 4-wave
    // workgroups.
    const bool even = split == nullptr && bounds == nullptr && o.rows_per_block <= 0 &&
                      rows_even(M, A.nnz, o.max_row_hint);
    const int waves = (o.waves == 2 || o.waves == 4 || o.waves == 8) ? o.waves
                      : even                                         ? 4
                                                                     : default_waves(slices);
    const int unroll = o.unroll == 8 ? 8 : 4;
    const bool sbuf = o.global_loads == 0 && b_fits_buffer(A.num_cols, N);

    RowblockArgs args{A.row_ptr, A.col_idx, A.values, B,       C,       bounds, M, N, A.num_cols,
                      0,         0,         slices,   slice_cols, nullptr, nullptr, 0};
    if (split != nullptr) {
        args.bounds     = nullptr;
        args.split_rows = split->rows;
        args.carry      = split->carry;
        args.nnz        = A.nnz;
        args.nblocks    = split->parts;
    } else if (bounds != nullptr) {
        args.nblocks = parts;
    } else {
        int rpb = o.rows_per_block;
        if (rpb <= 0 && even) {
            rpb = round_rows_per_block(M, A.nnz, slices, waves);
        } else if (rpb <= 0) {
            const double avg = A.nnz > 0 ? static_cast<double>(A.nnz) / M : 1.0;
            rpb = static_cast<int>(160.0 * waves / std::max(avg, 1.0) + 0.5);
            rpb = std::min(rpb, M / 512);
        }
        rpb = std::max(1, std::min(rpb, kRpCap));
        args.rows_per_block = rpb;
        args.nblocks = ceil_div(M, rpb);
    }
    const int grid = slices == 1 ? args.nblocks : ceil_div(args.nblocks, 8 / slices) * 8;
    hipError_t e;
    if (vec == 4) {
        e = dispatch_groups<4>(groups, waves, unroll, sbuf, args, grid, stream);
    } else if (vec == 2) {
        e = dispatch_groups<2>(groups, waves, unroll, sbuf, args, grid, stream);
    } else {
        e = dispatch_groups<1>(groups, waves, unroll, sbuf, args, grid, stream);
    }
    if (e == hipSuccess && split != nullptr) {
        hipLaunchKernelGGL(csr_split_fixup, dim3(split->parts), dim3(64), 0, stream, A.row_ptr,
                           split->rows, split->carry, C, M, N, static_cast<long long>(A.nnz),
                           split->parts);
        e = hipGetLastError();
    }
    return from_hip(e, "csr engine launch");
}

}  // namespace

Error launch_csr(CsrRole role, const CSR& A, const float* B, float* C, int N,
                 hipStream_t stream, const int* bounds, int parts, const EngineOpts* opts) {
    return launch_csr_impl(role, A, B, C, N, stream, bounds, parts, opts, nullptr);
}

int split_partition_parts(int nnz) {
    // Two workgroups per CU: measured on MI355X over power-law inputs of 0.6 M
    // to 2.5 M nonzeros, 256 .. 1536 parts are within 10% of each other and
    // 4096 parts lose 15-40% to per-workgroup set-up and the fix-up; more
    // parts only for very large inputs (at most 64 K nonzeros per part).
    long parts = std::max<long>(512, (static_cast<long>(nnz) + 65535) / 65536);
    return static_cast<int>(std::min<long>(parts, std::max(nnz, 1)));
}

bool split_pays(int max_row_nnz) {
    // A row longer than four workgroups' share (4 x 640 nonzeros at 4 waves
    // of 160) keeps one row-partitioned workgroup busy long after the others:
    // then the merge-path partition wins (power-law 8192^2: 32 -> 23 us;
    // 16384^2 with two column slices: 88 -> 69 us); on rows of similar length
    // it costs its second launch (5-50%).
    return max_row_nnz > 4 * 640;
}

bool row_groups_pay(int M, int N, int K, double avg_row, int max_row) {
    // Measured on MI355X against the row-block engine as the hybrid runs it
    // (uniform rows of 8 .. 300 entries, M = 1024 .. 32768, N = 64 .. 256,
    // the engine with the longest row as its hint; power-law rows capped at
    // 512 / 4096).  Row groups win 1.5 - 4x for N <= 32 and 1.1 - 1.7x for
    // N = 64 (not on 1024 rows of > 100 entries, 0.75 - 0.9x).  Above
    // N = 64 they win on short rows (N x average <= 4096), when B needs
    // column slices, and at N = 128 on >= 4096 rows (1.03 - 1.6x) or >= 2048
    // rows of up to 10600 / N entries -- except at 4097 .. 8192 rows of
    // >= 64 entries, where the engine's whole-round grid holds 1 - 2 rows
    // per wave and matches or beats them (0.97 - 1.00x).  Those wins need
    // even rows: power-law rows of mean 164 capped at 512 run 0.6 - 0.7x.
    // With this rule the mean loss to the faster form over the sweep is
    // 0.14% (worst 5.6%).  A row longer than both 16384 / column-lanes
    // entries and 8x the average would keep one workgroup busy far longer
    // than the rest (more than ~16 iterations of its workgroup-wide pass):
    // then the engine, which shares long rows between eight waves with more
    // entries per step, is the safer choice.
    if (N <= 0 || M <= 0 || !b_fits_buffer(K, N)) return false;
    const int vec    = N % 4 == 0 ? 4 : (N % 2 == 0 ? 2 : 1);
    const int slices = row_group_slices(K, N, avg_row);
    const int lc     = 1 << row_group_lc_log(M, ceil_div(ceil_div(N, slices), vec) * vec, vec);
    if (max_row > std::max(16384.0 / lc, 8.0 * avg_row)) return false;
    if (N <= 64) return M >= 2048 || avg_row <= 100.0;
    if (N * avg_row <= 2048.0 || (N <= 256 && slices > 1)) return true;
    if (max_row > 2.0 * avg_row + 32.0) return false;  // uneven rows
    if (N * avg_row <= 4096.0) return true;
    if (N > 128) return false;
    if (M > 4096 && M <= 8192 && avg_row >= 64.0) return false;
    return M >= 4096 || (M >= 2048 && N * avg_row <= 10600.0);
}

Error launch_csr_split(const CSR& A, const float* B, float* C, int N, hipStream_t stream,
                       const SplitPlan& plan, const EngineOpts* opts) {
    if (plan.parts < 1 || plan.rows == nullptr) {
        return fail(kInvalid, "split partition needs parts >= 1 and its row table");
    }
    if (plan.parts > std::max(A.nnz, 1)) {
        // an empty part would break the fix-up's runs of continuation parts
        return fail(kInvalid, "split partition needs parts <= max(nnz, 1) (got parts=" +
                                  std::to_string(plan.parts) + ", nnz=" +
                                  std::to_string(A.nnz) + ")");
    }
    if (plan.carry == nullptr && N > 0 && A.num_rows > 0) {
        return fail(kInvalid, "split partition needs a carry workspace of parts x N floats");
    }
    return launch_csr_impl(CsrRole::TiledV3, A, B, C, N, stream, nullptr, 0, opts, &plan);
}

bool khalf_pays(int K, int N) {
    // B over one XCD's 4 MiB L2 at full width, its half of the rows within it.
    // Measured on MI355X on c5 (16384^2 power-law, N = 128, B 8 MiB): the
    // merge-path engine 64.0 -> 53.9 us with each half's B rows resident in
    // its four XCDs' L2s, the fix-up 4.7 -> 6.5 us (it now also adds the
    // second half's partial C), 67.7 -> 60.1 us per launch.
    const long long row_bytes = static_cast<long long>(N) * 4;
    return N > 0 && N % 4 == 0 && K >= 2 && b_fits_buffer(K, N) &&
           static_cast<long long>(K) * row_bytes > (4LL << 20) &&
           static_cast<long long>((K + 1) / 2) * row_bytes <= (4LL << 20);
}

Error launch_csr_khalf(const KHalfPlan& p, const float* B, float* C, hipStream_t stream) {
    if (p.M < 0 || p.N < 0) return fail(kInvalid, "negative matrix dimension");
    if (p.M == 0 || p.N == 0) return ok();
    if (B == nullptr || C == nullptr || p.partial == nullptr || p.runs == nullptr) {
        return fail(kInvalid, "null device pointer");
    }
    if (p.N % 4 != 0 || !aligned(B, 16) || !aligned(C, 16)) {
        return fail(kUnsupported, "B-row halves need N % 4 == 0 and 16-byte aligned B and C");
    }
    for (int h = 0; h < 2; ++h) {
        if (p.parts[h] < 1 || p.parts[h] > std::max(p.half[h].nnz, 1) || p.rows[h] == nullptr ||
            p.carry[h] == nullptr) {
            return fail(kInvalid, "B-row halves: incomplete plan");
        }
    }
    const int N = p.N;
    RowblockArgs args{p.half[0].row_ptr, p.half[0].col_idx, p.half[0].values, B, C, nullptr,
                      p.M, N, p.K0, 0, p.parts[0], 1, N, p.rows[0], p.carry[0], p.half[0].nnz};
    args.halves      = 1;
    args.row_ptr1    = p.half[1].row_ptr;
    args.col_idx1    = p.half[1].col_idx;
    args.vals1       = p.half[1].values;
    args.B1          = B + static_cast<size_t>(p.K0) * N;
    args.C1          = p.partial;
    args.K1          = p.K - p.K0;
    args.split_rows1 = p.rows[1];
    args.carry1      = p.carry[1];
    args.nnz1        = p.half[1].nnz;
    args.nblocks1    = p.parts[1];
    const int grid   = 8 * ceil_div(std::max(p.parts[0], p.parts[1]), 4);
    hipError_t e = dispatch_groups<4>(pick_groups(N, 4, 0), 4, 4, true, args, grid, stream);
    if (e == hipSuccess) {
        const long long chunks = static_cast<long long>(p.M) * N / 4;
        hipLaunchKernelGGL(csr_khalf_fixup, dim3(static_cast<unsigned>((chunks + 255) / 256)),
                           dim3(256), 0, stream, C, p.partial, p.carry[0], p.carry[1],
                           reinterpret_cast<const int4*>(p.runs), N, chunks);
        e = hipGetLastError();
    }
    return from_hip(e, "csr B-row halves launch");
}

}  // namespace engine
}  // namespace spmm
