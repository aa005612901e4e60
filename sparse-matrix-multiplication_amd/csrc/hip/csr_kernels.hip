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
#include <cstdint>

#include "engine.h"
#include "spmm/utils.h"

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
//
// Per wave.  The wave streams its range in 64-entry chunks: lane q holds
// (col_idx, value) of entry q in VGPRs and v_readlane broadcasts entry after
// entry into SGPRs.  For each entry the wave loads the B row segment
// B[k, c0 .. c0 + 64*VEC) (VEC floats per lane, UNROLL rows in flight) and
// accumulates into a per-lane register tile.  A row boundary flushes the tile:
//   - a row that lies wholly inside the wave's range is stored to C;
//   - the first row of a range that started in an earlier wave goes to an LDS
//     slot (s_part[wave]);
//   - the last row of a range that continues in a later wave stays in the
//     registers of its owner, which after a barrier adds the LDS slots of the
//     following waves in wave order and stores it.
// The sum order is therefore fixed by the partition: results are
// deterministic run to run.
//
// Rows of the workgroup without nonzeros are zero-filled up front.  Row
// pointers are staged in LDS in windows of RP_CAP rows.
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
    int          rows_per_block;
};

constexpr int kRpCap = 1024;

template <int VEC>
__device__ __forceinline__ void store_cols(float* crow, int col, bool col_ok,
                                           typename Vec<VEC>::T v) {
    if (col_ok) {
        __builtin_nontemporal_store(v, reinterpret_cast<typename Vec<VEC>::T*>(crow + col));
    }
}

template <int VEC, int WAVES, int UNROLL>
__global__ __launch_bounds__(WAVES * 64) void csr_rowblock(RowblockArgs a) {
    using VT = typename Vec<VEC>::T;
    constexpr int COLS = kWave * VEC;
    static_assert(kWave % UNROLL == 0, "UNROLL must divide the wave size");

    __shared__ int   s_rp[kRpCap + 1];
    __shared__ VT    s_part[WAVES][kWave];
    __shared__ int   s_first[WAVES];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int N = a.N;

    int r_begin, r_end;
    if (a.bounds != nullptr) {
        r_begin = a.bounds[blockIdx.x];
        r_end   = a.bounds[blockIdx.x + 1];
    } else {
        r_begin = blockIdx.x * a.rows_per_block;
        r_end   = min(a.M, r_begin + a.rows_per_block);
    }

    for (int w0 = r_begin; w0 < r_end; w0 += kRpCap) {
        const int nr = min(r_end - w0, kRpCap);
        __syncthreads();  // the previous window is no longer read
        for (int i = threadIdx.x; i <= nr; i += WAVES * kWave) s_rp[i] = a.row_ptr[w0 + i];
        __syncthreads();

        // Zero-fill the rows of this window that hold no nonzeros.
        for (int base = wave * kWave; base < nr; base += WAVES * kWave) {
            const int i = base + lane;
            uint64_t empty = __ballot(i < nr && s_rp[i] == s_rp[i + 1]);
            while (empty) {
                const int b = __builtin_ctzll(empty);
                empty &= empty - 1;
                float* crow = a.C + static_cast<size_t>(w0 + base + b) * N;
                for (int c = lane * VEC; c < N; c += COLS) store_cols<VEC>(crow, c, true, vzero<VEC>());
            }
        }

        const int nz0 = s_rp[0];
        const int total = s_rp[nr] - nz0;
        if (total == 0) continue;  // uniform across the workgroup
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

        for (int c0 = 0; c0 < N; c0 += COLS) {
            const int col = c0 + lane * VEC;
            const bool col_ok = col < N;
            if (lane == 0) s_first[wave] = (pa < pb) ? -1 : -2;

            int owner_row = -1;  // local row this wave must finish after the barrier
            VT acc = vzero<VEC>();
            if (pa < pb) {
                int row = first;
                int row_stop = s_rp[row + 1];
                bool head = s_rp[row] < pa;  // row began in an earlier wave

                for (int base = pa; base < pb; base += kWave) {
                    const int cnt = min(kWave, pb - base);
                    int   kc = 0;
                    float vc = 0.f;
                    if (lane < cnt) {
                        kc = __builtin_nontemporal_load(a.col_idx + base + lane);
                        vc = __builtin_nontemporal_load(a.vals + base + lane);
                    }
                    for (int j = 0; j < cnt; j += UNROLL) {
                        VT bv[UNROLL];
#pragma unroll
                        for (int u = 0; u < UNROLL; ++u) {
                            const int q = j + u;
                            const int k = __builtin_amdgcn_readlane(kc, q);
                            const float* brow = a.B + static_cast<size_t>(k) * N;
                            bv[u] = (q < cnt && col_ok)
                                        ? *reinterpret_cast<const VT*>(brow + col)
                                        : vzero<VEC>();
                        }
#pragma unroll
                        for (int u = 0; u < UNROLL; ++u) {
                            const int q = j + u;
                            if (q < cnt) {
                                const int pos = base + q;
                                if (pos >= row_stop) {
                                    if (head) {
                                        s_part[wave][lane] = acc;
                                        if (lane == 0) s_first[wave] = row;
                                        head = false;
                                    } else {
                                        store_cols<VEC>(a.C + static_cast<size_t>(w0 + row) * N,
                                                        col, col_ok, acc);
                                    }
                                    acc = vzero<VEC>();
                                    // bounded by the window even for a malformed row_ptr
                                    do {
                                        ++row;
                                        row_stop = s_rp[row + 1];
                                    } while (row_stop <= pos && row < nr - 1);
                                }
                                const float v = __builtin_bit_cast(
                                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vc), q));
                                acc = v * bv[u] + acc;
                            }
                        }
                    }
                }
                // The row being accumulated when the range ends.
                if (row_stop == pb && !head) {
                    store_cols<VEC>(a.C + static_cast<size_t>(w0 + row) * N, col, col_ok, acc);
                } else if (head) {
                    s_part[wave][lane] = acc;
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
                    acc += s_part[w][lane];
                }
                store_cols<VEC>(a.C + static_cast<size_t>(w0 + owner_row) * N, col, col_ok, acc);
            }
            __syncthreads();  // s_part / s_first are rewritten by the next column pass
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

// Largest VEC the shapes allow: every lane's VEC floats must be in one row and
// naturally aligned.
int pick_vec(int N, const float* B, float* C, int want) {
    auto fits = [&](int v) {
        return N % v == 0 && aligned(B, sizeof(float) * v) && aligned(C, sizeof(float) * v);
    };
    if (want == 0) {
        // one column pass when possible, widest loads otherwise
        want = N <= 64 ? 1 : (N <= 128 ? 2 : 4);
    }
    for (int v = want; v > 1; v >>= 1) {
        if (fits(v)) return v;
    }
    return 1;
}

template <int VEC, int WAVES, int UNROLL>
hipError_t run_rowblock(const RowblockArgs& args, int grid, hipStream_t stream) {
    hipLaunchKernelGGL((csr_rowblock<VEC, WAVES, UNROLL>), dim3(grid), dim3(WAVES * kWave), 0,
                       stream, args);
    return hipGetLastError();
}

template <int VEC>
hipError_t dispatch_waves_unroll(int waves, int unroll, const RowblockArgs& args, int grid,
                                 hipStream_t stream) {
    if (waves == 8) {
        return unroll == 8 ? run_rowblock<VEC, 8, 8>(args, grid, stream)
                           : run_rowblock<VEC, 8, 16>(args, grid, stream);
    }
    return unroll == 8 ? run_rowblock<VEC, 4, 8>(args, grid, stream)
                       : run_rowblock<VEC, 4, 16>(args, grid, stream);
}

}  // namespace

int default_partition_parts(int num_rows, int nnz) {
    // About 1024 nonzeros per workgroup, at least one workgroup per CU and at
    // most one per row.
    long parts = (static_cast<long>(nnz) + 1023) / 1024;
    parts = std::max<long>(parts, 256);
    parts = std::min<long>(parts, std::max(num_rows, 1));
    return static_cast<int>(std::max<long>(parts, 1));
}

Error launch_csr(CsrRole role, const CSR& A, const float* B, float* C, int N,
                 hipStream_t stream, const int* bounds, int parts, const EngineOpts* opts) {
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
    if (role == CsrRole::Tiled && want_vec == 0) want_vec = 1;
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
    const int waves = o.waves == 8 ? 8 : 4;
    const int unroll = o.unroll == 8 ? 8 : 16;

    RowblockArgs args{A.row_ptr, A.col_idx, A.values, B, C, bounds, M, N, 0};
    int grid = 0;
    if (bounds != nullptr) {
        grid = parts;
    } else {
        int rpb = o.rows_per_block;
        if (rpb <= 0) {
            // About 128 nonzeros per wave on average.
            const double avg = A.nnz > 0 ? static_cast<double>(A.nnz) / M : 1.0;
            rpb = static_cast<int>(128.0 * waves / std::max(avg, 1.0) + 0.5);
        }
        rpb = std::max(1, std::min(rpb, kRpCap));
        args.rows_per_block = rpb;
        grid = ceil_div(M, rpb);
    }
    hipError_t e;
    if (vec == 4) {
        e = dispatch_waves_unroll<4>(waves, unroll, args, grid, stream);
    } else if (vec == 2) {
        e = dispatch_waves_unroll<2>(waves, unroll, args, grid, stream);
    } else {
        e = dispatch_waves_unroll<1>(waves, unroll, args, grid, stream);
    }
    return from_hip(e, "csr engine launch");
}

}  // namespace engine
}  // namespace spmm
