// BSR (16x16 fp16 blocks) x dense fp16 B on gfx950 matrix cores, and the
// fp32 -> fp16 conversion (roles of spmm_wmma and float_to_half,
// spmm_wmma.cu:18-23 and :49-117).
//
// MFMA operand layout used (v_mfma_f32_16x16x32_f16, wave64, lane = 16*g + t):
//   A operand: lane holds A[t][kmap(g, 0..7)]       (8 fp16)
//   B operand: lane holds B[kmap(g, 0..7)][t]       (8 fp16)
//   D        : lane holds D[4*g + i][t], i = 0..3   (4 fp32)
// kmap(g, i) = 8*g + i.  The contraction only needs A and B to use the same
// kmap, so blocks pair up as: g = 0,1 -> block b (its columns 8*g .. 8*g+7),
// g = 2,3 -> block b+1.
//
// B is K-contiguous in the operand but N-contiguous in memory, so each wave
// stages the 32 B rows of a block pair (its 16*J columns) in LDS with plain
// 16-byte row loads and reads the operand back column-wise.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "engine.h"
#include "spmm/utils.h"

typedef unsigned spmm_u32x4 __attribute__((ext_vector_type(4)));

// Structured buffer load (LLVM's AMDGPU intrinsic; index = record, offset =
// byte offset inside the record).  The intrinsic name is fixed by LLVM.
__device__ spmm_u32x4 sbuf_load_u32x4(__amdgpu_buffer_rsrc_t rsrc, int index, int offset,
                                      int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");
// Structured buffer load straight into LDS: every lane's `size` bytes land at
// the LDS address p + 16 * lane (gfx950 LDS DMA), nothing passes through VGPRs.
typedef __attribute__((address_space(3))) void* spmm_lds_ptr;
__device__ void sbuf_load_lds(__amdgpu_buffer_rsrc_t rsrc, spmm_lds_ptr p, int size, int index,
                              int offset, int soffset, int imm_offset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.lds");

namespace spmm {
namespace engine {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// fp32 -> fp16 (round to nearest even), 8 elements per lane on the aligned body.
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ src,
                                                         _Float16* __restrict__ dst, long n,
                                                         int vector_ok) {
    const long tid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (vector_ok) {
        const long i = tid * 8;
        if (i + 8 <= n) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(src + i);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(src + i + 4);
            f16x8 h;
            h[0] = static_cast<_Float16>(lo[0]);
            h[1] = static_cast<_Float16>(lo[1]);
            h[2] = static_cast<_Float16>(lo[2]);
            h[3] = static_cast<_Float16>(lo[3]);
            h[4] = static_cast<_Float16>(hi[0]);
            h[5] = static_cast<_Float16>(hi[1]);
            h[6] = static_cast<_Float16>(hi[2]);
            h[7] = static_cast<_Float16>(hi[3]);
            *reinterpret_cast<f16x8*>(dst + i) = h;
        } else {
            for (long e = i; e < n; ++e) dst[e] = static_cast<_Float16>(src[e]);
        }
    } else if (tid < n) {
        dst[tid] = static_cast<_Float16>(src[tid]);
    }
}

// C is written once and not read back by the kernel: streaming stores keep
// it from displacing A and B in L2 (measured on c4: 7.8 -> 7.5 us).
__device__ __forceinline__ void store_c(float* p, float v) { __builtin_nontemporal_store(v, p); }

struct BsrArgs {
    const int*      row_ptr;
    const int*      col_idx;
    const _Float16* vals;
    const _Float16* B;
    float*          C;
    int             M;
    int             K;
    int             N;
    int             block_rows;
    int             b_vec_ok;  // N % 8 == 0 and B 16-byte aligned
    int             block_cols;
    int             tiles_n;    // wave kernel: column tiles (grid is 1-D)
    int             wg_total;   // wave kernel: workgroups launched
    int             xcd_order;  // wave kernel: 1 = XCD-grouped workgroup order
    int             num_blocks;
};

// Workgroup -> (block-row group, column tile) for the 1-D wave-kernel grid.
// The hardware hands workgroup L to XCD L % 8.  With xcd_order, XCD x gets
// the contiguous logical range [x*T/8, (x+1)*T/8) (the first T % 8 XCDs one
// more), and logical ids run column tile fastest: each XCD works on its own
// band of block-rows with all their column tiles, so A blocks and the B rows
// that neighbouring block-rows share are fetched into one L2 only.
__device__ __forceinline__ void wave_tile_of(const BsrArgs& a, int& bx, int& by) {
    const int L = blockIdx.x;
    int l = L;
    if (a.xcd_order) {
        const int xcd = L & 7, idx = L >> 3;
        const int per = a.wg_total >> 3, rem = a.wg_total & 7;
        l = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    }
    bx = l / a.tiles_n;
    by = l - bx * a.tiles_n;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16.  Within each 16-lane block, lane s supplies the address
// of 4 consecutive fp16 values and output lane i receives element i % 4 of
// the values addressed by lanes 4e + i/4, e = 0..3: with lane s pointing at
// row s/4, columns 4*(s%4) .. +3 of a row-major [k][n] tile, lane i gets
// rows 0..3 of column i -- a K-contiguous MFMA B operand.
__device__ __forceinline__ s16x4 lds_read_tr16(const _Float16* p) {
    // generic -> LDS address-space cast; p always points into a __shared__ array
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(const_cast<_Float16*>(p)));
}

// ---------------------------------------------------------------------------
// Wave kernel (the default path): one wave = one block-row x 16*J columns,
// four independent waves per workgroup, no workgroup barriers.  Maximum
// parallelism and a small LDS footprint (one 32 x (16J+16) fp16 tile per
// wave) keep many waves resident, which is what hides the latency of the
// short dependent chain row_ptr -> col_idx -> (A, B) -> MFMA.
//   - The block-row's block-columns come in with one vector load (lane i
//     holds col_idx[first + i], 64 per chunk) and are broadcast with
//     v_readlane, so pairs need no further index loads.
//   - The A operands and B rows of the next D pairs are in flight while a
//     pair is multiplied (a ring of D register sets).
//   - B rows are written to the wave's LDS tile row-major (16-byte stores) and
//     read back as MFMA operands with ds_read_b64_tr_b16 (two per operand).
// LDS accesses of one wave execute in program order, so the single tile
// needs no barrier between a pair's reads and the next pair's writes.
// ---------------------------------------------------------------------------
template <int J, int D, bool VEC>
__global__ __launch_bounds__(256) void bsr_wave_kernel(BsrArgs a) {
    constexpr int NT  = 16 * J;          // columns per wave
    constexpr int S   = NT + 16;         // LDS row stride in fp16 (S/2 = 8 mod 32 banks)
    constexpr int CH  = NT / 8;          // 16-byte chunks per staged row
    constexpr int CPL = 32 * CH / 64;    // chunks per lane (J for the 32-row tile)
    __shared__ __attribute__((aligned(16))) _Float16 s_b[4][32 * S];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g    = lane >> 4;
    const int t    = lane & 15;
    int bx, by;
    wave_tile_of(a, bx, by);
    const int br   = bx * 4 + wave;
    const int n0   = by * NT;
    if (br >= a.block_rows) return;  // waves are independent: no barrier anywhere
    _Float16* tile = s_b[wave];

    const int bs = a.row_ptr[br];
    const int be = a.row_ptr[br + 1];

    f32x4 acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = f32x4(0.0f);

    // Registers of one pair: this lane's B chunks and A operand, and which of
    // them hold data.  Loads never branch: a lane whose row lies outside B
    // (past K, or the absent second block of an odd tail) reads a clamped,
    // valid address and its value is replaced by zero when it is used, so the
    // loads of all pairs in flight stay independent of each other.
    struct PairRegs {
        f16x8 b[CPL];
        f16x8 af;
        bool  b_ok[CPL];
        bool  a_ok;
    };
    // Pair = blocks base+p and base+p+1 of the row (p and p+1 inside the
    // column-index chunk ci that starts at block base).
    auto load_pair = [&](int base, int p, int cnt, int ci, PairRegs& r) {
        const bool two = p + 1 < cnt;
        const int bc0 = __builtin_amdgcn_readlane(ci, p);
        const int bc1 = __builtin_amdgcn_readlane(ci, two ? p + 1 : p);
        const int blk = base + p;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = lane + c * 64;
            const int s   = idx / CH;                 // staged row 0..31
            const int k   = (s < 16 ? bc0 : bc1) * 16 + (s & 15);
            const int n   = n0 + (idx % CH) * 8;
            const bool ok = (s < 16 || two) && k < a.K && n < a.N;
            r.b_ok[c] = ok;
            if constexpr (VEC) {
                const size_t off = ok ? static_cast<size_t>(k) * a.N + n : 0;
                r.b[c] = *reinterpret_cast<const f16x8*>(a.B + off);
            } else {
                const size_t row = ok ? static_cast<size_t>(k) * a.N : 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool in = ok && n + e < a.N;
                    const _Float16 x = a.B[in ? row + n + e : 0];
                    r.b[c][e] = in ? x : static_cast<_Float16>(0.0f);
                }
            }
        }
        // A operand: row t of block blk (g < 2) or blk+1 (g >= 2), columns 8*(g&1) .. +7
        r.a_ok = g < 2 || two;
        r.af = *reinterpret_cast<const f16x8*>(
            a.vals + static_cast<size_t>(blk + (r.a_ok ? (g >> 1) : 0)) * 256 + t * 16 +
            8 * (g & 1));
    };
    auto multiply = [&](const PairRegs& r) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = lane + c * 64;
            const f16x8 zero = f16x8(static_cast<_Float16>(0.0f));
            *reinterpret_cast<f16x8*>(&tile[(idx / CH) * S + (idx % CH) * 8]) =
                r.b_ok[c] ? r.b[c] : zero;
        }
        const f16x8 af = r.a_ok ? r.af : f16x8(static_cast<_Float16>(0.0f));
        const _Float16* rowp = &tile[(8 * g + (t >> 2)) * S + 4 * (t & 3)];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const s16x4 lo = lds_read_tr16(rowp + 16 * j);
            const s16x4 hi = lds_read_tr16(rowp + 4 * S + 16 * j);
            const s16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(f16x8, both),
                                                             acc[j], 0, 0, 0);
        }
    };

    // D pairs in flight.  Pair i of a chunk lives in ring slot i % D.  The
    // steady-state loop refills every slot it empties, so each slot's loads
    // are issued unconditionally and the wait before a multiply covers only
    // that slot's loads; the drain finishes the last (fewer than 2D) pairs.
    for (int c0 = bs; c0 < be; c0 += 64) {  // 64 blocks per column-index chunk
        const int cnt = min(64, be - c0);
        const int np  = (cnt + 1) >> 1;     // pairs in this chunk
        const int ci  = lane < cnt ? a.col_idx[c0 + lane] : 0;
        PairRegs ring[D];
#pragma unroll
        for (int d = 0; d < D; ++d) load_pair(c0, 2 * min(d, np - 1), cnt, ci, ring[d]);
        int i0 = 0;
        for (; i0 + 2 * D <= np; i0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                multiply(ring[d]);
                load_pair(c0, 2 * (i0 + d + D), cnt, ci, ring[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + d < np) {
                multiply(ring[d]);
                if (i0 + d + D < np) load_pair(c0, 2 * (i0 + d + D), cnt, ci, ring[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + D + d < np) multiply(ring[d]);
        }
    }

    // D layout: lane holds rows 4*g + i, column t of each 16-column tile.
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int col = n0 + 16 * j + t;
        if (col >= a.N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = br * 16 + 4 * g + i;
            if (row < a.M) store_c(a.C + static_cast<size_t>(row) * a.N + col, acc[j][i]);
        }
    }
}

// ---------------------------------------------------------------------------
// Record-addressed wave kernel (the default where it applies): the wave
// kernel's work split and ring, with B and the A blocks read as structured
// buffers -- one record per B row (N fp16) and one per 16x16 block.  The row
// or block number is the load's index operand, and the buffer range check
// returns zeros for an index past the end: rows >= K of a partial last
// block-column, and index -1 for the absent second block of an odd tail.  So
// a pair needs one index add per 16-byte chunk instead of 64-bit address
// arithmetic and per-lane zero selects (~30 -> ~6 vector instructions per
// pair).  The B rows of a pair go straight into the wave's LDS slot with
// buffer-to-LDS loads (no VGPR staging, no ds_write), one slot per pair in
// flight, each slot its own LDS object.  Measured on MI355X against the same
// kernel staging through VGPRs and ds_write (both at their default tiles):
// banded 8192^2 N=128 4.3 -> 4.1 us, block-diagonal 8192^2 N=256 6.4 -> 6.1
// us, identical results.  Needs N % 8 == 0 with 16-byte aligned B, N * 2 <= 16383 (record
// stride field), and B and A within 2 GiB each.
// ---------------------------------------------------------------------------
__device__ u32x4 sbuf_load_u32x4_dev(__amdgpu_buffer_rsrc_t rsrc, int index, int offset) {
    return sbuf_load_u32x4(rsrc, index, offset, 0, 0);
}

// Third dword of a gfx9 buffer resource: 32-bit data format, no swizzle.
constexpr int kBufWord3 = 0x00020000;

// s_waitcnt constraining only the vector-memory count (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    __builtin_amdgcn_sched_barrier(0);
}

template <int J, int D>
__device__ __forceinline__ void bsr_record_body(const BsrArgs& a, _Float16* __restrict__ s0,
                                                _Float16* __restrict__ s1,
                                                _Float16* __restrict__ s2,
                                                _Float16* __restrict__ s3) {
    constexpr int NT   = 16 * J;       // columns per wave
    constexpr int CH   = NT / 8;       // 16-byte chunks per staged row
    constexpr int CPL  = 32 * CH / 64; // chunks per lane (one load instruction each)
    constexpr int TILE = 32 * NT;      // fp16 per slot: the pair's 32 B rows, row-major
    constexpr int PER  = CPL + 1;      // vector-memory instructions per pair

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g    = lane >> 4;
    const int t    = lane & 15;
    int bx, by;
    wave_tile_of(a, bx, by);
    const int br   = bx * 4 + wave;
    const int n0   = by * NT;
    if (br >= a.block_rows) return;  // waves are independent: no barrier anywhere
    auto slot = [&](int d) -> _Float16* {
        return (d == 0 ? s0 : d == 1 ? s1 : d == 2 ? s2 : s3) + wave * TILE;
    };

    const __amdgpu_buffer_rsrc_t rec_b = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a.B), static_cast<short>(a.N * 2), a.K, kBufWord3);
    const __amdgpu_buffer_rsrc_t rec_a = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a.vals), static_cast<short>(512), a.num_blocks, kBufWord3);

    // Lane constants: load instruction c moves 16-byte chunk idx = lane + 64c,
    // staged row srow (block srow >= 16 of the pair), columns n .. n+7 at byte
    // offset nbyte of its B row, to slot offset 8 * idx fp16 (row-major).
    // Columns past N read a valid chunk of the row instead; their products
    // land in output columns >= N, which are never stored.
    int srow[CPL], nbyte[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = lane + c * 64;
        srow[c] = idx / CH;
        const int n = n0 + (idx % CH) * 8;
        nbyte[c] = (n < a.N ? n : 0) * 2;
    }
    // A operand: row t of block (first, g < 2) or (second, g >= 2), columns 8*(g&1) .. +7
    const int a_off = t * 32 + 16 * (g & 1);
    const int a_hi  = g >> 1;

    const int bs = a.row_ptr[br];
    const int be = a.row_ptr[br + 1];

    f32x4 acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = f32x4(0.0f);

    u32x4 af[D];
    // Pair = blocks base+p and base+p+1 of the row (p and p+1 inside the
    // column-index chunk ci that starts at block base), into ring slot d.
    auto load_pair = [&](int d, int base, int p, int cnt, int ci) {
        const bool two = p + 1 < cnt;
        const int bc0 = __builtin_amdgcn_readlane(ci, p);
        const int bc1 = two ? __builtin_amdgcn_readlane(ci, p + 1) : -1;  // rows -16..-1: zeros
        _Float16* dst = slot(d);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int sr = srow[c];
            sbuf_load_lds(rec_b, (spmm_lds_ptr)(dst + c * 512), 16,
                          (sr < 16 ? bc0 : bc1) * 16 + (sr & 15), nbyte[c], 0, 0, 0);
        }
        af[d] = sbuf_load_u32x4_dev(rec_a, (two || a_hi == 0) ? base + p + a_hi : -1, a_off);
    };
    auto multiply = [&](int d) {
        const f16x8 afv = __builtin_bit_cast(f16x8, af[d]);
        const _Float16* rowp = slot(d) + (8 * g + (t >> 2)) * NT + 4 * (t & 3);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const s16x4 lo = lds_read_tr16(rowp + 16 * j);
            const s16x4 hi = lds_read_tr16(rowp + 4 * NT + 16 * j);
            const s16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afv, __builtin_bit_cast(f16x8, both),
                                                             acc[j], 0, 0, 0);
        }
    };

    // D pairs in flight.  Vector-memory instructions retire in issue order,
    // so before slot d is read, waiting until at most (D-1) pairs' loads are
    // outstanding guarantees slot d's are done.  A slot is refilled only after
    // the MFMAs that consumed its reads, so its reads are complete by then.
    // The drain (fewer loads after each slot) waits for everything.
    for (int c0 = bs; c0 < be; c0 += 64) {  // 64 blocks per column-index chunk
        const int cnt = min(64, be - c0);
        const int np  = (cnt + 1) >> 1;
        const int ci  = lane < cnt ? a.col_idx[c0 + lane] : 0;
#pragma unroll
        for (int d = 0; d < D; ++d) load_pair(d, c0, 2 * min(d, np - 1), cnt, ci);
        int i0 = 0;
        for (; i0 + 2 * D <= np; i0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                wait_vmcnt<(D - 1) * PER>();
                multiply(d);
                load_pair(d, c0, 2 * (i0 + d + D), cnt, ci);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + d < np) {
                wait_vmcnt<0>();
                multiply(d);
                if (i0 + d + D < np) load_pair(d, c0, 2 * (i0 + d + D), cnt, ci);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + D + d < np) {
                wait_vmcnt<0>();
                multiply(d);
            }
        }
    }

    // D layout: lane holds rows 4*g + i, column t of each 16-column tile.
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int col = n0 + 16 * j + t;
        if (col >= a.N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = br * 16 + 4 * g + i;
            if (row < a.M) store_c(a.C + static_cast<size_t>(row) * a.N + col, acc[j][i]);
        }
    }
}

// The ring slots are separate LDS objects passed as restrict pointers: after
// inlining, every slot access carries its own alias scope, which lets the
// compiler's wait-count pass tell a read of slot d from the buffer-to-LDS
// writes still in flight into the other slots.
template <int J, int D>
__global__ __launch_bounds__(256) void bsr_record_kernel(BsrArgs a) {
    constexpr int TILE = 32 * 16 * J;
    static_assert(D == 2 || D == 4, "ring depth 2 or 4");
    __shared__ __attribute__((aligned(16))) _Float16 s_b0[4 * TILE];
    __shared__ __attribute__((aligned(16))) _Float16 s_b1[4 * TILE];
    __shared__ __attribute__((aligned(16))) _Float16 s_b2[D == 4 ? 4 * TILE : 8];
    __shared__ __attribute__((aligned(16))) _Float16 s_b3[D == 4 ? 4 * TILE : 8];
    bsr_record_body<J, D>(a, s_b0, s_b1, s_b2, s_b3);
}

// ---------------------------------------------------------------------------
// Multi-row wave kernel: one wave = R consecutive block-rows x 16*J columns.
// The wave walks the union of the R block-rows' (sorted) block-column lists
// with R scalar cursors; every union pair's 32 B rows are loaded and staged
// in LDS once and feed R MFMAs (one per block-row, zero A where a block-row
// has no block at that column).  Neighbouring block-rows of banded and
// block-diagonal matrices share most block-columns, so B traffic through the
// CU and LDS falls by up to R without any workgroup barrier.
//   - The R block-rows' blocks are contiguous in col_idx; when they total at
//     most 64 they come in with one vector load and are merged in one
//     segment.  Longer ones are taken block-row by block-row in chunks of 64
//     (the other cursors empty).
//   - The union cursor advances inside load_pair, so pairs are produced in
//     order; loads are unconditional (exhausted cursors give masked loads of
//     clamped valid addresses), as in the wave kernel.
// ---------------------------------------------------------------------------
template <int R, int J, int D, bool VEC>
struct MultirowWave {
    static constexpr int NT  = 16 * J;
    static constexpr int S   = NT + 16;
    static constexpr int CH  = NT / 8;
    static constexpr int CPL = 32 * CH / 64;
    static constexpr int kNone = 0x7fffffff;

    struct PairRegs {
        f16x8 b[CPL];
        f16x8 af[R];
        bool  b_ok[CPL];
        bool  a_ok[R];
        bool  valid;  // wave-uniform: the pair holds at least one union element
    };

    const BsrArgs& a;
    _Float16*      tile;
    int            lane, g, t, n0;
    f32x4          acc[R][J];
    // Current segment: lanes [0, cnt) of ci hold col_idx[base + lane]; list r
    // (block-row r) is lanes [cur[r], end[r]).
    int            base, ci;
    int            cur[R], end[R];

    __device__ MultirowWave(const BsrArgs& args, _Float16* t_, int n0_) : a(args), tile(t_), n0(n0_) {
        lane = threadIdx.x & 63;
        g    = lane >> 4;
        t    = lane & 15;
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < J; ++j) acc[r][j] = f32x4(0.0f);
        }
    }

    // Next union element: its block-column (-1 when the lists are exhausted)
    // and, per block-row, its block index (-1 where the block-row has none).
    __device__ void next_union(int& bc, int (&blk)[R]) {
        int c[R];
        int m = kNone;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int v = __builtin_amdgcn_readlane(ci, min(cur[r], 63));
            c[r] = cur[r] < end[r] ? v : kNone;
            m = min(m, c[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool has = m != kNone && c[r] == m;
            blk[r] = has ? base + cur[r] : -1;
            cur[r] += has ? 1 : 0;
        }
        bc = m == kNone ? -1 : m;
    }

    __device__ void load_pair(PairRegs& rg) {
        int bc0, bc1, blk0[R], blk1[R];
        next_union(bc0, blk0);
        next_union(bc1, blk1);
        rg.valid = bc0 >= 0;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = lane + c * 64;
            const int s   = idx / CH;
            const int bc  = s < 16 ? bc0 : bc1;
            const int k   = bc * 16 + (s & 15);
            const int n   = n0 + (idx % CH) * 8;
            const bool ok = bc >= 0 && k < a.K && n < a.N;
            rg.b_ok[c] = ok;
            if constexpr (VEC) {
                const size_t off = ok ? static_cast<size_t>(k) * a.N + n : 0;
                rg.b[c] = *reinterpret_cast<const f16x8*>(a.B + off);
            } else {
                const size_t row = ok ? static_cast<size_t>(k) * a.N : 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool in = ok && n + e < a.N;
                    const _Float16 x = a.B[in ? row + n + e : 0];
                    rg.b[c][e] = in ? x : static_cast<_Float16>(0.0f);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int blk = g < 2 ? blk0[r] : blk1[r];
            rg.a_ok[r] = blk >= 0;
            rg.af[r] = *reinterpret_cast<const f16x8*>(
                a.vals + static_cast<size_t>(blk >= 0 ? blk : base) * 256 + t * 16 + 8 * (g & 1));
        }
    }

    __device__ void multiply(const PairRegs& rg) {
        const f16x8 zero = f16x8(static_cast<_Float16>(0.0f));
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = lane + c * 64;
            *reinterpret_cast<f16x8*>(&tile[(idx / CH) * S + (idx % CH) * 8]) =
                rg.b_ok[c] ? rg.b[c] : zero;
        }
        const _Float16* rowp = &tile[(8 * g + (t >> 2)) * S + 4 * (t & 3)];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const s16x4 lo = lds_read_tr16(rowp + 16 * j);
            const s16x4 hi = lds_read_tr16(rowp + 4 * S + 16 * j);
            const s16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            const f16x8 bop = __builtin_bit_cast(f16x8, both);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const f16x8 af = rg.a_ok[r] ? rg.af[r] : zero;
                acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bop, acc[r][j], 0, 0, 0);
            }
        }
    }

    // Walks the union of the current segment's lists.  Every slot of the ring
    // is refilled unconditionally after its turn, so each iteration issues
    // the same loads and the wait before a multiply covers only that slot.
    // The union comes out in order: once slot 0 holds no union element, no
    // later pair does.
    __device__ void run_segment(int base_, int cnt) {
        base = base_;
        ci = lane < cnt ? a.col_idx[base + lane] : 0;
        PairRegs ring[D];
#pragma unroll
        for (int d = 0; d < D; ++d) load_pair(ring[d]);
        while (ring[0].valid) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (ring[d].valid) multiply(ring[d]);
                load_pair(ring[d]);
                // keep the slots' loads in issue order (the memory counter
                // retires in order): a slot's wait then covers only its own
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    __device__ void store(int br0) {
        // D layout: lane holds rows 4*g + i, column t of each 16-column tile.
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int br = br0 + r;
            if (br >= a.block_rows) break;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int col = n0 + 16 * j + t;
                if (col >= a.N) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = br * 16 + 4 * g + i;
                    if (row < a.M) store_c(a.C + static_cast<size_t>(row) * a.N + col, acc[r][j][i]);
                }
            }
        }
    }
};

template <int R, int J, int D, bool VEC>
__global__ __launch_bounds__(256) void bsr_multirow_kernel(BsrArgs a) {
    constexpr int S = 16 * J + 16;
    __shared__ __attribute__((aligned(16))) _Float16 s_b[4][32 * S];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int bx, by;
    wave_tile_of(a, bx, by);
    const int br0 = (bx * 4 + wave) * R;
    if (br0 >= a.block_rows) return;  // waves are independent: no barrier anywhere
    MultirowWave<R, J, D, VEC> w(a, s_b[wave], by * 16 * J);

    int rp[R + 1];
#pragma unroll
    for (int r = 0; r <= R; ++r) rp[r] = a.row_ptr[min(br0 + r, a.block_rows)];
    const int tot = rp[R] - rp[0];
    if (tot <= 64) {
        // the R block-rows' blocks are contiguous: one segment, all lists
#pragma unroll
        for (int r = 0; r < R; ++r) {
            w.cur[r] = rp[r] - rp[0];
            w.end[r] = rp[r + 1] - rp[0];
        }
        if (tot > 0) w.run_segment(rp[0], tot);
    } else {
        // block-row by block-row in chunks of 64 blocks (other lists empty)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            for (int c0 = rp[r]; c0 < rp[r + 1]; c0 += 64) {
                const int cnt = min(64, rp[r + 1] - c0);
#pragma unroll
                for (int q = 0; q < R; ++q) {
                    w.cur[q] = 0;
                    w.end[q] = q == r ? cnt : 0;
                }
                w.run_segment(c0, cnt);
            }
        }
    }
    w.store(br0);
}

// ---------------------------------------------------------------------------
// Split-K wave kernel: a workgroup of 4 waves owns one block-row x 16*J
// columns; wave w multiplies the block pairs p = w, w+4, w+8, ... of the
// block-row (pairs of consecutive blocks, as in the wave kernel), so each
// wave's dependent chain is a quarter as long and four times as many waves
// are in flight.  The four partial tiles are summed through LDS after one
// workgroup barrier; wave w adds rows 4w .. 4w+3 of the tile and stores them.
// ---------------------------------------------------------------------------
template <int J, int D, bool VEC>
__global__ __launch_bounds__(256) void bsr_splitk_kernel(BsrArgs a) {
    constexpr int NT  = 16 * J;
    constexpr int S   = NT + 16;
    constexpr int CH  = NT / 8;
    constexpr int CPL = 32 * CH / 64;
    __shared__ __attribute__((aligned(16))) _Float16 s_b[4][32 * S];
    __shared__ float s_part[4][16][NT + 1];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g    = lane >> 4;
    const int t    = lane & 15;
    int bx, by;
    wave_tile_of(a, bx, by);
    const int br = bx;  // grid = block_rows x column tiles: always a valid block-row
    const int n0 = by * NT;
    _Float16* tile = s_b[wave];
    const int bs = a.row_ptr[br];
    const int be = a.row_ptr[br + 1];

    f32x4 acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = f32x4(0.0f);

    struct PairRegs {
        f16x8 b[CPL];
        f16x8 af;
        bool  b_ok[CPL];
        bool  a_ok;
    };
    // pair q of the chunk = blocks 2q and 2q+1 of chunk ci (which starts at block base)
    auto load_pair = [&](int base, int q, int cnt, int ci, PairRegs& r) {
        const int p = min(2 * q, cnt - 1);  // clamped past the end: masked below
        const bool live = 2 * q < cnt;
        const bool two = live && p + 1 < cnt;
        const int bc0 = __builtin_amdgcn_readlane(ci, p);
        const int bc1 = __builtin_amdgcn_readlane(ci, two ? p + 1 : p);
        const int blk = base + p;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = lane + c * 64;
            const int s   = idx / CH;
            const int k   = (s < 16 ? bc0 : bc1) * 16 + (s & 15);
            const int n   = n0 + (idx % CH) * 8;
            const bool ok = live && (s < 16 || two) && k < a.K && n < a.N;
            r.b_ok[c] = ok;
            if constexpr (VEC) {
                const size_t off = ok ? static_cast<size_t>(k) * a.N + n : 0;
                r.b[c] = *reinterpret_cast<const f16x8*>(a.B + off);
            } else {
                const size_t row = ok ? static_cast<size_t>(k) * a.N : 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool in = ok && n + e < a.N;
                    const _Float16 x = a.B[in ? row + n + e : 0];
                    r.b[c][e] = in ? x : static_cast<_Float16>(0.0f);
                }
            }
        }
        r.a_ok = live && (g < 2 || two);
        r.af = *reinterpret_cast<const f16x8*>(
            a.vals + static_cast<size_t>(blk + (r.a_ok ? (g >> 1) : 0)) * 256 + t * 16 +
            8 * (g & 1));
    };
    auto multiply = [&](const PairRegs& r) {
        const f16x8 zero = f16x8(static_cast<_Float16>(0.0f));
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = lane + c * 64;
            *reinterpret_cast<f16x8*>(&tile[(idx / CH) * S + (idx % CH) * 8]) =
                r.b_ok[c] ? r.b[c] : zero;
        }
        const f16x8 af = r.a_ok ? r.af : zero;
        const _Float16* rowp = &tile[(8 * g + (t >> 2)) * S + 4 * (t & 3)];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const s16x4 lo = lds_read_tr16(rowp + 16 * j);
            const s16x4 hi = lds_read_tr16(rowp + 4 * S + 16 * j);
            const s16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(f16x8, both),
                                                             acc[j], 0, 0, 0);
        }
    };

    for (int c0 = bs; c0 < be; c0 += 64) {
        const int cnt = min(64, be - c0);
        const int np  = (cnt + 1) >> 1;
        const int mine = np > wave ? (np - wave + 3) >> 2 : 0;  // pairs wave, wave+4, ...
        if (mine == 0) continue;
        const int ci = lane < cnt ? a.col_idx[c0 + lane] : 0;
        PairRegs ring[D];
#pragma unroll
        for (int d = 0; d < D; ++d) load_pair(c0, wave + 4 * d, cnt, ci, ring[d]);
        int i0 = 0;
        for (; i0 + 2 * D <= mine; i0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                multiply(ring[d]);
                load_pair(c0, wave + 4 * (i0 + d + D), cnt, ci, ring[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + d < mine) {
                multiply(ring[d]);
                if (i0 + d + D < mine) load_pair(c0, wave + 4 * (i0 + d + D), cnt, ci, ring[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (i0 + D + d < mine) multiply(ring[d]);
        }
    }

    // Partial tiles -> LDS (lane holds rows 4g+i, column 16j+t), one barrier,
    // then wave w sums rows 4w .. 4w+3 over the four partials.
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s_part[wave][4 * g + i][16 * j + t] = acc[j][i];
    }
    __syncthreads();
    for (int e = lane; e < 4 * NT; e += 64) {
        const int lr  = 4 * wave + e / NT;
        const int col = e % NT;
        const float v = s_part[0][lr][col] + s_part[1][lr][col] + s_part[2][lr][col] +
                        s_part[3][lr][col];
        const int row = br * 16 + lr;
        if (row < a.M && n0 + col < a.N) store_c(a.C + static_cast<size_t>(row) * a.N + n0 + col, v);
    }
}

// ---------------------------------------------------------------------------
// Row-group kernel.
//
// A workgroup of RG waves owns RG consecutive block-rows (one per wave) and
// a tile of NT = 16*J columns.  It first ORs the block-columns of its
// block-rows into an LDS bitmap, then walks that union in ascending pairs
// (bc0, bc1): each pair's 32 B rows x NT columns are loaded once into LDS,
// row-major, with 16-byte loads, and every wave that owns a block at bc0 or
// bc1 multiplies it by the staged rows.  Block-rows with shared block-columns
// (banded, block-diagonal) therefore read each B tile once per workgroup
// instead of once per block-row.
//
// The B operand is read back with ds_read_b64_tr_b16, which returns the
// transpose of a 4 (k) x 16 (n) fp16 tile to each 16-lane block: lane s of the
// block addresses row 8g + s/4 (+4 for the second read), columns 4*(s%4) ..
// +3, and lane t receives rows 8g .. 8g+3 (8g+4 .. 8g+7) of column t, i.e. the
// K-contiguous B operand of v_mfma_f32_16x16x32_f16.
//
// Pairs are processed in batches of P: all B tiles and A operands of a batch
// are requested into registers before any is used, then stored to P LDS
// tiles, so a batch costs one memory latency instead of one per pair.
// ---------------------------------------------------------------------------
constexpr int kMaxUnionWords = 2048;  // union bitmap of up to 65536 block-columns

template <int RG, int J, int P>
__global__ __launch_bounds__(RG * 64) void bsr_rowgroup_kernel(BsrArgs a) {
    constexpr int NT          = 16 * J;      // columns per workgroup
    constexpr int S           = NT + 16;     // LDS row stride in fp16: S/2 = 8 (mod 32) banks
    constexpr int CH          = NT / 8;      // 16-byte chunks per staged row
    constexpr int TILE_CHUNKS = 32 * CH;
    constexpr int THREADS     = RG * 64;
    constexpr int CPT         = (TILE_CHUNKS + THREADS - 1) / THREADS;  // chunks per thread

    // Dynamic LDS: P tiles of 32 x S fp16 (one per pair of a batch), then the
    // union bitmap sized to the matrix's block-columns.
    extern __shared__ __attribute__((aligned(16))) unsigned char s_dyn[];
    _Float16 (*s_b)[32 * S] = reinterpret_cast<_Float16 (*)[32 * S]>(s_dyn);
    uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_dyn + sizeof(_Float16) * P * 32 * S);

    const int tid    = threadIdx.x;
    const int lane   = tid & 63;
    const int wave   = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g      = lane >> 4;
    const int t      = lane & 15;
    const int br     = blockIdx.x * RG + wave;
    const int n0     = blockIdx.y * NT;
    const int nwords = (a.block_cols + 31) / 32;

    int bs = 0, be = 0;
    if (br < a.block_rows) {
        bs = a.row_ptr[br];
        be = a.row_ptr[br + 1];
    }
    // this wave's own block list, 64 block-columns per register chunk; the
    // first chunk also feeds the union below
    int ptr = bs, chunk = bs;
    int my_col = (bs + lane < be) ? a.col_idx[bs + lane] : 0x7fffffff;

    // ---- union of the group's block-columns
    for (int i = tid; i < nwords; i += THREADS) s_bits[i] = 0u;
    __syncthreads();
    for (int b = bs + lane; b < be; b += 64) {
        const int bc = b - bs < 64 ? my_col : a.col_idx[b];
        if (static_cast<unsigned>(bc) < static_cast<unsigned>(a.block_cols)) {
            atomicOr(&s_bits[bc >> 5], 1u << (bc & 31));
        }
    }
    __syncthreads();

    auto current_col = [&]() -> int {
        if (ptr >= be) return 0x7fffffff;
        if (ptr - chunk >= 64) {
            chunk = ptr;
            my_col = (ptr + lane < be) ? a.col_idx[ptr + lane] : 0x7fffffff;
        }
        return __builtin_amdgcn_readlane(my_col, ptr - chunk);
    };

    // ---- cursor over the union (identical in every thread)
    int cw = -1;
    uint32_t cbits = 0u;
    auto next_col = [&]() -> int {
        while (cbits == 0u) {
            if (++cw >= nwords) return -1;
            cbits = s_bits[cw];
        }
        const int b = __builtin_ctz(cbits);
        cbits &= cbits - 1u;
        return cw * 32 + b;
    };

    auto load_tile = [&](int bc0, int bc1, f16x8 (&r)[CPT]) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int idx = tid + c * THREADS;
            f16x8 v = f16x8(static_cast<_Float16>(0.0f));
            if (idx < TILE_CHUNKS) {
                const int s  = idx / CH;
                const int bc = s < 16 ? bc0 : bc1;
                const int k  = bc * 16 + (s & 15);
                const int n  = n0 + (idx % CH) * 8;
                if (bc >= 0 && k < a.K && n < a.N) {
                    const _Float16* src = a.B + static_cast<size_t>(k) * a.N + n;
                    if (a.b_vec_ok && n + 8 <= a.N) {
                        v = *reinterpret_cast<const f16x8*>(src);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            if (n + e < a.N) v[e] = src[e];
                        }
                    }
                }
            }
            r[c] = v;
        }
    };
    auto store_tile = [&](int buf, const f16x8 (&r)[CPT]) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int idx = tid + c * THREADS;
            if (idx < TILE_CHUNKS) {
                *reinterpret_cast<f16x8*>(&s_b[buf][(idx / CH) * S + (idx % CH) * 8]) = r[c];
            }
        }
    };
    // A operand of this wave for the pair; consumes the wave's matching blocks.
    auto load_a = [&](int bc0, int bc1, bool& any) -> f16x8 {
        int blk0 = -1, blk1 = -1;
        if (current_col() == bc0) blk0 = ptr++;
        if (bc1 >= 0 && current_col() == bc1) blk1 = ptr++;
        any = blk0 >= 0 || blk1 >= 0;
        const int blk = g < 2 ? blk0 : blk1;
        f16x8 af = f16x8(static_cast<_Float16>(0.0f));
        if (blk >= 0) {
            af = *reinterpret_cast<const f16x8*>(a.vals + static_cast<size_t>(blk) * 256 + t * 16 +
                                                 8 * (g & 1));
        }
        return af;
    };

    f32x4 acc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = f32x4(0.0f);

    // Batches of up to P pairs: every B tile and A operand of a batch is
    // requested before any is used, so a batch costs one memory latency.
    while (true) {
        int bcl[2 * P];
        int npairs = 0;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            bcl[2 * p]     = next_col();
            bcl[2 * p + 1] = bcl[2 * p] >= 0 ? next_col() : -1;
            npairs += bcl[2 * p] >= 0 ? 1 : 0;
        }
        if (npairs == 0) break;  // uniform across the workgroup

        f16x8 treg[P][CPT];
        f16x8 af[P];
        bool  any[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            any[p] = false;
            af[p]  = f16x8(static_cast<_Float16>(0.0f));
            if (p < npairs) {
                load_tile(bcl[2 * p], bcl[2 * p + 1], treg[p]);
                af[p] = load_a(bcl[2 * p], bcl[2 * p + 1], any[p]);
            }
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (p < npairs) store_tile(p, treg[p]);
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (p < npairs && any[p]) {
                const _Float16* rowp = &s_b[p][(8 * g + (t >> 2)) * S + 4 * (t & 3)];
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const s16x4 lo = lds_read_tr16(rowp + 16 * j);
                    const s16x4 hi = lds_read_tr16(rowp + 4 * S + 16 * j);
                    const s16x8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        af[p], __builtin_bit_cast(f16x8, both), acc[j], 0, 0, 0);
                }
            }
        }
        if (npairs < P) break;
        __syncthreads();  // the next batch overwrites the tiles
    }

    if (br < a.block_rows) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int col = n0 + 16 * j + t;
            if (col >= a.N) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = br * 16 + 4 * g + i;
                if (row < a.M) store_c(a.C + static_cast<size_t>(row) * a.N + col, acc[j][i]);
            }
        }
    }
}

Error fail(int status, std::string msg) { return Error{status, std::move(msg)}; }

Error from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return Error{};
    return fail(kHipError, std::string(what) + ": " + hipGetErrorString(e));
}

// B rows and A blocks fit structured-buffer records: the record stride field
// holds at most 16383 bytes and each buffer must stay within 2 GiB.
bool records_fit(const BsrArgs& a) {
    return a.b_vec_ok && static_cast<long long>(a.N) * 2 <= 16383 &&
           static_cast<long long>(a.K) * a.N * 2 <= 0x7fffffffLL &&
           static_cast<long long>(a.num_blocks) * 512 <= 0x7fffffffLL;
}

template <int J, int D>
hipError_t run_wave(BsrArgs args, hipStream_t stream, bool pointer_addressing) {
    args.tiles_n = ceil_div(args.N, 16 * J);
    const long total = static_cast<long>(ceil_div(args.block_rows, 4)) * args.tiles_n;
    if (total > 0x7fffffffL) return hipErrorInvalidConfiguration;
    args.wg_total = static_cast<int>(total);
    dim3 grid(args.wg_total);
    if (!pointer_addressing && records_fit(args)) {
        hipLaunchKernelGGL((bsr_record_kernel<J, D == 1 ? 2 : D>), grid, dim3(256), 0, stream,
                           args);
        return hipGetLastError();
    }
    if (args.b_vec_ok) {
        hipLaunchKernelGGL((bsr_wave_kernel<J, D, true>), grid, dim3(256), 0, stream, args);
    } else {
        hipLaunchKernelGGL((bsr_wave_kernel<J, D, false>), grid, dim3(256), 0, stream, args);
    }
    return hipGetLastError();
}

template <int J>
hipError_t dispatch_wave(int depth, bool pointer_addressing, const BsrArgs& args,
                         hipStream_t stream) {
    return depth == 1 ? run_wave<J, 1>(args, stream, pointer_addressing)
                      : (depth == 2 ? run_wave<J, 2>(args, stream, pointer_addressing)
                                    : run_wave<J, 4>(args, stream, pointer_addressing));
}

template <int R, int J, int D>
hipError_t run_multirow(BsrArgs args, hipStream_t stream) {
    args.tiles_n = ceil_div(args.N, 16 * J);
    const long total = static_cast<long>(ceil_div(args.block_rows, 4 * R)) * args.tiles_n;
    if (total > 0x7fffffffL) return hipErrorInvalidConfiguration;
    args.wg_total = static_cast<int>(total);
    dim3 grid(args.wg_total);
    if (args.b_vec_ok) {
        hipLaunchKernelGGL((bsr_multirow_kernel<R, J, D, true>), grid, dim3(256), 0, stream, args);
    } else {
        hipLaunchKernelGGL((bsr_multirow_kernel<R, J, D, false>), grid, dim3(256), 0, stream, args);
    }
    return hipGetLastError();
}

template <int J, int D>
hipError_t run_splitk(BsrArgs args, hipStream_t stream) {
    args.tiles_n = ceil_div(args.N, 16 * J);
    const long total = static_cast<long>(args.block_rows) * args.tiles_n;
    if (total > 0x7fffffffL) return hipErrorInvalidConfiguration;
    args.wg_total = static_cast<int>(total);
    dim3 grid(args.wg_total);
    if (args.b_vec_ok) {
        hipLaunchKernelGGL((bsr_splitk_kernel<J, D, true>), grid, dim3(256), 0, stream, args);
    } else {
        hipLaunchKernelGGL((bsr_splitk_kernel<J, D, false>), grid, dim3(256), 0, stream, args);
    }
    return hipGetLastError();
}

hipError_t dispatch_splitk(int j, int depth, const BsrArgs& args, hipStream_t stream) {
    if (j == 1) return depth == 1 ? run_splitk<1, 1>(args, stream) : run_splitk<1, 2>(args, stream);
    if (j == 2) return depth == 1 ? run_splitk<2, 1>(args, stream) : run_splitk<2, 2>(args, stream);
    return depth == 1 ? run_splitk<4, 1>(args, stream) : run_splitk<4, 2>(args, stream);
}

template <int R>
hipError_t dispatch_multirow(int j, int depth, const BsrArgs& args, hipStream_t stream) {
    if (j == 1) return depth == 1 ? run_multirow<R, 1, 1>(args, stream) : run_multirow<R, 1, 2>(args, stream);
    if (j == 2) return depth == 1 ? run_multirow<R, 2, 1>(args, stream) : run_multirow<R, 2, 2>(args, stream);
    return depth == 1 ? run_multirow<R, 4, 1>(args, stream) : run_multirow<R, 4, 2>(args, stream);
}

template <int RG, int J>
hipError_t run_rowgroup(const BsrArgs& args, hipStream_t stream) {
    dim3 grid(ceil_div(args.block_rows, RG), ceil_div(args.N, 16 * J));
    // Batch of up to 8 pairs (16 block-columns: one diagonal block of c4, a
    // whole banded row group of c3), fewer when each thread stages several
    // 16-byte chunks per tile, to bound the staging registers (P * CPT <= 8).
    constexpr int CPT = (32 * 2 * J + RG * 64 - 1) / (RG * 64);
    constexpr int P = (8 / CPT) < 2 ? 2 : 8 / CPT;
    constexpr size_t tiles_bytes = sizeof(_Float16) * P * 32 * (16 * J + 16);
    const size_t lds = tiles_bytes + sizeof(uint32_t) * ((args.block_cols + 31) / 32);
    hipLaunchKernelGGL((bsr_rowgroup_kernel<RG, J, P>), grid, dim3(RG * 64), lds, stream, args);
    return hipGetLastError();
}

template <int RG>
hipError_t dispatch_rowgroup(int j, const BsrArgs& args, hipStream_t stream) {
    switch (j) {
        case 1: return run_rowgroup<RG, 1>(args, stream);
        case 2: return run_rowgroup<RG, 2>(args, stream);
        case 8: return run_rowgroup<RG, 8>(args, stream);
        default: return run_rowgroup<RG, 4>(args, stream);
    }
}

}  // namespace

Error launch_float_to_half(const float* src, half* dst, long n, hipStream_t stream) {
    if (n < 0) return fail(kInvalid, "negative element count");
    if (n == 0) return Error{};
    if (src == nullptr || dst == nullptr) return fail(kInvalid, "null device pointer");
    const bool vec = (reinterpret_cast<uintptr_t>(src) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(dst) % 16 == 0);
    const long threads = vec ? (n + 7) / 8 : n;
    const long blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffL) return fail(kInvalid, "element count too large");
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, src, reinterpret_cast<_Float16*>(dst), n, vec ? 1 : 0);
    return from_hip(hipGetLastError(), "float_to_half launch");
}

Error launch_bsr(const BSR& A, const half* B, float* C, int N, hipStream_t stream,
                 const BsrOpts* opts) {
    if (A.num_rows < 0 || A.num_cols < 0 || A.num_blocks < 0 || N < 0) {
        return fail(kInvalid, "negative matrix dimension");
    }
    if (A.block_rows != (A.num_rows + 15) / 16 || A.block_cols != (A.num_cols + 15) / 16) {
        return fail(kInvalid, "BSR block dimensions do not match num_rows / num_cols");
    }
    if (A.num_rows == 0 || N == 0) return Error{};
    if (A.row_ptr == nullptr || C == nullptr || B == nullptr) {
        return fail(kInvalid, "null device pointer");
    }
    if (A.num_blocks > 0 && (A.col_idx == nullptr || A.values == nullptr)) {
        return fail(kInvalid, "null device pointer");
    }
    if (reinterpret_cast<uintptr_t>(A.values) % 16 != 0) {
        return fail(kInvalid, "BSR values must be 16-byte aligned");
    }
    BsrArgs args{A.row_ptr,
                 A.col_idx,
                 reinterpret_cast<const _Float16*>(A.values),
                 reinterpret_cast<const _Float16*>(B),
                 C,
                 A.num_rows,
                 A.num_cols,
                 N,
                 A.block_rows,
                 (N % 8 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0) ? 1 : 0,
                 A.block_cols,
                 0,
                 0,
                 0,
                 A.num_blocks};
    const BsrOpts o = opts ? *opts : BsrOpts{};
    args.xcd_order = o.xcd_order == 2 ? 0 : 1;
    hipError_t e;
    const int nwords = (A.block_cols + 31) / 32;
    const bool use_groups = o.row_group != 0 && !o.per_wave && nwords <= kMaxUnionWords;
    if (!use_groups) {
        // Defaults of the wave kernel, from a sweep of 92 MI355X runs (uniform,
        // banded, block-diagonal and power-law, M = 4096 .. 16384, N = 64 ..
        // 512).  Four 16-column tiles per wave halve the A-block re-reads of
        // two tiles and win once the grid still has >= 1024 waves at four
        // tiles, unless block-rows are short (< 12 blocks) and the grid is
        // under 2048 waves: then the extra waves of two tiles hide more latency
        // (e.g. uniform 8192^2 density 0.01 N=128: 67 -> 48 us; banded 8192^2
        // half-bandwidth 64 N=128 stays at two tiles, 4.0 vs 4.1 us).  Four
        // pairs in flight pay on long block-rows: >= 30 blocks at two tiles,
        // >= 96 at four (uniform 4096^2 density 0.01 N=128: 26.4 -> 20.3 us).
        // The pointer-arithmetic form keeps two tiles and two pairs: it has no
        // buffer-to-LDS staging, and four tiles measured slower there.
        const bool rec = o.addressing != 1 && records_fit(args);
        const double bpr = A.block_rows > 0 ? static_cast<double>(A.num_blocks) / A.block_rows : 0.0;
        const long waves4 = static_cast<long>(A.block_rows) * ((N + 63) / 64);
        const int j_auto =
            N <= 16 ? 1
                    : ((rec && waves4 >= 1024 && (bpr >= 12.0 || waves4 >= 2048)) ? 4 : 2);
        const int j = (o.tiles == 1 || o.tiles == 2 || o.tiles == 4) ? o.tiles : j_auto;
        const int d_auto = (rec && bpr >= (j == 4 ? 96.0 : 30.0)) ? 4 : 2;
        const int d = (o.depth == 1 || o.depth == 2 || o.depth == 4) ? o.depth : d_auto;
        if (o.split == 4) {
            e = dispatch_splitk(j, d == 1 ? 1 : 2, args, stream);
            return from_hip(e, "spmm_wmma launch");
        }
        if (o.rows == 2 || o.rows == 4) {
            const int dm = d == 1 ? 1 : 2;
            e = o.rows == 2 ? dispatch_multirow<2>(j, dm, args, stream)
                            : dispatch_multirow<4>(j, dm, args, stream);
            return from_hip(e, "spmm_wmma launch");
        }
        const bool ptr = o.addressing == 1;
        e = j == 1 ? dispatch_wave<1>(d, ptr, args, stream)
                   : (j == 2 ? dispatch_wave<2>(d, ptr, args, stream)
                             : dispatch_wave<4>(d, ptr, args, stream));
        return from_hip(e, "spmm_wmma launch");
    }
    int j = o.tiles;
    if (j != 1 && j != 2 && j != 4 && j != 8) j = N <= 16 ? 1 : (N <= 32 ? 2 : 4);
    if (o.row_group == 8) {
        e = dispatch_rowgroup<8>(j, args, stream);
    } else if (o.row_group == 2) {
        e = dispatch_rowgroup<2>(j, args, stream);
    } else if (o.row_group == 1) {
        e = dispatch_rowgroup<1>(j, args, stream);
    } else {
        e = dispatch_rowgroup<4>(j, args, stream);
    }
    return from_hip(e, "spmm_wmma launch");
}

}  // namespace engine
}  // namespace spmm
