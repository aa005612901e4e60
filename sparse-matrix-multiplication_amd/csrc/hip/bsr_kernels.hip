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
#include <initializer_list>
#include <type_traits>

#include "amdgcn.h"
#include "engine.h"
#include "spmm/utils.h"

namespace spmm {
namespace engine {

namespace {

using namespace dev;  // vector types, buffer loads, waits, barriers (amdgcn.h)

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

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

// The record kernel stores its 16-byte C row chunks with device scope
// (kStoreDevice, the sc1 bit).  Measured on MI355X against streaming stores of
// the same chunks (A/B over three rounds, results bit-identical): c3 3.84 ->
// 3.65 us, c4 5.88 -> 5.79 us per launch.  The CSR kernels measured slower
// with it (c1 +7%, c2 +1.5%, c5 +2-3%) and keep streaming stores.

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
    int             c_vec_ok;   // C 16-byte aligned (with b_vec_ok: rows of 16-byte chunks)
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

    // Lane constants: load instruction c fills 16-byte position idx = lane +
    // 64c of the slot, staged row srow (block srow >= 16 of the pair).  The
    // slot is row-major with its chunks XOR-swizzled per row (chunk k of row
    // r at position k ^ swz(r)), which spreads the rows one
    // ds_read_b64_tr_b16 touches over all LDS banks; so position idx holds
    // chunk (idx % CH) ^ swz(srow): columns n .. n+7, byte offset nbyte of
    // its B row.  Columns past N read a valid chunk of the row instead; their
    // products land in output columns >= N, which are never stored.
    auto swz = [](int r) { return (2 * ((r >> 1) ^ (r >> 3))) & (CH - 1); };
    int srow[CPL], nbyte[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int idx = lane + c * 64;
        srow[c] = idx / CH;
        const int n = n0 + ((idx % CH) ^ swz(srow[c])) * 8;
        nbyte[c] = (n < a.N ? n : 0) * 2;
    }
    // B operand reads: rows 8g + t/4 (lo) and +4 (hi), chunk 2j + (t & 3) / 2
    // of the row, bytes 8 * (t & 1) of it; swz(r) is even, so the swizzle
    // XORs the tile index j with swz(r) / 2.
    const int h_lo  = swz(8 * g + (t >> 2)) >> 1;
    const int h_hi  = swz(8 * g + (t >> 2) + 4) >> 1;
    const int in_lo = (8 * g + (t >> 2)) * NT + ((t & 3) >> 1) * 8 + (t & 1) * 4;  // fp16 units
    const int in_hi = in_lo + 4 * NT;
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
        const _Float16* st = slot(d);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const s16x4 lo = lds_read_tr16(st + in_lo + (j ^ h_lo) * 16);
            const s16x4 hi = lds_read_tr16(st + in_hi + (j ^ h_hi) * 16);
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
    if (a.c_vec_ok) {
        // The tile goes through the wave's first ring slot (16 x NT fp32 is
        // exactly its size, and every load into it has landed) and leaves
        // row-major in 16-byte stores: each store instruction writes whole
        // NT-column row segments instead of 64-byte pieces of four rows.
        // Measured on MI355X: c3 3.87 -> 3.71 us, c4 5.83 -> 5.74 us per launch.
        wait_vmcnt<0>();
        float* ct = reinterpret_cast<float*>(slot(0));
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) ct[(4 * g + i) * NT + 16 * j + t] = acc[j][i];
        }
        constexpr int LPR = NT / 4;    // lanes per row, 4 floats each
        constexpr int RPI = 64 / LPR;  // rows per store instruction
        const int lr = lane / LPR;
        const int lc = (lane % LPR) * 4;
        // The block-row's C rows as one raw buffer (at most 16 x 8191 floats,
        // so byte offsets fit 32 bits whatever the size of C).
        const int rows_here = min(16, a.M - br * 16);
        const __amdgpu_buffer_rsrc_t c_rows = __builtin_amdgcn_make_buffer_rsrc(
            a.C + static_cast<size_t>(br) * 16 * a.N, static_cast<short>(0),
            rows_here * a.N * 4, kBufWord3);
#pragma unroll
        for (int s = 0; s < 16 / RPI; ++s) {
            const int r   = s * RPI + lr;
            const f32x4 v = *reinterpret_cast<const f32x4*>(ct + r * NT + lc);
            const int col = n0 + lc;  // N % 8 == 0: a chunk is all in or all out
            if (r < rows_here && col < a.N) {
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), c_rows,
                                                       (r * a.N + col) * 4, 0, kStoreDevice);
            }
        }
        return;
    }
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
// Shared-panel kernel: a workgroup owns R consecutive block-rows (16R rows of
// C) and NT = 16*J columns, and multiplies them by B one union block pair at
// a time.
//   1. Union of the R block-rows' block-column lists (contiguous in col_idx).
//      Fast path, when every block-column lies within 64 of the smallest and
//      there are at most 256 entries: each wave ORs a 64-bit mask per
//      block-row with DPP and one barrier combines the waves.  Otherwise an
//      LDS bitmap over all block-columns (up to kPanelMaxWords * 32) and an
//      exclusive prefix of its words' popcounts rank every block-column.
//   2. The union's slots go into lane-indexed registers (per slot: the
//      block-column, and this wave's blocks there or -1), which the pipeline
//      reads with v_readlane: a pair costs the scalar unit only its slot
//      numbers, and the pipeline reads no LDS but the B stages.
//   3. Slots are multiplied in pairs (two 16-deep blocks are one K = 32 step
//      of v_mfma_f32_16x16x32_f16).  A pair's 32 B rows x NT columns are
//      loaded once per workgroup straight into an LDS stage (buffer-to-LDS
//      loads, XOR-swizzled against bank conflicts) and read by every wave
//      with ds_read_b64_tr_b16; each wave loads the A operands of its own
//      block-rows (an absent block has index -1 and reads as zeros through
//      the buffer range check).  D stages in flight, one barrier per pair.
//   4. The four waves form a WR x (4/WR) grid over the tile: a wave multiplies
//      R/WR block-rows by J/(4/WR) 16-column tiles.
// Lists that are not strictly ascending or hold block-columns outside the
// matrix, and matrices wider than the bitmap, use the identity union (slot u =
// entry u of the concatenated lists): correct for any BSR, at up to R times
// the matrix-core work.
//
// What it buys, measured on MI355X (rocprofv3 counters, c4): the wave
// kernel's four waves of a workgroup already share their B tiles through the
// vector L1 -- both kernels make the same 263 K L2 read requests per launch
// -- so the panel saves L1 accesses (0.66 M vs 1.44 M of 64 bytes) but pays
// barriers, lockstep phases and LDS read bandwidth.  It is faster only on
// wide B with long block-rows (N >= 256 and 24 - 64 blocks per block-row:
// 1.03 - 1.31x, e.g. block-diagonal 512 at N = 512 12.6 -> 10.8 us), which is
// where the launcher picks it; c3 and c4 stay on the wave kernel.
// ---------------------------------------------------------------------------
constexpr int kPanelMaxWords = 256;  // union bitmap: up to 8192 block-columns (K <= 131072)
constexpr int kPanelSlots    = 126;  // union slots per pass (two registers per lane, lane 127 free)

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    return v;
}

// OR of a 64-bit value over the 64 lanes of a wave (all lanes active): DPP
// xor-1 and xor-2 inside quads, then half-row and row mirrors give every
// lane its row's OR, and the four rows are combined from lanes 0, 16, 32, 48.
__device__ __forceinline__ uint64_t wave_or64(uint64_t v) {
    unsigned lo = static_cast<unsigned>(v), hi = static_cast<unsigned>(v >> 32);
    lo |= __builtin_amdgcn_update_dpp(0u, lo, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    hi |= __builtin_amdgcn_update_dpp(0u, hi, 0xB1, 0xF, 0xF, false);
    lo |= __builtin_amdgcn_update_dpp(0u, lo, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    hi |= __builtin_amdgcn_update_dpp(0u, hi, 0x4E, 0xF, 0xF, false);
    lo |= __builtin_amdgcn_update_dpp(0u, lo, 0x141, 0xF, 0xF, false);  // row_half_mirror
    hi |= __builtin_amdgcn_update_dpp(0u, hi, 0x141, 0xF, 0xF, false);
    lo |= __builtin_amdgcn_update_dpp(0u, lo, 0x140, 0xF, 0xF, false);  // row_mirror
    hi |= __builtin_amdgcn_update_dpp(0u, hi, 0x140, 0xF, 0xF, false);
    const unsigned rlo = __builtin_amdgcn_readlane(lo, 0) | __builtin_amdgcn_readlane(lo, 16) |
                         __builtin_amdgcn_readlane(lo, 32) | __builtin_amdgcn_readlane(lo, 48);
    const unsigned rhi = __builtin_amdgcn_readlane(hi, 0) | __builtin_amdgcn_readlane(hi, 16) |
                         __builtin_amdgcn_readlane(hi, 32) | __builtin_amdgcn_readlane(hi, 48);
    return (static_cast<uint64_t>(rhi) << 32) | rlo;
}

__device__ __forceinline__ uint64_t below(int p) {  // bits 0 .. p-1, p in [0, 64)
    return (1ull << p) - 1ull;
}

template <int R, int J, int WR, int D>
__device__ __forceinline__ void bsr_panel_body(const BsrArgs& a, _Float16* __restrict__ s0,
                                               _Float16* __restrict__ s1,
                                               _Float16* __restrict__ s2,
                                               _Float16* __restrict__ s3,
                                               uint32_t* __restrict__ s_bits,
                                               int* __restrict__ s_pre, int* __restrict__ s_ucol,
                                               int* __restrict__ s_blk,
                                               uint64_t* __restrict__ s_mask,
                                               int* __restrict__ s_misc) {
    constexpr int WC  = 4 / WR;
    constexpr int TR  = R / WR;          // block-rows per wave
    constexpr int TC  = J / WC;          // 16-column tiles per wave
    constexpr int NT  = 16 * J;          // columns per workgroup
    constexpr int CH  = NT / 8;          // 16-byte chunks per staged B row
    constexpr int CPT = 32 * CH / 256;   // chunks per thread per pair
    constexpr int PER = CPT + TR;        // vector-memory instructions per thread per pair
    static_assert(WR * WC == 4 && TR * WR == R && TC * WC == J, "wave grid");
    static_assert(CPT >= 1 && CPT * 256 == 32 * CH, "whole chunks per thread");
    static_assert(64 / CH <= 16, "a wave's chunks of one load stay inside one block");
    static_assert(D == 2 || D == 4, "2 or 4 stages");

    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g    = lane >> 4;
    const int t    = lane & 15;
    const int wr   = wave / WC;
    const int wc   = wave % WC;
    int bx, by;
    wave_tile_of(a, bx, by);
    const int br0 = bx * R;
    const int n0  = by * NT;
    auto stage = [&](int d) -> _Float16* { return d == 0 ? s0 : d == 1 ? s1 : d == 2 ? s2 : s3; };

    const __amdgpu_buffer_rsrc_t rec_b = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a.B), static_cast<short>(a.N * 2), a.K, kBufWord3);
    const __amdgpu_buffer_rsrc_t rec_a = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a.vals), static_cast<short>(512), a.num_blocks, kBufWord3);

    // Block-rows br0 .. br0+R-1 (those past the matrix are empty); their
    // lists are contiguous in col_idx from e0.
    int rp[R + 1];
#pragma unroll
    for (int r = 0; r <= R; ++r) rp[r] = a.row_ptr[min(br0 + r, a.block_rows)];
    const int e0 = rp[0];
    const int T  = rp[R] - e0;
    auto list_of = [&](int e) {  // block-row (0 .. R-1) of entry e0 + e
        int r = 0;
#pragma unroll
        for (int i = 1; i < R; ++i) r += (e0 + e >= rp[i]) ? 1 : 0;
        return r;
    };
    auto list_start = [&](int e) {  // first entry of e0 + e's block-row (selects, no indexing)
        int st = rp[0];
#pragma unroll
        for (int i = 1; i < R; ++i) st = (e0 + e >= rp[i]) ? rp[i] : st;
        return st;
    };
    // Span of the block-columns from the lists' first and last entries.
    int lo = 0x7fffffff, hi = -1;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (rp[r + 1] > rp[r]) {
            lo = min(lo, a.col_idx[rp[r]]);
            hi = max(hi, a.col_idx[rp[r + 1] - 1]);
        }
    }
    // Stage layout: row-major 32 x NT fp16, its 16-byte chunks XOR-swizzled
    // per row (chunk c of row r sits at position c ^ swz(r)), which spreads
    // the sixteen rows one ds_read_b64_tr_b16 touches over all banks (4
    // conflict-free cycles instead of 16 with 32 banks).  A buffer-to-LDS load
    // puts lane i's 16 bytes at a fixed position, so the swizzle picks which
    // chunk each lane loads: load c of a pair fills position idx = 256c + tid,
    // i.e. staged row srow, with chunk (idx % CH) ^ swz(srow): columns n ..
    // n+7.  Rows 0-15 hold the pair's first block-column, 16-31 the second
    // (the same half for a whole wave's load).  Columns past N read a valid
    // chunk of the row instead; their products land in output columns >= N,
    // which are never stored.
    auto swz = [](int r) { return (2 * ((r >> 1) ^ (r >> 3))) & (CH - 1); };
    int srow[CPT], nbyte[CPT];
    bool second[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int idx = c * 256 + tid;
        srow[c]   = idx / CH;
        second[c] = __builtin_amdgcn_readfirstlane(srow[c] >> 4) != 0;
        const int n = n0 + ((idx % CH) ^ swz(srow[c])) * 8;
        nbyte[c] = (n < a.N ? n : 0) * 2;
    }

    // A operand: row t of the pair's block g >> 1, columns 8 * (g & 1) .. +7
    const int a_off = t * 32 + 16 * (g & 1);
    // B operand reads: lane (g, t) addresses rows 8g + t/4 (lo) and +4 (hi),
    // chunk 2 * tile + (t & 3) / 2 of the row, bytes 8 * (t & 1) of it; with
    // swz(r) even, the swizzle XORs the tile index with swz(r) / 2.
    const int row_lo = 8 * g + (t >> 2);
    const int h_lo   = swz(row_lo) >> 1;
    const int h_hi   = swz(row_lo + 4) >> 1;
    const int in_lo  = row_lo * NT + ((t & 3) >> 1) * 8 + (t & 1) * 4;  // fp16 units
    const int in_hi  = in_lo + 4 * NT;

    f32x4 acc[TR][TC];
#pragma unroll
    for (int i = 0; i < TR; ++i) {
#pragma unroll
        for (int j = 0; j < TC; ++j) acc[i][j] = f32x4(0.0f);
    }
    u32x4 af[D][TR];

    int off_lo[TC], off_hi[TC];  // per tile: this lane's B operand addresses in a stage
#pragma unroll
    for (int j = 0; j < TC; ++j) {
        off_lo[j] = in_lo + ((wc * TC + j) ^ h_lo) * 16;
        off_hi[j] = in_hi + ((wc * TC + j) ^ h_hi) * 16;
    }
    auto compute = [&](int d) {
        const _Float16* st = stage(d);
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            const s16x4 lo4 = lds_read_tr16(st + off_lo[j]);
            const s16x4 hi4 = lds_read_tr16(st + off_hi[j]);
            const s16x8 both = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            const f16x8 bop = __builtin_bit_cast(f16x8, both);
#pragma unroll
            for (int i = 0; i < TR; ++i) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8, af[d][i]), bop, acc[i][j], 0, 0, 0);
            }
        }
    };

    // This thread's entry (the fast path needs at most one per thread).
    const int  x    = tid < T ? a.col_idx[e0 + tid] : 0;
    const int  xp   = tid < T && tid > 0 ? a.col_idx[e0 + tid - 1] : -1;
    const int  my_r = list_of(tid);
    // ---- 1. union of the R lists (fast path: DPP masks and one barrier;
    // otherwise the LDS bitmap and its word prefix; identity union for lists
    // that fail the checks or matrices wider than the bitmap).
    const bool fast_shape = T > 0 && T <= 256 && lo >= 0 && hi - lo < 64;
    const int  nwords     = (a.block_cols + 31) >> 5;
    const bool fits       = nwords <= kPanelMaxWords;
    bool bad = false;
    if (fast_shape) {
        const bool ok = tid >= T || (static_cast<unsigned>(x) < static_cast<unsigned>(a.block_cols) &&
                                     x >= lo && x - lo < 64 &&
                                     (e0 + tid == list_start(tid) || xp < x));
        const uint64_t bit = (tid < T && ok) ? (1ull << (x - lo)) : 0ull;
        uint64_t wm[R];
#pragma unroll
        for (int r = 0; r < R; ++r) wm[r] = wave_or64(my_r == r ? bit : 0ull);
        const bool wbad = __ballot(!ok) != 0;
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) s_mask[wave * R + r] = wm[r];
            s_misc[4 + wave] = wbad ? 1 : 0;
        }
    } else {
        if (fits) {
            for (int w = tid; w < nwords; w += 256) s_bits[w] = 0u;
        }
        if (tid == 0) s_misc[0] = fits ? 0 : 1;  // 1: identity union
    }
    for (int i = tid; i < kPanelSlots * R; i += 256) s_blk[i] = -1;
    __syncthreads();
    uint64_t rmask[R];  // fast path: block-row r's block-columns, bit = column - lo
    if (fast_shape) {
        bad = (s_misc[4] | s_misc[5] | s_misc[6] | s_misc[7]) != 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            rmask[r] = s_mask[r] | s_mask[R + r] | s_mask[2 * R + r] | s_mask[3 * R + r];
        }
    }
    const bool use_fast = fast_shape && !bad;
    bool identity = fast_shape ? bad : false;
    if (!fast_shape) {
        for (int e = tid; e < T; e += 256) {
            const int xe = e < 256 ? x : a.col_idx[e0 + e];
            const bool wrong = static_cast<unsigned>(xe) >= static_cast<unsigned>(a.block_cols) ||
                               (e0 + e != list_start(e) && a.col_idx[e0 + e - 1] >= xe);
            if (wrong) {
                s_misc[0] = 1;  // every writer stores 1
            } else if (fits) {
                atomicOr(&s_bits[xe >> 5], 1u << (xe & 31));
            }
        }
        __syncthreads();
        identity = s_misc[0] != 0;
        if (!identity) {
            if (wave == 0) {  // lane l: words 4l .. 4l+3 (nwords <= 256)
                int pc[4], sum = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int w = 4 * lane + k;
                    pc[k] = w < nwords ? __builtin_popcount(s_bits[w]) : 0;
                    sum += pc[k];
                }
                const int incl = wave_inclusive_scan(sum, lane);
                int run = incl - sum;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (4 * lane + k < nwords) s_pre[4 * lane + k] = run;
                    run += pc[k];
                }
                if (lane == 63) s_misc[1] = incl;
            }
            __syncthreads();
        }
    }
    uint64_t umask = 0ull;
    if (use_fast) {
#pragma unroll
        for (int r = 0; r < R; ++r) umask |= rmask[r];
    }
    const int U = use_fast ? __builtin_popcountll(umask) : (identity ? T : s_misc[1]);
    // This wave's block-rows wr*TR .. wr*TR+TR-1: first entries and masks,
    // picked with selects (a runtime index into rp / rmask would put the
    // arrays in scratch memory).
    int      my_rp[TR];
    uint64_t my_mask[TR];
#pragma unroll
    for (int i = 0; i < TR; ++i) {
        my_rp[i]   = 0;
        my_mask[i] = 0ull;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r == wr * TR + i) {
                my_rp[i] = rp[r];
                if (use_fast) my_mask[i] = rmask[r];
            }
        }
    }

    // ---- 2. the pass's slot tables in registers: lane l of tcol[k] holds the
    // block-column of union slot 64k + l (-1 past the pass's end), lane l of
    // tblk[i][k] the block of this wave's block-row i at that slot (-1 where
    // it has none).  The pipeline reads them with v_readlane (a vector
    // instruction), so a pair costs the scalar unit only its slot numbers and
    // reads no LDS but the B stages.  Lane 63 of the last table always holds
    // -1 (a pass has at most kPanelSlots <= 126 slots): slot numbers are
    // clamped to it, so the zero pairs past the end need no test.
    int tcol[2], tblk[TR][2];
    // Pipeline over a pass of uc slots: pair q (slots 2q, 2q+1) lives in
    // stage q % D.  Before pair q is read, each thread waits until its own
    // loads of pair q have landed (loads retire in issue order, so the D - 2
    // later pairs' loads may stay outstanding) and the barrier makes every
    // thread's share visible.  The barrier is a bare s_barrier:
    // __syncthreads' release fence would also wait for the later pairs'
    // buffer-to-LDS writes, draining the ring at every pair.  A wave reaches
    // it with its LDS reads of pair q - 1 complete (the matrix-core
    // instructions consumed them), and the stage refilled right after it held
    // pair q - 1.  Every issue is unconditional: pairs past the last one read
    // -1 and load zeros (out of range, no memory traffic), so the loads in
    // flight are the same on every path and the compiler's own wait counts
    // stay exact.
    auto pipeline = [&](int uc, auto two_tables) {
        constexpr bool TWO = decltype(two_tables)::value;
        auto pick = [&](const int (&v)[2], int u) -> int {
            if constexpr (TWO) {
                const int uu = min(u, 127);
                return uu < 64 ? __builtin_amdgcn_readlane(v[0], uu)
                               : __builtin_amdgcn_readlane(v[1], uu - 64);
            } else {
                return __builtin_amdgcn_readlane(v[0], min(u, 63));
            }
        };
        auto issue = [&](int d, int q) {
            _Float16* dst = stage(d);
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
                const int bc = pick(tcol, 2 * q + (second[c] ? 1 : 0));  // -1: rows -16..-1, zeros
                sbuf_load_lds(rec_b, (spmm_lds_ptr)(dst + (c * 256 + wave * 64) * 8), 16,
                              bc * 16 + (srow[c] & 15), nbyte[c], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < TR; ++i) {
                const int b0 = pick(tblk[i], 2 * q);
                const int b1 = pick(tblk[i], 2 * q + 1);
                af[d][i] = sbuf_load_u32x4_dev(rec_a, (g >> 1) ? b1 : b0, a_off);
            }
        };
        const int npairs = (uc + 1) >> 1;
#pragma unroll
        for (int d = 0; d < D - 1; ++d) issue(d, d);
        const int rounds = (npairs + D - 1) / D * D;
        for (int q0 = 0; q0 < rounds; q0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                wait_vmcnt<(D - 2) * PER>();
                lds_barrier();
                issue((d + D - 1) % D, q0 + d + D - 1);
                if (q0 + d < npairs) compute(d);
            }
        }
        wait_vmcnt<0>();  // the zero loads of the pairs past the end
    };

    if (use_fast) {
        // Lane p stands for block-column lo + p: if it is in the union, its
        // slot is the number of union columns below it, and ds_permute pushes
        // its table entries to that lane (lanes outside the union push to lane
        // 63, which is at or past U and is reset to -1).
        const bool in_u = ((umask >> lane) & 1ull) != 0;
        const int  addr = (in_u ? __builtin_popcountll(umask & below(lane)) : 63) * 4;
        const int  col  = __builtin_amdgcn_ds_permute(addr, lo + lane);
        tcol[0] = lane < U ? col : -1;
        tcol[1] = -1;
#pragma unroll
        for (int i = 0; i < TR; ++i) {
            const bool has = ((my_mask[i] >> lane) & 1ull) != 0;
            const int blk = has ? my_rp[i] + __builtin_popcountll(my_mask[i] & below(lane)) : -1;
            const int got = __builtin_amdgcn_ds_permute(addr, blk);
            tblk[i][0] = lane < U ? got : -1;
            tblk[i][1] = -1;
        }
        if (U <= 63) {
            pipeline(U, std::integral_constant<bool, false>());
        } else {
            pipeline(U, std::integral_constant<bool, true>());
        }
    } else {
        for (int u0 = 0; u0 < U; u0 += kPanelSlots) {
            const int uc = min(kPanelSlots, U - u0);
            if (u0 > 0) {  // the first pass's table was cleared before the union
                for (int i = tid; i < uc * R; i += 256) s_blk[i] = -1;
                __syncthreads();
            }
            for (int e = tid; e < T; e += 256) {
                const int xe = e < 256 ? x : a.col_idx[e0 + e];
                int u = e - u0;
                if (!identity) {
                    u = s_pre[xe >> 5] +
                        __builtin_popcount(s_bits[xe >> 5] & ((1u << (xe & 31)) - 1u)) - u0;
                }
                if (u >= 0 && u < uc) {
                    s_blk[u * R + list_of(e)] = e0 + e;
                    s_ucol[u] = xe;
                }
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int u = 64 * k + lane;
                tcol[k] = u < uc ? s_ucol[u] : -1;
#pragma unroll
                for (int i = 0; i < TR; ++i) tblk[i][k] = u < uc ? s_blk[u * R + wr * TR + i] : -1;
            }
            if (uc <= 63) {
                pipeline(uc, std::integral_constant<bool, false>());
            } else {
                pipeline(uc, std::integral_constant<bool, true>());
            }
            __syncthreads();  // the next pass rewrites the tables and the stages
        }
    }



    // D layout: lane holds rows 4*g + i, column t of each 16-column tile.
#pragma unroll
    for (int i = 0; i < TR; ++i) {
        const int br = br0 + wr * TR + i;
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            const int col = n0 + (wc * TC + j) * 16 + t;
            if (col >= a.N) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int row = br * 16 + 4 * g + k;
                if (row < a.M) store_c(a.C + static_cast<size_t>(row) * a.N + col, acc[i][j][k]);
            }
        }
    }
}

// The stages and tables are separate LDS objects passed as restrict pointers
// (as in the record kernel): the wait-count pass then sees that reading one
// stage does not depend on buffer-to-LDS writes still going into another.
template <int R, int J, int WR, int D>
__global__ __launch_bounds__(256) void bsr_panel_kernel(BsrArgs a) {
    constexpr int TILE = 32 * 16 * J;
    __shared__ __attribute__((aligned(16))) _Float16 s_b0[TILE];
    __shared__ __attribute__((aligned(16))) _Float16 s_b1[TILE];
    __shared__ __attribute__((aligned(16))) _Float16 s_b2[D >= 3 ? TILE : 8];
    __shared__ __attribute__((aligned(16))) _Float16 s_b3[D >= 4 ? TILE : 8];
    __shared__ uint32_t s_bits[kPanelMaxWords];
    __shared__ int s_pre[kPanelMaxWords];
    __shared__ int s_ucol[kPanelSlots];
    __shared__ int s_blk[kPanelSlots * R];
    __shared__ uint64_t s_mask[4 * R];
    __shared__ int s_misc[8];
    bsr_panel_body<R, J, WR, D>(a, s_b0, s_b1, s_b2, s_b3, s_bits, s_pre, s_ucol, s_blk, s_mask,
                                s_misc);
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

template <int R, int J, int WR, int D>
hipError_t run_panel(BsrArgs args, hipStream_t stream) {
    args.tiles_n = ceil_div(args.N, 16 * J);
    const long total = static_cast<long>(ceil_div(args.block_rows, R)) * args.tiles_n;
    if (total > 0x7fffffffL) return hipErrorInvalidConfiguration;
    args.wg_total = static_cast<int>(total);
    hipLaunchKernelGGL((bsr_panel_kernel<R, J, WR, D>), dim3(args.wg_total), dim3(256), 0, stream,
                       args);
    return hipGetLastError();
}

// Panel shapes: R block-rows x 16J columns per workgroup, each wave four
// 16-column tiles (waves 4 x 1 for J = 4, 2 x 2 for J = 8).
// Stages in flight: 2 or 4.
template <int R, int J>
hipError_t dispatch_panel(int depth, const BsrArgs& args, hipStream_t stream) {
    constexpr int WR = J == 4 ? 4 : 2;
    return depth <= 2 ? run_panel<R, J, WR, 2>(args, stream) : run_panel<R, J, WR, 4>(args, stream);
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
                 A.num_blocks,
                 reinterpret_cast<uintptr_t>(C) % 16 == 0 ? 1 : 0};
    const BsrOpts o = opts ? *opts : BsrOpts{};
    if (o.row_group != 0 && o.row_group != 1 && o.row_group != 4 && o.row_group != 8) {
        return fail(kInvalid, "row_group must be 0, 1, 4 or 8");
    }
    // Option values no kernel has are refused; with the kernel chosen
    // explicitly (row_group 1 / per_wave, row_group 4 / 8) so are the values
    // that kernel lacks.  Under the automatic choice a value the chosen kernel
    // lacks takes that kernel's default.
    const auto one_of = [](int v, std::initializer_list<int> ok) {
        for (int x : ok) {
            if (v == x) return true;
        }
        return false;
    };
    if (!one_of(o.tiles, {0, 1, 2, 4, 8}) || !one_of(o.depth, {0, 1, 2, 4})) {
        return fail(kInvalid, "tiles must be 0, 1, 2, 4 or 8 and depth 0, 1, 2 or 4");
    }
    const bool panel_forced = !o.per_wave && (o.row_group == 4 || o.row_group == 8);
    const bool wave_forced = o.per_wave || o.row_group == 1;
    if (panel_forced && (!one_of(o.tiles, {0, 4, 8}) || !one_of(o.depth, {0, 2, 4}))) {
        return fail(kInvalid, "shared-panel kernel: tiles must be 0, 4 or 8 and depth 0, 2 or 4");
    }
    if (wave_forced && o.tiles == 8) {
        return fail(kInvalid, "wave kernel: tiles must be 0, 1, 2 or 4");
    }
    args.xcd_order = o.xcd_order == 2 ? 0 : 1;
    hipError_t e;
    const bool rec = o.addressing != 1 && records_fit(args);
    const double bpr = A.block_rows > 0 ? static_cast<double>(A.num_blocks) / A.block_rows : 0.0;
    // Shared-panel kernel (R = 4, 64 columns, 2 stages): automatic on wide B
    // with long block-rows of structured inputs, the cells where it measured
    // faster than the wave kernel (N >= 256, 24 - 64 blocks per block-row:
    // 1.03 - 1.31x over 36 block-diagonal and banded inputs); explicit
    // row_group 4 / 8 forces it.
    const bool panel_auto = rec && N >= 256 && A.block_cols <= kPanelMaxWords * 32 &&
                            bpr >= 24.0 && bpr <= 64.0;
    const bool panel = !o.per_wave && rec &&
                       (o.row_group == 4 || o.row_group == 8 || (o.row_group == 0 && panel_auto));
    if (panel) {
        const int R = o.row_group == 8 ? 8 : 4;
        const int j = o.tiles == 8 ? 8 : 4;
        const int d = o.depth == 4 ? 4 : 2;  // 0 (or a wave-only 1 when automatic): 2
        if (R == 4) {
            e = j == 4 ? dispatch_panel<4, 4>(d, args, stream) : dispatch_panel<4, 8>(d, args, stream);
        } else {
            e = j == 4 ? dispatch_panel<8, 4>(d, args, stream) : dispatch_panel<8, 8>(d, args, stream);
        }
        return from_hip(e, "spmm_wmma launch");
    }
    // Defaults of the wave kernel, from a sweep of 92 MI355X runs (uniform,
    // banded, block-diagonal and power-law, M = 4096 .. 16384, N = 64 .. 512).
    // Four 16-column tiles per wave halve the A-block re-reads of two tiles
    // and win once the grid still has >= 1024 waves at four tiles, unless
    // block-rows are short (< 12 blocks) and the grid is under 2048 waves:
    // then the extra waves of two tiles hide more latency (e.g. uniform
    // 8192^2 density 0.01 N=128: 67 -> 48 us).  Four pairs in flight pay on
    // long block-rows: >= 30 blocks at two tiles, >= 96 at four (uniform
    // 4096^2 density 0.01 N=128: 26.4 -> 20.3 us).  The pointer-arithmetic
    // form keeps two tiles and two pairs: it has no buffer-to-LDS staging,
    // and four tiles measured slower there.
    const long waves4 = static_cast<long>(A.block_rows) * ((N + 63) / 64);
    const int j_auto =
        N <= 16 ? 1 : ((rec && waves4 >= 1024 && (bpr >= 12.0 || waves4 >= 2048)) ? 4 : 2);
    const int j = (o.tiles == 1 || o.tiles == 2 || o.tiles == 4) ? o.tiles : j_auto;
    const int d_auto = (rec && bpr >= (j == 4 ? 96.0 : 30.0)) ? 4 : 2;
    const int d = (o.depth == 1 || o.depth == 2 || o.depth == 4) ? o.depth : d_auto;
    const bool ptr = o.addressing == 1;
    e = j == 1 ? dispatch_wave<1>(d, ptr, args, stream)
               : (j == 2 ? dispatch_wave<2>(d, ptr, args, stream)
                         : dispatch_wave<4>(d, ptr, args, stream));
    return from_hip(e, "spmm_wmma launch");
}

}  // namespace engine
}  // namespace spmm
