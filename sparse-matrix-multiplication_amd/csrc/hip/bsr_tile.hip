// Run-panel BSR x dense fp16 kernel on gfx950 matrix cores: the form of
// spmm_wmma (spmm_wmma.cu:49-117) that spmm_hybrid_run runs on structured
// inputs, whose block-rows hold runs of consecutive block-columns (banded and
// block-diagonal matrices).
//
// A plan, built once with the BSR, describes each panel of R consecutive
// block-rows in one 32-int record: the union of their runs (first block-column
// u0 and width U, contiguous) and, per block-row, its run as union slots
// [lo, hi) and the A block of slot lo.  The kernel then needs one scalar load
// before it can address every A block and B row of its panel; the reference
// kernel walks row_ptr and col_idx block by block.
//
// Workgroup = one panel x NT columns of C; its multiplying waves form a
// WR x WC grid (each wave RW = R / WR block-rows x TC = NT / (16 WC) 16-column
// tiles).  Three forms share the plan, the B staging and the operand layouts
// (the shape table in engine.h names the form as KIND):
//   - producer / consumer (KIND 2, 3; the default): four waves only issue
//     buffer-to-LDS loads of the panel's B rows (and, KIND 2, its A blocks)
//     chunk by chunk, four waves only multiply; one barrier per chunk.  Each
//     block-row's run is paired from its own first slot, (lo, lo+1), ..., in
//     v_mfma_f32_16x16x32_f16, an odd last block in v_mfma_f32_16x16x16_f16,
//     so the matrix cores multiply exactly the stored blocks.
//   - one-shot and ring (KIND 1, 0): four waves that both load and multiply,
//     A operands in VGPRs, the union's slots paired as (2q, 2q+1) with a
//     16x16x16 MFMA for a run end on an odd slot; the ring (NB chunk buffers,
//     NB - 1 chunks in flight) covers unions wider than the one-shot forms
//     hold.
//   - In all of them the union's B rows (16 per slot, NT columns) are staged
//     with buffer-to-LDS loads (no VGPR staging), XOR-swizzled in 16-byte units
//     against bank conflicts and read as MFMA operands with ds_read_b64_tr_b16;
//     a pair's B operand is read once per wave for all of the wave's
//     block-rows that hold it.  The operands are swapped (B^T as the M-side
//     operand, A^T as the N-side one), so a lane's accumulators are four
//     consecutive columns of one C row and C leaves in 16-byte stores straight
//     from the registers.
// Needs N % 8 == 0 with 16-byte aligned B and C, N * 2 <= 16383 bytes (the
// record stride field) and A and B within 2 GiB each.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "amdgcn.h"
#include "engine.h"
#include "hip_status.h"

namespace spmm {
namespace engine {

namespace {

using namespace dev;

struct TileArgs {
    const int*      desc;  // panels x kTileDescInts
    const _Float16* vals;
    const _Float16* B;
    float*          C;
    int             M;
    int             K;
    int             N;
    int             tiles_n;   // column tiles of NT
    int             wg_total;  // panels * tiles_n
    int             num_blocks;
};

// Swizzle of a staged B row's 16-byte chunks: chunk c of staged row r sits at
// position c ^ swz(r).  The LDS has 64 four-byte banks (256 bytes per pass)
// and serves a ds_read_b64_tr_b16 in two passes of 32 lanes.  The four lanes
// of a row read 32 contiguous bytes (eight banks), so a pass is conflict-free
// when its eight rows land on eight different 8-bank groups.  A pair read
// (rows 8g + t/4, or + 4) puts rows r0 .. r0+3 and r0+8 .. r0+11 in a pass,
// a 16-deep read (rows 4g + t/4) rows r0 .. r0+7 (r0 a multiple of 16, or of
// 4 / 8 for the upper sets).  A row is 16 CH bytes, so 16 / CH rows share a
// 256-byte bank line and rows r, r' of a pass start on the same bank when
// r = r' mod 16 / CH; the swizzle moves a row's reads by s(r) = swz(r) / 2
// 32-byte units, and such rows need different s.  With x = bit 2 ^ bit 3 of
// r: s = x (CH = 4), s = bit 1 | x << 1 (CH = 8), s = (r & 3) | x << 2
// (CH = 16).  The period is 16 rows.
// (Swizzles built for 32 banks and 16-lane passes, 2 (r & 3) for CH >= 8 and
// 2 ((r >> 1) & 1) for CH = 4, left two rows of every pass on one group:
// two conflict cycles per read, rocprofv3 SQ_LDS_BANK_CONFLICT = 2 x
// SQ_INSTS_LDS.)
template <int CH>
__device__ __forceinline__ int tile_swz(int r) {
    const int x = ((r >> 2) ^ (r >> 3)) & 1;
    return CH >= 16 ? 2 * ((r & 3) | (x << 2))
         : CH == 8  ? 2 * (((r >> 1) & 1) | (x << 1))
         : CH == 4  ? 2 * x
                    : 0;
}

// Workgroup -> (panel, column tile).  The hardware hands workgroup L to XCD
// L % 8; logical ids are handed out so that XCD x gets a contiguous range of
// panels with all their column tiles, and panels that share B rows (a band,
// a diagonal block) are fetched into one L2.
__device__ __forceinline__ void tile_of(const TileArgs& a, int& panel, int& ct) {
    const int L = blockIdx.x;
    const int xcd = L & 7, idx = L >> 3;
    const int per = a.wg_total >> 3, rem = a.wg_total & 7;
    const int l = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    panel = l / a.tiles_n;
    ct    = l - panel * a.tiles_n;
}

template <int R, int NT, int WC, int CS, int NB, bool ONE>
__device__ __forceinline__ void tile_body(const TileArgs& a, _Float16* __restrict__ s0,
                                          _Float16* __restrict__ s1, _Float16* __restrict__ s2,
                                          _Float16* __restrict__ s3, _Float16* __restrict__ s4,
                                          _Float16* __restrict__ s5) {
    constexpr int WR   = 4 / WC;            // wave rows
    constexpr int RW   = R / WR;            // block-rows per wave
    constexpr int TC   = NT / 16 / WC;      // 16-column tiles per wave
    constexpr int CH   = NT / 8;            // 16-byte chunks per staged row
    constexpr int ROWS = CS * 16;           // staged B rows per chunk
    constexpr int LB   = ROWS * CH / 256;   // buffer-to-LDS loads per wave per chunk
    constexpr int PP   = CS / 2;            // slot pairs per chunk
    static_assert(WR * WC == 4 && R % WR == 0 && TC >= 1, "wave grid");
    static_assert(CS % 2 == 0 && (ROWS * CH) % 256 == 0, "chunk shape");
    static_assert(NB >= 2 && NB <= 6 && LB * (NB - 2) < 64, "ring depth");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr   = wave / WC;
    const int wc   = wave - wr * WC;
    const int g    = lane >> 4;
    const int t    = lane & 15;
    int panel, ct;
    tile_of(a, panel, ct);
    const int n0 = ct * NT;

    auto buf = [&](int b) -> _Float16* {
        return b == 0 ? s0 : b == 1 ? s1 : b == 2 ? s2 : b == 3 ? s3 : b == 4 ? s4 : s5;
    };

    // The panel record: union (u0, U) and this wave's block-rows' runs.
    const int* d = a.desc + static_cast<size_t>(panel) * kTileDescInts;
    const int u0 = d[0];
    const int U  = d[1];
    int lo[RW], hi[RW], ab[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        lo[i] = d[2 + wr * RW + i];
        hi[i] = d[2 + R + wr * RW + i];
        ab[i] = d[2 + 2 * R + wr * RW + i];
    }
    const int nch = (U + CS - 1) / CS;

    const u32x4 words_b = buffer_words(a.B, a.N * 2, a.K);
    const __amdgpu_buffer_rsrc_t rec_a = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a.vals), static_cast<short>(512), a.num_blocks, kBufWord3);

    // Buffer-to-LDS load c of this wave fills 16-byte positions
    // (4c + wave) * 64 + lane of a chunk buffer: staged row sr, position pos,
    // which holds chunk pos ^ swz(sr) of the row.  Columns past N read a valid
    // chunk of the row instead; their products land in output columns >= N,
    // which are never stored.
    int srow[LB], nbyte[LB];
#pragma unroll
    for (int c = 0; c < LB; ++c) {
        const int piece = (c * 4 + wave) * 64 + lane;
        srow[c] = piece / CH;
        const int n = n0 + ((piece % CH) ^ tile_swz<CH>(srow[c])) * 8;
        nbyte[c] = (n < a.N ? n : 0) * 2;
    }
    // Operand reads (fp16 units inside a pair's 32 staged rows).  Full pair:
    // rows 8g + t/4 (lo) and + 4 (hi) give lane 16g + t rows 8g .. 8g+7 of
    // column t.  Half pair (slot s of the pair): rows 16s + 4g + t/4 give rows
    // 4g .. 4g+3 of the slot's block.  Tile j' sits at 16-fp16 unit j' ^ h.
    const int r_lo = 8 * g + (t >> 2);
    const int sub  = ((t & 3) >> 1) * 8 + (t & 1) * 4;
    const int in_lo = r_lo * NT + sub, h_lo = tile_swz<CH>(r_lo) >> 1;
    const int in_hi = (r_lo + 4) * NT + sub, h_hi = tile_swz<CH>(r_lo + 4) >> 1;
    const int r_h0 = 4 * g + (t >> 2);
    const int in_h0 = r_h0 * NT + sub, h_h0 = tile_swz<CH>(r_h0) >> 1;
    const int in_h1 = (r_h0 + 16) * NT + sub, h_h1 = tile_swz<CH>(r_h0 + 16) >> 1;

    f32x4 acc[RW][TC];
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < TC; ++j) acc[i][j] = f32x4(0.0f);

    u32x4 af[NB][RW][PP];

    // A operands of chunk k into ring slot b: one 16-byte load per block-row
    // and pair whatever the pair holds, so every path issues the same loads
    // and the compiler's waits on them stay exact.  Both blocks: row t,
    // columns 8(g&1) .. +7 of block 2q + (g>>1) (the 16x32 operand).  One
    // block: row t, columns 4g .. 4g+3 of it (the 16x16 operand) are the low
    // half of the load at column 4g (g < 3) or the high half of the load at
    // column 8 (g = 3, which keeps the load inside the block).  Neither:
    // index -1 reads zeros without touching memory.
    const int off_full = t * 32 + 16 * (g & 1);
    const int off_half = t * 32 + (g < 3 ? 8 * g : 16);
    const int g_hi     = g >> 1;
    // Which slots of pair q0, q0 + 1 block-row i holds, as 0 / -1 masks
    // computed with scalar arithmetic (slot numbers are far below 2^30).
    auto holds = [&](int i, int q) { return ~((q - lo[i]) >> 31) & ((q - hi[i]) >> 31); };
    auto issue_a = [&](int k, int b) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
#pragma unroll
            for (int p = 0; p < PP; ++p) {
                const int q0 = 2 * (k * PP + p);
                const int m0 = holds(i, q0), m1 = holds(i, q0 + 1);
                const int full_m = m0 & m1;
                const int add = (g_hi & full_m) | (m1 & ~m0 & 1);
                const int idx = (ab[i] + q0 - lo[i] + add) | ~(m0 | m1);
                const int off = off_half ^ ((off_half ^ off_full) & full_m);
                af[b][i][p] = sbuf_load_u32x4(rec_a, idx, off, 0, 0);
                __builtin_amdgcn_sched_barrier(0);  // issue in program order, each as soon as ready
            }
        }
    };
    // B rows of chunk k into buffer b (rows past the union read zeros).
    auto issue_b = [&](int k, int b) {
        const unsigned dst = lds_address(buf(b));
        const int row0 = (u0 + k * CS) * 16;
        const int lim  = (U - k * CS) * 16;
#pragma unroll
        for (int c = 0; c < LB; ++c) {
            lds_dma_x4(words_b, dst + (c * 4 + wave) * 64 * 16,
                       srow[c] < lim ? row0 + srow[c] : -1, nbyte[c]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto compute = [&](int k, int b) {
        const _Float16* st = buf(b);
#pragma unroll
        for (int p = 0; p < PP; ++p) {
            const int q0 = 2 * (k * PP + p);
            const _Float16* pr = st + p * 32 * NT;
            bool full[RW], half[RW];
            bool any_full = false;
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                const int m0 = holds(i, q0), m1 = holds(i, q0 + 1);
                full[i] = (m0 & m1) != 0;
                half[i] = (m0 ^ m1) != 0;
                any_full = any_full || full[i];
            }
            if (any_full) {
                f16x8 bf[TC];
#pragma unroll
                for (int j = 0; j < TC; ++j) {
                    const int jj = wc * TC + j;
                    const s16x4 x = lds_read_tr16(pr + in_lo + (jj ^ h_lo) * 16);
                    const s16x4 y = lds_read_tr16(pr + in_hi + (jj ^ h_hi) * 16);
                    const s16x8 both = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                    bf[j] = __builtin_bit_cast(f16x8, both);
                }
#pragma unroll
                for (int i = 0; i < RW; ++i) {
                    if (full[i]) {
                        const f16x8 av = __builtin_bit_cast(f16x8, af[b][i][p]);
#pragma unroll
                        for (int j = 0; j < TC; ++j) {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], av,
                                                                               acc[i][j], 0, 0, 0);
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                if (half[i]) {
                    const bool first = holds(i, q0) != 0;  // the pair's first slot is the one held
                    const int in = first ? in_h0 : in_h1;
                    const int hh = first ? h_h0 : h_h1;
                    const u32x4 v = af[b][i][p];
                    const u32x2 a2 = g < 3 ? u32x2{v[0], v[1]} : u32x2{v[2], v[3]};
                    const f16x4 av = __builtin_bit_cast(f16x4, a2);
#pragma unroll
                    for (int j = 0; j < TC; ++j) {
                        const int jj = wc * TC + j;
                        const f16x4 bv =
                            __builtin_bit_cast(f16x4, lds_read_tr16(pr + in + (jj ^ hh) * 16));
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(bv, av, acc[i][j], 0,
                                                                          0, 0);
                    }
                }
            }
        }
    };
    // Every chunk issues the same LPC loads (chunks past the union read
    // nothing: index -1), so the loads in flight are known at compile time,
    // and before multiplying chunk k a wave waits until at most X loads are
    // out, X = the loads issued after chunk k's last B load (loads retire in
    // issue order).  The compiler waits for the A operands (VGPRs) itself.
    constexpr int LPC = LB + RW * PP;
    if constexpr (ONE) {
        // One shot: all NB chunks (the host guarantees the union fits) are
        // issued up front, A operands first, then the B rows chunk by chunk;
        // chunk b is multiplied as soon as its rows have landed.
        static_assert(NB * LPC < 64, "vmcnt is 6 bits");
#pragma unroll
        for (int b = 0; b < NB; ++b) issue_a(b, b);
#pragma unroll
        for (int b = 0; b < NB; ++b) issue_b(b, b);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b < nch) {
                switch (NB - 1 - b) {  // b is a constant once unrolled
                    case 0: wait_vmcnt<0>(); break;
                    case 1: wait_vmcnt<LB>(); break;
                    case 2: wait_vmcnt<2 * LB>(); break;
                    case 3: wait_vmcnt<3 * LB>(); break;
                    case 4: wait_vmcnt<4 * LB>(); break;
                    default: wait_vmcnt<(NB >= 6 ? 5 * LB : 0)>(); break;
                }
                lds_barrier();  // every wave's rows of chunk b have landed
                compute(b, b);
            }
        }
    } else {
        // Ring: the prologue issues the A operands of chunks 0 .. NB-2, then
        // their B rows; iteration k issues chunk k + NB - 1 (A, then B) into
        // the buffer of chunk k - 1.  X: in the first NB - 1 iterations the
        // prologue's later B rows plus the iterations' own chunks, afterwards
        // NB - 2 whole chunks.
        static_assert((NB - 1) * LPC < 64, "vmcnt is 6 bits");
        auto wait_chunk = [&](bool first, int b) {
            if (first && b <= NB - 2) {
                switch (b) {
                    case 0: wait_vmcnt<(NB - 2) * LB>(); break;
                    case 1: wait_vmcnt<(NB >= 3 ? (NB - 3) * LB + LPC : 0)>(); break;
                    case 2: wait_vmcnt<(NB >= 4 ? (NB - 4) * LB + 2 * LPC : 0)>(); break;
                    case 3: wait_vmcnt<(NB >= 5 ? (NB - 5) * LB + 3 * LPC : 0)>(); break;
                    default: wait_vmcnt<(NB >= 6 ? (NB - 6) * LB + 4 * LPC : 0)>(); break;
                }
            } else {
                wait_vmcnt<(NB - 2) * LPC>();
            }
        };
#pragma unroll
        for (int b = 0; b < NB - 1; ++b) issue_a(b, b);
#pragma unroll
        for (int b = 0; b < NB - 1; ++b) issue_b(b, b);
        for (int k0 = 0; k0 < nch; k0 += NB) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int k = k0 + b;
                if (k < nch) {
                    wait_chunk(k0 == 0, b);
                    // Every wave's loads of chunk k have landed, and every
                    // wave has finished multiplying chunk k - 1, whose buffer
                    // is refilled next.
                    lds_barrier();
                    const int nb = (b + NB - 1) % NB;
                    issue_a(k + NB - 1, nb);
                    issue_b(k + NB - 1, nb);
                    compute(k, b);
                }
            }
        }
    }
    wait_vmcnt<0>();  // the loads past the union, before the wave ends

    // Lane 16g + t holds C[row t][cols 4g .. 4g+3] of each 16x16 tile.
    const int rows_here = min(R * 16, a.M - panel * R * 16);
    const __amdgpu_buffer_rsrc_t c_rows = __builtin_amdgcn_make_buffer_rsrc(
        a.C + static_cast<size_t>(panel) * R * 16 * a.N, static_cast<short>(0),
        rows_here * a.N * 4, kBufWord3);
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const int r = (wr * RW + i) * 16 + t;
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            const int col = n0 + (wc * TC + j) * 16 + 4 * g;
            if (col < a.N) {  // rows past M fall outside the buffer and are dropped
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]),
                                                       c_rows, (r * a.N + col) * 4, 0,
                                                       kStoreDevice);
            }
        }
    }
}

// The chunk buffers are separate LDS objects passed as restrict pointers:
// after inlining every buffer access carries its own alias scope, so the
// compiler's wait-count pass can tell a read of one buffer from the
// buffer-to-LDS writes still in flight into the others.
template <int R, int NT, int WC, int CS, int NB, bool ONE>
__global__ __launch_bounds__(256) void bsr_tile_kernel(TileArgs a) {
    constexpr int BUF = CS * 16 * NT;
    __shared__ __attribute__((aligned(16))) _Float16 b0[BUF];
    __shared__ __attribute__((aligned(16))) _Float16 b1[BUF];
    __shared__ __attribute__((aligned(16))) _Float16 b2[NB >= 3 ? BUF : 8];
    __shared__ __attribute__((aligned(16))) _Float16 b3[NB >= 4 ? BUF : 8];
    __shared__ __attribute__((aligned(16))) _Float16 b4[NB >= 5 ? BUF : 8];
    __shared__ __attribute__((aligned(16))) _Float16 b5[NB >= 6 ? BUF : 8];
    tile_body<R, NT, WC, CS, NB, ONE>(a, b0, b1, b2, b3, b4, b5);
}

// ---------------------------------------------------------------------------
// Producer / consumer form (the whole union of a panel in LDS at once):
// NC + NP waves, waves NC .. NC+NP-1 only issue buffer-to-LDS loads of the
// panel's A blocks and B rows, chunk by chunk, and waves 0 .. NC-1 only
// multiply, so the multiplication of chunk k overlaps the loads of the
// chunks after it and no multiplying wave ever waits for the vector-memory
// issue queue (the launcher runs four of each: one or two producers, or
// eight consumers on twice the rows or columns, measured slower).  One
// workgroup barrier per chunk: a producer passes barrier k once its own
// loads of chunk k have landed, a consumer passes it before multiplying
// chunk k.
//   LDS: B rows of union slots 0 .. NB*CS-1 contiguously (16 rows per slot,
//   NT columns, 16-byte chunks XOR-swizzled by staged row), and the A blocks
//   of each block-row at slot granularity (512 bytes each).
//   Consumers pair each block-row's run from its own first slot (lo, lo+1),
//   (lo+2, lo+3), ... in 16x32 MFMAs and take an odd last block in a 16x16
//   one; a pair is multiplied at the barrier of the chunk holding its second
//   slot.  When the wave's block-rows share their run, a pair's B operand is
//   read once for all of them.
// ---------------------------------------------------------------------------
template <int R, int NT, int WC, int CS, int NB, bool AV, int NC, int NP>
__device__ __forceinline__ void pc_body(const TileArgs& a, _Float16* __restrict__ Bs,
                                        _Float16* __restrict__ As) {
    constexpr int WR  = NC / WC;         // consumer wave rows
    constexpr int RW  = R / WR;          // block-rows per consumer wave
    constexpr int TC  = NT / 16 / WC;    // 16-column tiles per consumer wave
    constexpr int CH  = NT / 8;          // 16-byte chunks per staged B row
    constexpr int NS  = NB * CS;         // union slots held
    constexpr int PP  = CS / 2;          // pairs completed per chunk and block-row (at most)
    constexpr int TA  = AV ? 0 : R * CS / 2;  // A loads per chunk (two blocks each)
    constexpr int TBL = CS * 16 * CH / 64;  // B loads per chunk
    constexpr int LPP = (TA + TBL) / NP;  // loads per producer wave per chunk
    static_assert(WR * WC == NC && R % WR == 0 && TC >= 1, "wave grid");
    static_assert(CS % 2 == 0 && (TA + TBL) % NP == 0, "chunk shape");
    static_assert(NB * LPP < 64, "vmcnt is 6 bits");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g    = lane >> 4;
    const int t    = lane & 15;
    int panel, ct;
    tile_of(a, panel, ct);
    const int n0 = ct * NT;

    // The record is read-only for the kernel's lifetime: read through the
    // constant address space, so it comes in with scalar loads.
    const __attribute__((address_space(4))) int* d =
        (const __attribute__((address_space(4))) int*)(a.desc) +
        static_cast<size_t>(panel) * kTileDescInts;
    const int u0 = d[0];
    const int U  = d[1];
    const int nch = (U + CS - 1) / CS;

    if (wave >= NC) {
        // ---- producer ----
        // Producer pw loads the A blocks of block-rows pw*RP .. pw*RP+RP-1
        // (two slots per load) and every fourth B load of each chunk.  Its
        // lane constants do not depend on the chunk: a chunk is CS*16 staged
        // rows, a multiple of the swizzle's period.
        constexpr int RP  = AV ? 1 : R / NP;   // block-rows per producer (A in LDS)
        constexpr int BPP = TBL / NP;          // B loads per producer per chunk
        static_assert((AV || R % NP == 0) && TBL % NP == 0 && (CS * 16) % 32 == 0,
                      "producer split");
        const int pw = wave - NC;
        int lo[RP], hi[RP], ab[RP];
#pragma unroll
        for (int q = 0; q < RP; ++q) {
            const int r = pw * RP + q;
            lo[q] = d[2 + r];
            hi[q] = d[2 + R + r];
            ab[q] = d[2 + 2 * R + r];
        }
        const u32x4 words_a = buffer_words(a.vals, 512, a.num_blocks);
        const u32x4 words_b = buffer_words(a.B, a.N * 2, a.K);
        const unsigned as_base = lds_address(As) + pw * RP * NS * 512;
        const unsigned bs_base = lds_address(Bs) + pw * 1024;
        const int half_lane = lane >> 5;          // A: which block of the load's two
        const int a_c       = lane & 31;          // A: 16-byte chunk position inside the block
        const int a_off     = (a_c ^ ((a_c >> 3) & 1)) * 16;  // the source chunk it holds
        int b_sr[BPP], b_nbyte[BPP];
#pragma unroll
        for (int s = 0; s < BPP; ++s) {
            const int piece = (NP * s + pw) * 64 + lane;
            b_sr[s] = piece / CH;  // staged row inside the chunk
            const int n = n0 + ((piece % CH) ^ tile_swz<CH>(b_sr[s])) * 8;
            b_nbyte[s] = (n < a.N ? n : 0) * 2;
        }
        // Chunk k's loads; the A blocks' 16-byte chunks are permuted inside
        // each block (chunk c at position c ^ ((c >> 3) & 1)), which makes
        // the consumers' 16-byte operand reads conflict-free.
        auto issue = [&](int k) {
#pragma unroll
            for (int q = 0; q < (AV ? 0 : RP); ++q) {
#pragma unroll
                for (int m = 0; m < CS / 2; ++m) {
                    const int v0 = k * CS + 2 * m;
                    const int v  = v0 + half_lane;
                    // a run slot of the block-row, or -1 (zeros, no memory access)
                    const int idx = (v >= lo[q] && v < hi[q]) ? ab[q] + v - lo[q] : -1;
                    lds_dma_x4(words_a, as_base + (q * NS + v0) * 512, idx, a_off);
                }
            }
#pragma unroll
            for (int s = 0; s < BPP; ++s) {
                const int rs  = k * CS * 16 + b_sr[s];  // staged row inside the panel
                const int row = rs < U * 16 ? u0 * 16 + rs : -1;
                lds_dma_x4(words_b, bs_base + (k * CS * 16 * NT + NP * s * 512) * 2, row,
                           b_nbyte[s]);
            }
        };
        // Loads run kLook chunks ahead of the barriers: after issuing chunk k
        // the producer waits for chunk k - kLook + 1 (the loads of the
        // kLook - 1 chunks after it may stay in flight) and passes its
        // barrier, so the consumers start on chunk 0 while later chunks are
        // still being issued.
        constexpr int kLook = 2;
        // (later < NB, so later * LPP < 64; the clamp only keeps the
        // unreachable cases' template arguments in range)
        constexpr int L1 = LPP < 64 ? LPP : 0, L2 = 2 * LPP < 64 ? 2 * LPP : 0;
        constexpr int L3 = 3 * LPP < 64 ? 3 * LPP : 0, L4 = 4 * LPP < 64 ? 4 * LPP : 0;
        constexpr int L5 = 5 * LPP < 64 ? 5 * LPP : 0;
        auto wait_chunks_out = [&](int later) {
            switch (later) {
                case 0: wait_vmcnt<0>(); break;
                case 1: wait_vmcnt<L1>(); break;
                case 2: wait_vmcnt<L2>(); break;
                case 3: wait_vmcnt<L3>(); break;
                case 4: wait_vmcnt<L4>(); break;
                default: wait_vmcnt<(NB >= 6 ? L5 : 0)>(); break;
            }
        };
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            issue(k);
            const int j = k - (kLook - 1);
            if (j >= 0 && j < nch) {
                wait_chunks_out(kLook - 1);
                lds_barrier();
            }
        }
#pragma unroll
        for (int j = NB - kLook + 1; j < NB; ++j) {
            if (j >= 0 && j < nch) {
                wait_chunks_out(NB - 1 - j);
                lds_barrier();
            }
        }
        wait_vmcnt<0>();  // the loads past the union, before the wave ends
        return;
    }

    // ---- consumer ----
    const int wr = wave / WC;
    const int wc = wave - wr * WC;
    int lo[RW], hi[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        lo[i] = d[2 + wr * RW + i];
        hi[i] = d[2 + R + wr * RW + i];
    }
    bool shared = true;
#pragma unroll
    for (int i = 1; i < RW; ++i) shared = shared && lo[i] == lo[0] && hi[i] == hi[0];
    // Pairs of block-row i completed by chunk k: [P(k), P(k+1)), P(k) = the
    // pairs whose second slot lies below slot k*CS.
    auto pairs_below = [&](int i, int slot) {
        const int x = slot >= lo[i] ? (slot - lo[i]) >> 1 : 0;
        return min(x, (hi[i] - lo[i]) >> 1);
    };
    // AV: the A operands come straight from global memory into VGPRs, all of
    // them before the first barrier: per chunk k, pair slot pp and block-row
    // i the 16x32 operand of pair P(k) + pp (row t, columns 8(g&1) .. +7 of
    // block 2p + (g>>1) of the run), index -1 (zeros, no memory access) when
    // the chunk completes fewer pairs; and per block-row the 16x16 operand of
    // an odd run's last block (row t, columns 4g .. 4g+3: the low half of a
    // 16-byte load at column 4g, or the high half of the load at column 8 for
    // g = 3, which keeps the load inside the block).  A consumer issues no
    // other loads, so the compiler's waits on them are exact.
    u32x4 avg[AV ? NB : 1][PP][RW];
    u32x4 avt[RW];
    if constexpr (AV) {
        const __amdgpu_buffer_rsrc_t rec_a = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>(a.vals), static_cast<short>(512), a.num_blocks, kBufWord3);
        const int off_full = t * 32 + 16 * (g & 1);
        const int off_half = t * 32 + (g < 3 ? 8 * g : 16);
        int ab[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) ab[i] = d[2 + 2 * R + wr * RW + i];
#pragma unroll
        for (int k = 0; k < NB; ++k) {
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                const int p0 = pairs_below(i, k * CS), p1 = pairs_below(i, (k + 1) * CS);
#pragma unroll
                for (int pp = 0; pp < PP; ++pp) {
                    const int p = p0 + pp;
                    const int idx = p < p1 ? ab[i] + 2 * p + (g >> 1) : -1;
                    avg[k][pp][i] = sbuf_load_u32x4(rec_a, idx, off_full, 0, 0);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int cnt = hi[i] - lo[i];
            avt[i] = sbuf_load_u32x4(rec_a, (cnt & 1) ? ab[i] + cnt - 1 : -1, off_half, 0, 0);
        }
    }

    f32x4 acc[RW][TC];
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < TC; ++j) acc[i][j] = f32x4(0.0f);

    // Lane constants of the operand reads.  B (fp16 units): a pair starting at
    // slot u reads staged rows 16u + 8g + t/4 (and + 4); a single block at
    // slot v rows 16v + 4g + t/4.  A (bytes): block (row, slot) at
    // (row * NS + slot) * 512, row t, columns 8(g&1) (pair, block slot +
    // (g>>1)) or 4g (single block).
    const int r_lo = 8 * g + (t >> 2);
    const int r_h  = 4 * g + (t >> 2);
    const int sub  = ((t & 3) >> 1) * 8 + (t & 1) * 4;
    const int a_x    = 2 * t + (g & 1);        // the A chunk a pair operand needs
    const int a_pair = (g >> 1) * 512 + (a_x ^ ((a_x >> 3) & 1)) * 16;
    const int a_y    = 2 * t + (g >> 1);       // the A chunk holding a single-block operand
    const int a_one  = (a_y ^ ((a_y >> 3) & 1)) * 16 + 8 * (g & 1);
    auto b_read = [&](int row, int jj) -> s16x4 {  // row: staged row this lane addresses
        return lds_read_tr16(Bs + row * NT + sub + ((jj ^ (tile_swz<CH>(row) >> 1)) * 16));
    };
    auto a_read8 = [&](int byte) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(As) + byte);
    };
    auto a_read4 = [&](int byte) -> f16x4 {
        return *reinterpret_cast<const f16x4*>(reinterpret_cast<const char*>(As) + byte);
    };
    auto compute = [&](int k) {
        if (shared) {
            const int p0 = pairs_below(0, k * CS), p1 = pairs_below(0, (k + 1) * CS);
            f16x8 bf[PP][TC];
            f16x8 af[PP][RW];
#pragma unroll
            for (int pp = 0; pp < PP; ++pp) {
                // reads are issued whether or not the pair exists (slot clamped
                // into the buffer), so their count is fixed
                const int u = min(lo[0] + 2 * (p0 + pp), NS - 2);
#pragma unroll
                for (int j = 0; j < TC; ++j) {
                    const s16x4 x = b_read(16 * u + r_lo, wc * TC + j);
                    const s16x4 y = b_read(16 * u + r_lo + 4, wc * TC + j);
                    const s16x8 both = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                    bf[pp][j] = __builtin_bit_cast(f16x8, both);
                }
#pragma unroll
                for (int i = 0; i < RW; ++i) {
                    if constexpr (AV) {
                        af[pp][i] = __builtin_bit_cast(f16x8, avg[k][pp][i]);
                    } else {
                        af[pp][i] = a_read8(((wr * RW + i) * NS + u) * 512 + a_pair);
                    }
                }
            }
#pragma unroll
            for (int pp = 0; pp < PP; ++pp) {
                if (p0 + pp < p1) {
#pragma unroll
                    for (int i = 0; i < RW; ++i)
#pragma unroll
                        for (int j = 0; j < TC; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[pp][j], af[pp][i],
                                                                               acc[i][j], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                const int p0 = pairs_below(i, k * CS), p1 = pairs_below(i, (k + 1) * CS);
                f16x8 bf[PP][TC];
                f16x8 af[PP];
#pragma unroll
                for (int pp = 0; pp < PP; ++pp) {
                    const int u = min(lo[i] + 2 * (p0 + pp), NS - 2);
#pragma unroll
                    for (int j = 0; j < TC; ++j) {
                        const s16x4 x = b_read(16 * u + r_lo, wc * TC + j);
                        const s16x4 y = b_read(16 * u + r_lo + 4, wc * TC + j);
                        const s16x8 both = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                        bf[pp][j] = __builtin_bit_cast(f16x8, both);
                    }
                    if constexpr (AV) {
                        af[pp] = __builtin_bit_cast(f16x8, avg[k][pp][i]);
                    } else {
                        af[pp] = a_read8(((wr * RW + i) * NS + u) * 512 + a_pair);
                    }
                }
#pragma unroll
                for (int pp = 0; pp < PP; ++pp) {
                    if (p0 + pp < p1) {
#pragma unroll
                        for (int j = 0; j < TC; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[pp][j], af[pp],
                                                                               acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        // An odd run's last block, in the chunk that holds it.
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int v = hi[i] - 1;
            if (((hi[i] - lo[i]) & 1) && v >= k * CS && v < (k + 1) * CS) {
                f16x4 av;
                if constexpr (AV) {
                    const u32x4 w = avt[i];
                    av = __builtin_bit_cast(f16x4, g < 3 ? u32x2{w[0], w[1]} : u32x2{w[2], w[3]});
                } else {
                    av = a_read4(((wr * RW + i) * NS + v) * 512 + a_one);
                }
#pragma unroll
                for (int j = 0; j < TC; ++j) {
                    const f16x4 bv = __builtin_bit_cast(f16x4, b_read(16 * v + r_h, wc * TC + j));
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(bv, av, acc[i][j], 0, 0, 0);
                }
            }
        }
    };
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        if (k < nch) {
            lds_barrier();  // chunk k has landed
            compute(k);
        }
    }

    // Lane 16g + t holds C[row t][cols 4g .. 4g+3] of each 16x16 tile.
    const int rows_here = min(R * 16, a.M - panel * R * 16);
    const __amdgpu_buffer_rsrc_t c_rows = __builtin_amdgcn_make_buffer_rsrc(
        a.C + static_cast<size_t>(panel) * R * 16 * a.N, static_cast<short>(0),
        rows_here * a.N * 4, kBufWord3);
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const int r = (wr * RW + i) * 16 + t;
#pragma unroll
        for (int j = 0; j < TC; ++j) {
            const int col = n0 + (wc * TC + j) * 16 + 4 * g;
            if (col < a.N) {  // rows past M fall outside the buffer and are dropped
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]),
                                                       c_rows, (r * a.N + col) * 4, 0,
                                                       kStoreDevice);
            }
        }
    }
}

template <int R, int NT, int WC, int CS, int NB, bool AV, int NC, int NP>
__global__ __launch_bounds__(64 * (NC + NP)) void bsr_tile_pc_kernel(TileArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 Bs[NB * CS * 16 * NT];
    __shared__ __attribute__((aligned(16))) _Float16 As[AV ? 8 : R * NB * CS * 256];
    pc_body<R, NT, WC, CS, NB, AV, NC, NP>(a, Bs, As);
}

template <int R, int NT, int WC, int CS, int NB, bool AV, int NC, int NP>
hipError_t run_tile_pc(TileArgs args, int panels, hipStream_t stream) {
    args.tiles_n = (args.N + NT - 1) / NT;
    const long total = static_cast<long>(panels) * args.tiles_n;
    if (total > 0x7fffffffL) return hipErrorInvalidConfiguration;
    args.wg_total = static_cast<int>(total);
    hipLaunchKernelGGL((bsr_tile_pc_kernel<R, NT, WC, CS, NB, AV, NC, NP>), dim3(args.wg_total),
                       dim3(64 * (NC + NP)), 0, stream, args);
    return hipGetLastError();
}

Error fail(int status, std::string msg) { return Error{status, std::move(msg)}; }

template <int R, int NT, int WC, int CS, int NB, bool ONE>
hipError_t run_tile(TileArgs args, int panels, hipStream_t stream) {
    args.tiles_n = (args.N + NT - 1) / NT;
    const long total = static_cast<long>(panels) * args.tiles_n;
    if (total > 0x7fffffffL) return hipErrorInvalidConfiguration;
    args.wg_total = static_cast<int>(total);
    hipLaunchKernelGGL((bsr_tile_kernel<R, NT, WC, CS, NB, ONE>), dim3(args.wg_total), dim3(256), 0,
                       stream, args);
    return hipGetLastError();
}

// One launcher per shape, instantiating only the kernel its kind names.
template <int R, int NT, int WC, int CS, int NB, int KIND>
hipError_t run_shape(TileArgs args, int panels, hipStream_t stream) {
    if constexpr (KIND >= 2) {
        return run_tile_pc<R, NT, WC, CS, NB, KIND == 3, 4, 4>(args, panels, stream);
    } else {
        return run_tile<R, NT, WC, CS, NB, KIND == 1>(args, panels, stream);
    }
}

}  // namespace

int tile_shape_count() { return static_cast<int>(sizeof(kTileShapes) / sizeof(kTileShapes[0])); }

// Measured on MI355X (c3: banded 8192^2 half-bandwidth 64, N = 128; c4:
// block-diagonal 32 x 256^2, N = 256; per launch, back to back): the producer
// / consumer forms beat the forms whose multiplying waves also issue the
// loads, and 32 (N <= 128) or 64 columns per workgroup beat wider tiles,
// whose fewer workgroups overlap less of each workgroup's load -> multiply
// -> store chain (c3 3.24 us at 32 columns, 3.30 at 64, 4.2 at 128; c4 4.34
// us at 64, 4.7 - 5.3 at 128, also with eight multiplying waves).  At 32
// columns consumers loading their A operands straight into VGPRs (KIND 3)
// win (c3 3.24 against 3.32 with A staged in LDS); at 64 columns on c4 A in
// LDS (KIND 2) does (4.34 against 4.48).  Unions wider than the one-shot
// forms hold take the ring.
int default_tile_shape(int R, int max_union, int M, int N) {
    const auto fits = [&](int id) {
        return kTileShapes[id].NB * kTileShapes[id].CS >= max_union;
    };
    if (R == 8) return fits(0) ? 0 : 11;
    if (N <= 128) return fits(14) ? 14 : fits(15) ? 15 : 10;
    return fits(3) ? 3 : 10;
}

int default_tile_rows(int M, int N) { return 4; }

namespace {
bool tile_plan_shape_ok(int R) { return R == 4 || R == 8; }
}  // namespace

Error bsr_tile_plan_from_host(const int* row_ptr, const int* col_idx, int block_rows,
                              int block_cols, int R, std::vector<int>* desc, int* max_union) {
    *max_union = 0;
    if (!tile_plan_shape_ok(R)) return fail(kInvalid, "panel block-rows must be 4 or 8");
    if (block_rows < 0 || block_cols < 0) return fail(kInvalid, "negative block dimension");
    const int panels = (block_rows + R - 1) / R;
    desc->assign(static_cast<size_t>(panels) * kTileDescInts, 0);
    for (int p = 0; p < panels; ++p) {
        int* d = desc->data() + static_cast<size_t>(p) * kTileDescInts;
        int first[8], last[8], cnt[8];
        int u0 = 0, u1 = 0;
        bool any = false;
        for (int r = 0; r < R; ++r) {
            const int br = p * R + r;
            cnt[r] = 0;
            if (br >= block_rows) continue;
            const int s = row_ptr[br], e = row_ptr[br + 1];
            if (s < 0 || e < s) return fail(kUnsupported, "row_ptr is not a prefix sum");
            cnt[r] = e - s;
            if (cnt[r] == 0) continue;
            first[r] = col_idx[s];
            last[r]  = col_idx[e - 1];
            // a run: strictly consecutive block-columns inside the matrix
            if (first[r] < 0 || last[r] >= block_cols || last[r] - first[r] + 1 != cnt[r]) {
                return fail(kUnsupported, "a block-row is not a run of consecutive block-columns");
            }
            for (int x = s + 1; x < e; ++x) {
                if (col_idx[x] != col_idx[x - 1] + 1) {
                    return fail(kUnsupported,
                                "a block-row is not a run of consecutive block-columns");
                }
            }
            if (!any || first[r] < u0) u0 = first[r];
            if (!any || last[r] + 1 > u1) u1 = last[r] + 1;
            any = true;
        }
        if (!any) continue;  // all zero: U = 0, the panel stores zeros
        // The union must be covered without gaps (every staged slot is used).
        std::vector<char> cover(static_cast<size_t>(u1 - u0), 0);
        for (int r = 0; r < R; ++r) {
            if (cnt[r] > 0) std::fill(cover.begin() + (first[r] - u0), cover.begin() + (last[r] + 1 - u0), 1);
        }
        if (std::find(cover.begin(), cover.end(), 0) != cover.end()) {
            return fail(kUnsupported, "a panel's runs leave a gap");
        }
        d[0] = u0;
        d[1] = u1 - u0;
        *max_union = std::max(*max_union, u1 - u0);
        for (int r = 0; r < R; ++r) {
            const int br = p * R + r;
            if (cnt[r] == 0) continue;
            d[2 + r]         = first[r] - u0;
            d[2 + R + r]     = first[r] - u0 + cnt[r];
            d[2 + 2 * R + r] = row_ptr[br];
        }
    }
    return Error{};
}

Error bsr_tile_plan_build(const BSR& d_A, int R, BsrTilePlan* out, hipStream_t stream) {
    *out = BsrTilePlan{};
    if (d_A.block_rows < 0 || d_A.num_blocks < 0) return fail(kInvalid, "negative matrix dimension");
    std::vector<int> rp(static_cast<size_t>(d_A.block_rows) + 1), ci(static_cast<size_t>(d_A.num_blocks));
    if (d_A.row_ptr == nullptr || (d_A.num_blocks > 0 && d_A.col_idx == nullptr)) {
        return fail(kInvalid, "null device pointer");
    }
    SPMM_TRY_HIP(hipMemcpyAsync(rp.data(), d_A.row_ptr, sizeof(int) * rp.size(),
                                hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    if (!ci.empty()) {
        SPMM_TRY_HIP(hipMemcpyAsync(ci.data(), d_A.col_idx, sizeof(int) * ci.size(),
                                    hipMemcpyDeviceToHost, stream), "hipMemcpyAsync");
    }
    SPMM_TRY_HIP(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (rp[0] != 0 || rp.back() != d_A.num_blocks) {
        return fail(kUnsupported, "row_ptr does not span the blocks");
    }
    std::vector<int> desc;
    int max_union = 0;
    SPMM_TRY(bsr_tile_plan_from_host(rp.data(), ci.data(), d_A.block_rows, d_A.block_cols, R,
                                     &desc, &max_union));
    SPMM_TRY_HIP(hipMalloc(&out->desc, sizeof(int) * (desc.empty() ? 1 : desc.size())), "hipMalloc");
    const hipError_t e =
        hipMemcpy(out->desc, desc.data(), sizeof(int) * desc.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        bsr_tile_plan_free(out);
        return hip_error(e, "hipMemcpy");
    }
    out->R          = R;
    out->panels     = static_cast<int>(desc.size() / kTileDescInts);
    out->num_rows   = d_A.num_rows;
    out->num_cols   = d_A.num_cols;
    out->block_rows = d_A.block_rows;
    out->num_blocks = d_A.num_blocks;
    out->max_union  = max_union;
    out->row_ptr    = d_A.row_ptr;
    out->col_idx    = d_A.col_idx;
    return Error{};
}

void bsr_tile_plan_free(BsrTilePlan* p) {
    if (p->desc) (void)hipFree(p->desc);
    *p = BsrTilePlan{};
}

Error launch_bsr_tile(const BsrTilePlan& plan, const BSR& A, const half* B, float* C, int N,
                      hipStream_t stream, int shape) {
    if (N < 0) return fail(kInvalid, "negative matrix dimension");
    if (plan.desc == nullptr && plan.panels > 0) return fail(kInvalid, "empty plan");
    if (A.num_rows != plan.num_rows || A.num_cols != plan.num_cols ||
        A.block_rows != plan.block_rows || A.num_blocks != plan.num_blocks ||
        A.row_ptr != plan.row_ptr || A.col_idx != plan.col_idx) {
        return fail(kInvalid, "the plan was built for another matrix");
    }
    if (A.num_rows == 0 || N == 0) return Error{};
    if (B == nullptr || C == nullptr || (A.num_blocks > 0 && A.values == nullptr)) {
        return fail(kInvalid, "null device pointer");
    }
    if (N % 8 != 0 || reinterpret_cast<uintptr_t>(B) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(C) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(A.values) % 16 != 0) {
        return fail(kUnsupported, "the run-panel kernel needs N % 8 == 0 and 16-byte aligned "
                                  "B, C and values");
    }
    if (static_cast<long long>(N) * 2 > 16383 ||
        static_cast<long long>(A.num_cols) * N * 2 > 0x7fffffffLL ||
        static_cast<long long>(A.num_blocks) * 512 > 0x7fffffffLL ||
        static_cast<long long>(plan.R) * 16 * N * 4 > 0x7fffffffLL) {
        return fail(kUnsupported, "operands outside the kernel's buffer records");
    }
    if (shape < 0) shape = default_tile_shape(plan.R, plan.max_union, A.num_rows, N);
    if (shape >= tile_shape_count() || kTileShapes[shape].R != plan.R) {
        return fail(kInvalid, "tile shape does not match the plan");
    }
    if (kTileShapes[shape].KIND != 0 &&
        kTileShapes[shape].NB * kTileShapes[shape].CS < plan.max_union) {
        return fail(kInvalid, "the plan's widest union does not fit this one-shot tile shape");
    }
    TileArgs args{plan.desc,
                  reinterpret_cast<const _Float16*>(A.values),
                  reinterpret_cast<const _Float16*>(B),
                  C,
                  A.num_rows,
                  A.num_cols,
                  N,
                  0,
                  0,
                  A.num_blocks};
    hipError_t e = hipSuccess;
    switch (shape) {
#define SPMM_TILE_CASE(ID, R_, NT_, WC_, CS_, NB_, KIND_) \
    case ID: e = run_shape<R_, NT_, WC_, CS_, NB_, KIND_>(args, plan.panels, stream); break;
        SPMM_TILE_SHAPES(SPMM_TILE_CASE)
#undef SPMM_TILE_CASE
        default: return fail(kInvalid, "unknown tile shape");
    }
    if (e != hipSuccess) return fail(kHipError, std::string("bsr_tile launch: ") + hipGetErrorString(e));
    return Error{};
}

}  // namespace engine
}  // namespace spmm
