// Design study, not part of the engine: the data movement of an SpMM kernel
// that keeps a column slice of B resident in LDS instead of gathering B rows
// through the vector-memory path, measured on the volumes of a uniform CSR
// matrix (c2: M = K = 8192, 82 entries per row, N = 128).
//
// Shape under study: a workgroup owns 256 rows x a 16-column slice of B and C
// (16 waves, a quad of lanes per row, 4 floats per lane).  It stages its B
// slice in chunks of KC rows with buffer-to-LDS loads (triple buffer, one
// barrier per chunk), and every quad reads `per_row` staged B rows in total,
// spread evenly over the chunks, at pseudo-random positions inside each chunk.
// A (column indices and values) is not read at all: the skeleton measures the
// ceiling of the design before its A traffic and row bookkeeping.
//
// Modes (one kernel instantiation each, so a kernel trace tells them apart):
//   base      barriers and C stores only
//   fills     + the B-slice chunk fills
//   lds       + the LDS reads, no fills
//   both      fills and LDS reads: the design's ceiling
//   lds_half  the LDS reads with half the quads masked in each read and twice
//             the read instructions (how partly idle reads cost)
//
//   slab_skeleton [--m 8192] [--n 128] [--per-row 82] [--kc 512|768]
//                 [--reps 50] [--mode all|base|fills|lds|both|lds_half]

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Structured buffer load straight into LDS (LLVM's AMDGPU intrinsic): lane
// i's `size` bytes land at p + 16 * i.
__device__ void sbuf_load_lds(__amdgpu_buffer_rsrc_t rsrc, lds_ptr_t p, int size, int index,
                              int offset, int soffset, int imm_offset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.lds");

#define CHECK(x)                                                                        \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            std::exit(1);                                                               \
        }                                                                               \
    } while (0)

namespace {

enum Mode { kBase = 0, kFills = 1, kLds = 2, kBoth = 3, kLdsHalf = 6 };

constexpr int kWaves   = 16;
constexpr int kRowsWg  = kWaves * 16;  // a quad per row, 16 rows per wave
constexpr int kSlice   = 16;           // columns of B and C per workgroup

template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int KC, int MODE>
__global__ __launch_bounds__(kWaves * 64) void slab_skeleton_kernel(const float* B, float* C,
                                                                    int M, int K, int N,
                                                                    int per_row) {
    constexpr bool FILLS = (MODE & 1) != 0;
    constexpr bool READS = (MODE & 2) != 0;
    constexpr bool HALF  = (MODE & 4) != 0;
    constexpr int  FPL   = KC / kRowsWg;  // fill instructions per lane per chunk
    static_assert(KC % kRowsWg == 0, "whole fill instructions");
    __shared__ f32x4 buf[3][KC * 4];

    const int lane  = threadIdx.x & 63;
    const int wave  = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q     = lane & 3;
    const int quad  = lane >> 2;
    const int S     = N / kSlice;
    const int s     = blockIdx.x % S;  // slice s of every row block: XCD s % 8
    const int rb    = blockIdx.x / S;
    const int row   = rb * kRowsWg + wave * 16 + quad;
    const int c0    = s * kSlice;
    const int nch   = (K + KC - 1) / KC;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(B), static_cast<short>(N * 4), K, 0x00020000);

    // Chunk ch: B rows ch*KC .. +KC-1 (rows >= K read zeros), 64 bytes of
    // each, into buffer ch % 3; a wave's instruction fills 16 rows.
    auto fill = [&](int ch) {
        f32x4* dst = buf[ch % 3];
#pragma unroll
        for (int i = 0; i < FPL; ++i) {
            const int r = i * kRowsWg + wave * 16;
            sbuf_load_lds(rsrc, (lds_ptr_t)(dst + r * 4), 16, ch * KC + r + quad,
                          (c0 + q * 4) * 4, 0, 0, 0);
        }
    };
    f32x4 acc = f32x4(0.0f);
    unsigned h = static_cast<unsigned>(row) * 2654435761u + 12345u;
    const int base_cnt = per_row / nch;
    const int extra    = per_row - base_cnt * nch;
    if constexpr (FILLS) {
        fill(0);
        if (nch > 1) fill(1);
    } else {
        // Without fills the buffers still get defined contents once, so the
        // compiler cannot fold the reads of never-written LDS away.
        for (int i = threadIdx.x; i < 3 * KC * 4; i += kWaves * 64) {
            buf[i / (KC * 4)][i % (KC * 4)] = f32x4(static_cast<float>(i & 7));
        }
    }
    for (int ch = 0; ch < nch; ++ch) {
        if constexpr (FILLS) {
            if (ch + 1 < nch) wait_vmcnt<FPL>();  // chunk ch landed, ch + 1 may be in flight
            else wait_vmcnt<0>();
        }
        lds_barrier();  // chunk ch visible; every wave is done with chunk ch - 1
        if constexpr (FILLS) {
            if (ch + 2 < nch) fill(ch + 2);  // into the buffer chunk ch - 1 used
        }
        if constexpr (READS) {
            const f32x4* src = buf[ch % 3];
            const int cnt = base_cnt + (ch < extra ? 1 : 0);
            const int steps = HALF ? 2 * cnt : cnt;
            for (int j = 0; j < steps; ++j) {
                h = h * 1664525u + 1013904223u;
                const int r = static_cast<int>((h >> 8) % KC);
                if (!HALF || ((j + quad) & 1) == 0) acc += src[r * 4 + q] * static_cast<float>(j + 1);
            }
        }
    }
    if (row < M) {
        __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(C + static_cast<size_t>(row) * N +
                                                                  c0 + q * 4));
    }
}

struct Args {
    int m = 8192, n = 128, per_row = 82, kc = 768, reps = 50;
    std::string mode = "all";
};

template <int KC, int MODE>
double time_mode(const Args& a, const float* B, float* C) {
    const dim3 grid((a.m / kRowsWg) * (a.n / kSlice));
    auto launch = [&] {
        hipLaunchKernelGGL((slab_skeleton_kernel<KC, MODE>), grid, dim3(kWaves * 64), 0, 0, B, C,
                           a.m, a.m, a.n, a.per_row);
    };
    for (int i = 0; i < 5; ++i) launch();
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    std::vector<float> per;
    for (int b = 0; b < 5; ++b) {
        CHECK(hipEventRecord(e0));
        for (int i = 0; i < a.reps; ++i) launch();
        CHECK(hipEventRecord(e1));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        per.push_back(ms * 1e3f / a.reps);
    }
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    std::sort(per.begin(), per.end());
    return per[per.size() / 2];
}

template <int KC>
void run_all(const Args& a, const float* B, float* C) {
    struct M {
        const char* name;
        double (*fn)(const Args&, const float*, float*);
    };
    const M modes[] = {{"base", &time_mode<KC, kBase>},
                       {"fills", &time_mode<KC, kFills>},
                       {"lds", &time_mode<KC, kLds>},
                       {"both", &time_mode<KC, kBoth>},
                       {"lds_half", &time_mode<KC, kLdsHalf>}};
    for (const M& m : modes) {
        if (a.mode != "all" && a.mode != m.name) continue;
        const double us = m.fn(a, B, C);
        std::printf("mode=%s kc=%d m=%d n=%d per_row=%d us=%.2f\n", m.name, KC, a.m, a.n,
                    a.per_row, us);
        std::fflush(stdout);
    }
}

}  // namespace

int main(int argc, char** argv) {
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string k = argv[i];
        if (i + 1 >= argc) {
            std::fprintf(stderr, "missing value for %s\n", k.c_str());
            return 2;
        }
        const char* v = argv[++i];
        if (k == "--m") a.m = std::atoi(v);
        else if (k == "--n") a.n = std::atoi(v);
        else if (k == "--per-row") a.per_row = std::atoi(v);
        else if (k == "--kc") a.kc = std::atoi(v);
        else if (k == "--reps") a.reps = std::atoi(v);
        else if (k == "--mode") a.mode = v;
        else {
            std::fprintf(stderr, "unknown option %s\n", k.c_str());
            return 2;
        }
    }
    if (a.m <= 0 || a.m % kRowsWg != 0 || a.n <= 0 || a.n % kSlice != 0 || a.n * 4 > 16383 ||
        a.per_row < 0 || a.reps <= 0 || (a.kc != 512 && a.kc != 768)) {
        std::fprintf(stderr,
                     "need --m a multiple of %d, --n a multiple of %d with n*4 <= 16383, "
                     "--kc 512 or 768, --reps > 0\n", kRowsWg, kSlice);
        return 2;
    }
    float *B = nullptr, *C = nullptr;
    CHECK(hipMalloc(&B, static_cast<size_t>(a.m) * a.n * 4));
    CHECK(hipMalloc(&C, static_cast<size_t>(a.m) * a.n * 4));
    CHECK(hipMemset(B, 0, static_cast<size_t>(a.m) * a.n * 4));
    if (a.kc == 512) run_all<512>(a, B, C);
    else run_all<768>(a, B, C);
    CHECK(hipFree(B));
    CHECK(hipFree(C));
    return 0;
}
