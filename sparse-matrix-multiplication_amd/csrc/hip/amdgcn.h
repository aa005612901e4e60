#pragma once
// gfx950 device helpers shared by the BSR matrix-core kernels: structured
// buffer loads (to VGPRs and straight into LDS), the transposing LDS read that
// builds K-contiguous MFMA operands, and explicit wait / barrier forms.

#include <hip/hip_runtime.h>

#include <cstdint>

typedef unsigned spmm_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned spmm_u32x2 __attribute__((ext_vector_type(2)));

// Structured buffer loads (LLVM's AMDGPU intrinsics; index = record, offset =
// byte offset inside the record).  The intrinsic names are fixed by LLVM.  An
// index at or past the buffer's record count reads zeros and touches no
// memory (index -1 is used for "absent").
__device__ spmm_u32x4 sbuf_load_u32x4(__amdgpu_buffer_rsrc_t rsrc, int index, int offset,
                                      int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");
__device__ spmm_u32x2 sbuf_load_u32x2(__amdgpu_buffer_rsrc_t rsrc, int index, int offset,
                                      int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v2i32");
// Structured buffer load straight into LDS: every lane's `size` bytes land at
// the LDS address p + size * lane (gfx950 LDS DMA), nothing passes through VGPRs.
typedef __attribute__((address_space(3))) void* spmm_lds_ptr;
__device__ void sbuf_load_lds(__amdgpu_buffer_rsrc_t rsrc, spmm_lds_ptr p, int size, int index,
                              int offset, int soffset, int imm_offset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.lds");

namespace spmm {
namespace engine {
namespace dev {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef short    s16x4 __attribute__((ext_vector_type(4)));
typedef short    s16x8 __attribute__((ext_vector_type(8)));

// Third dword of a gfx9 buffer resource: 32-bit data format, no swizzle.
constexpr int kBufWord3 = 0x00020000;

// Cache-policy operand of a buffer store with device scope (the sc1 bit).
constexpr int kStoreDevice = 16;

// ds_read_b64_tr_b16.  Within each 16-lane block, lane s supplies the address
// of 4 consecutive fp16 values and output lane i receives element i % 4 of
// the values addressed by lanes 4e + i/4, e = 0..3: with lane s pointing at
// row r0 + s/4, columns c0 + 4*(s%4) .. +3 of a row-major [k][n] tile, lane i
// gets rows r0 .. r0+3 of column c0 + i -- a K-contiguous MFMA operand.
__device__ __forceinline__ s16x4 lds_read_tr16(const _Float16* p) {
    // generic -> LDS address-space cast; p always points into a __shared__ array
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(const_cast<_Float16*>(p)));
}

// s_waitcnt constraining only the vector-memory count (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    __builtin_amdgcn_sched_barrier(0);
}

// A gfx9 buffer resource as four SGPR words: base address, record stride in
// bytes (14 bits), record count, and kBufWord3.
__device__ __forceinline__ u32x4 buffer_words(const void* base, int stride, int records) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(base);
    return u32x4{static_cast<unsigned>(a),
                 static_cast<unsigned>((a >> 32) & 0xffffu) | (static_cast<unsigned>(stride) << 16),
                 static_cast<unsigned>(records), static_cast<unsigned>(kBufWord3)};
}

// Structured 16-byte-per-lane buffer load into LDS (lane i's bytes land at
// LDS address lds + 16 i), issued as inline assembly.  The compiler then does
// not know that these loads write LDS, so it adds no waits of its own before
// LDS reads; the caller waits (vmcnt) and synchronises before reading the
// data.  The loads still count in vmcnt: callers that count their loads
// include them, and the compiler's own vmcnt waits (for loads it issued)
// only grow stricter from loads it does not see.
// M0 carries the LDS address.  The kernels that use this issue no other
// instruction that reads M0, so no value of the compiler's lives there.
__device__ __forceinline__ void lds_dma_x4(u32x4 rsrc, unsigned lds, int index, int offset) {
    const u32x2 va = {static_cast<unsigned>(index), static_cast<unsigned>(offset)};
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 idxen offen lds"
        :
        : "s"(lds), "v"(va), "s"(rsrc)
        : "m0");
#pragma clang diagnostic pop
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_address(const void* p) {
    return static_cast<unsigned>(reinterpret_cast<uintptr_t>(
        (__attribute__((address_space(3))) const void*)(p)));
}

// Workgroup barrier without a memory fence: the caller has already waited
// for the LDS writes (and buffer-to-LDS loads) its partners must see.  The
// memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace dev
}  // namespace engine
}  // namespace spmm
