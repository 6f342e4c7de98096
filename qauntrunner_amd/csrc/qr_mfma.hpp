// qr_mfma.hpp -- shared device helpers of the MFMA kernels (gfx950): operand types,
// LDS barriers and the buffer-load LDS DMA.
#pragma once

#include "qr_common.hpp"

#include <type_traits>

namespace qr {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// v_mfma_f32_16x16x32_{f16,bf16}; lane layout (checked on gfx950):
//   A[m = lane%16][k = 8*(lane/16)+i], B[k = 8*(lane/16)+i][n = lane%16],
//   D[m = 4*(lane/16)+r][n = lane%16].
__device__ __forceinline__ f32x4_t mfma16(f16x8_t a, f16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Workgroup barrier ordering LDS only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup barrier for data written with ds_write while an LDS-DMA is in flight:
// it waits for this wave's LDS instructions (lgkmcnt) only.
__device__ __forceinline__ void lds_barrier_dma_in_flight() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding: vmcnt bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).  The empty asm with a memory clobber keeps
// the compiler from moving LDS reads of DMA-written data above the wait (the waitcnt
// builtin itself is not a memory operation for the optimiser).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
    asm volatile("" ::: "memory");
}
// this wave's LDS-DMA writes have all landed
__device__ __forceinline__ void wait_dma() { wait_vmcnt<0>(); }


// 16 bytes per lane from a raw buffer into LDS at lds + 16 * lane (buffer_load_dwordx4
// ... lds); out-of-range offsets read zeros.  `lds` must be the same for every lane of
// the wave (it becomes M0, which the compiler sets).  The compiler does not track when
// an LDS DMA lands, so completion is awaited explicitly (wait_vmcnt, then a barrier when
// other waves read the data) before the data is read.
template <int AUX = 0>
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, const char* lds, uint32_t voffset,
                                                  uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (__attribute__((address_space(3))) void*)(const_cast<char*>(lds)), 16, voffset, soffset, 0, AUX);
}

}  // namespace qr
