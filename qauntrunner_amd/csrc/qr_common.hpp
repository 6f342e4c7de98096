// qr_common.hpp -- shared host/device helpers of libqr_attn (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "qr_attn.h"

namespace qr {

constexpr int kPageTokens = QR_PAGE_TOKENS;
constexpr int kPageShift = 8;  // log2(kPageTokens)

// ---------------------------------------------------------------- errors
// Thread-local message behind qr_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define QR_CHECK_ARG(cond, ...)                \
    do {                                       \
        if (!(cond)) {                         \
            ::qr::set_error(__VA_ARGS__);      \
            return QR_ERR_INVALID_ARGUMENT;    \
        }                                      \
    } while (0)

#define QR_HIP(call)                                                                  \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) {                                                       \
            ::qr::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),    \
                            __FILE__, __LINE__);                                      \
            return e_ == hipErrorOutOfMemory ? QR_ERR_OUT_OF_MEMORY : QR_ERR_HIP;     \
        }                                                                             \
    } while (0)

#define QR_TRY(expr)                 \
    do {                             \
        int s_ = (expr);             \
        if (s_ != QR_OK) return s_;  \
    } while (0)

__host__ __device__ inline int dtype_size(int dt) { return dt == QR_DTYPE_F32 ? 4 : 2; }
__host__ __device__ inline bool dtype_valid(int dt) {
    return dt == QR_DTYPE_F32 || dt == QR_DTYPE_F16 || dt == QR_DTYPE_BF16;
}

// ---------------------------------------------------------------- separately rounded ops
// One IEEE fp32 multiply / add / subtract each, never fused into an FMA.  clang's HIP
// __fmul_rn and friends are plain operators that inherit contraction from where they
// are defined; these carry the pragma in their own bodies, so each product is rounded
// before it is added, as the reference's RyuJIT code rounds it.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// ---------------------------------------------------------------- device scalar codecs
// 16-bit values travel as raw bits.  Decoding is exact.  Encoding follows the
// reference codecs: Dtypes.FloatToF16 (Dtypes.cs:100-126) and
// Dtypes.FloatToBf16 (Dtypes.cs:132-139).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));  // v_cvt_f32_f16: exact, subnormals kept
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Normal range: add half an ulp of the target (bit 12) and truncate, so ties
// go away from zero.  Below 2^-14: round to nearest even on the dropped bits.
__device__ __forceinline__ uint16_t f32_to_f16_bits_ref(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t biased = (x >> 23) & 0xFFu;
    int e = static_cast<int>(biased) - 127;
    const uint32_t man = x & 0x7FFFFFu;
    if (biased == 0xFFu) return static_cast<uint16_t>(sign | 0x7C00u | (man ? 0x200u : 0u));
    if (e > 15) return static_cast<uint16_t>(sign | 0x7C00u);
    if (e >= -14) {
        uint32_t r = man + 0x1000u;
        if (r & 0x800000u) { r = 0; ++e; }
        return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e + 15) << 10) | (r >> 13));
    }
    if (e < -25) return static_cast<uint16_t>(sign);
    const uint32_t full = 0x800000u | man;
    const int shift = -e - 1;  // 14..24: keeps the bits at or above 2^-24
    uint32_t q = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return static_cast<uint16_t>(sign | q);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits_ref(float f) {
    uint32_t x = __float_as_uint(f);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return static_cast<uint16_t>(x >> 16);
}

// ---------------------------------------------------------------- wave64 lane exchange
// DPP moves within a 16-lane row.  Every pattern used here maps a lane to a
// partner lane of the same row, so bound_ctrl never substitutes zero.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, true));
}
// quad_perm(1,0,3,2): partner = lane ^ 1
__device__ __forceinline__ float dpp_xor1(float v) { return dpp_mov<0xB1>(v); }
// quad_perm(2,3,0,1): partner = lane ^ 2
__device__ __forceinline__ float dpp_xor2(float v) { return dpp_mov<0x4E>(v); }
// row_half_mirror: lane i <-> 7-i inside each group of 8 (swaps the two quads)
__device__ __forceinline__ float dpp_half_mirror(float v) { return dpp_mov<0x141>(v); }
// row_mirror: lane i <-> 15-i inside each row of 16 (swaps the two halves)
__device__ __forceinline__ float dpp_mirror(float v) { return dpp_mov<0x140>(v); }

// Sum over aligned groups of `lanes` consecutive lanes (1, 2, 4, 8, 16 or 32).
// Every lane of a group ends with the bit-identical group sum, because each
// step adds the same two operands in every lane (IEEE addition commutes).
__device__ __forceinline__ float group_sum(float x, int lanes) {
    if (lanes >= 2) x += dpp_xor1(x);
    if (lanes >= 4) x += dpp_xor2(x);
    if (lanes >= 8) x += dpp_half_mirror(x);
    if (lanes >= 16) x += dpp_mirror(x);
    if (lanes >= 32) x += __shfl_xor(x, 16);
    return x;
}

// Pair reductions across rows of 16 lanes (gfx950 v_permlane16_swap / v_permlane32_swap,
// no LDS round trip): every lane gets op(x of its lane, x of lane ^ 16) (resp. ^ 32).
// The swap hands each lane the values of both lanes of its pair (element 0 the lower
// lane's, element 1 the upper's, checked on gfx950), so both lanes combine the same two
// operands in the same order and end bit-identical.
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Raw buffer resources and the cache-policy bits of the buffer intrinsics (gfx9 family).
constexpr int kBufferFlags = 0x00020000;  // raw buffer resource word 3
constexpr int kCacheSc1 = 16;             // sc1: device scope
constexpr int kCacheNt = 2;               // nt: streamed data, read once (whole lines per wave load)

// ---------------------------------------------------------------- 16-byte vector loads
struct alignas(16) U32x4 { uint32_t x, y, z, w; };

__device__ __forceinline__ U32x4 load16(const void* p) {
    return *reinterpret_cast<const U32x4*>(p);
}

// Widen one 16-byte chunk of cache elements to fp32.
template <typename KT> struct Chunk;
template <> struct Chunk<float> {
    static constexpr int kElems = 4;
    __device__ __forceinline__ static void widen(const U32x4& c, float* o) {
        o[0] = __uint_as_float(c.x); o[1] = __uint_as_float(c.y);
        o[2] = __uint_as_float(c.z); o[3] = __uint_as_float(c.w);
    }
};
struct F16Tag {};
struct BF16Tag {};
template <> struct Chunk<F16Tag> {
    static constexpr int kElems = 8;
    __device__ __forceinline__ static void widen(const U32x4& c, float* o) {
        const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = f16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xFFFFu));
            o[2 * i + 1] = f16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
        }
    }
};
template <> struct Chunk<BF16Tag> {
    static constexpr int kElems = 8;
    __device__ __forceinline__ static void widen(const U32x4& c, float* o) {
        const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(w[i] << 16);
            o[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
};

}  // namespace qr
