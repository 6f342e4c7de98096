// qr_dequant.hpp -- weight-row formats (QuantFormat, Dtypes.cs:6-50) and device decoders
// that reproduce BlockDequantizer.Dequantize (Core/Quantization/BlockDequantizer.cs)
// bit for bit: every multiply and subtract is one separately rounded fp32 operation
// (mul_rn / sub_rn), as the reference's RyuJIT scalar code performs it.
#pragma once

#include "qr_common.hpp"

namespace qr {

struct FormatSpec {
    int block;  // weights per block
    int bytes;  // bytes per block
};

// Dtypes.cs:38-50 for the formats decoded on the device.
__host__ __device__ inline bool weight_format_spec(int fmt, FormatSpec* s) {
    switch (fmt) {
    case QR_FMT_F32: *s = {1, 4}; return true;
    case QR_FMT_F16: *s = {1, 2}; return true;
    case QR_FMT_BF16: *s = {1, 2}; return true;
    case QR_FMT_Q4_0: *s = {32, 20}; return true;
    case QR_FMT_Q8_0: *s = {32, 34}; return true;
    case QR_FMT_Q4_K: *s = {256, 144}; return true;
    case QR_FMT_Q6_K: *s = {256, 210}; return true;
    default: return false;
    }
}

// Bytes of a row of n weights, or -1 when the format is not decoded here or n is
// not a whole number of blocks.
inline long long weight_row_bytes(int fmt, long long n) {
    FormatSpec s;
    if (!weight_format_spec(fmt, &s) || n < 0 || n % s.block) return -1;
    return n / s.block * s.bytes;
}

// ---------------------------------------------------------------- decoders
// deq2<FMT>(row, k): weights k and k+1 (k even) of the row whose first byte is `row`.
// The loads are 2-byte aligned whenever `row` is (every format's block and field
// offsets are even); Q4_K additionally reads its 16-byte header as one 16-byte load,
// which needs a 16-byte aligned row (Q4_K rows are 144-byte multiples).  `row` may point to global or LDS memory.

__device__ __forceinline__ float h2f(uint16_t h) { return f16_bits_to_f32(h); }
__device__ __forceinline__ float2 mul2(float d, int q0, int q1) {
    return make_float2(mul_rn(d, static_cast<float>(q0)), mul_rn(d, static_cast<float>(q1)));
}

// The decoders are split into raw<FMT>(row, k), the loads only, and dec<FMT>(raw, k),
// the arithmetic, so that a kernel can keep many rows of loads in flight before it
// decodes any; deq2 = dec(raw).  raw reads through a row accessor: PtrRow (a plain
// pointer to global or LDS memory) or BufRow (a buffer resource plus a scalar row
// offset, so that a load costs no per-lane address arithmetic).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct PtrRow {
    const uint8_t* p;
    __device__ __forceinline__ uint32_t u8(int o) const { return p[o]; }
    __device__ __forceinline__ uint32_t u16(int o) const { return *reinterpret_cast<const uint16_t*>(p + o); }
    __device__ __forceinline__ uint32_t u32(int o) const { return *reinterpret_cast<const uint32_t*>(p + o); }
    __device__ __forceinline__ u32x4_t u128(int o) const { return *reinterpret_cast<const u32x4_t*>(p + o); }
    __device__ __forceinline__ float2 f2(int o) const { return *reinterpret_cast<const float2*>(p + o); }
};

struct BufRow {
    __amdgpu_buffer_rsrc_t r;
    uint32_t so;  // byte offset of the row inside the buffer (uniform)
    __device__ __forceinline__ uint32_t u8(int o) const { return __builtin_amdgcn_raw_buffer_load_b8(r, o, so, kCacheNt); }
    __device__ __forceinline__ uint32_t u16(int o) const { return __builtin_amdgcn_raw_buffer_load_b16(r, o, so, kCacheNt); }
    __device__ __forceinline__ uint32_t u32(int o) const { return __builtin_amdgcn_raw_buffer_load_b32(r, o, so, kCacheNt); }
    __device__ __forceinline__ u32x4_t u128(int o) const { return __builtin_amdgcn_raw_buffer_load_b128(r, o, so, kCacheNt); }
    __device__ __forceinline__ float2 f2(int o) const {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, o, so, kCacheNt);
        return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
    }
};

template <int FMT> struct Raw;

// ---- F32 / F16 / BF16
template <> struct Raw<QR_FMT_F32> { float2 v; };
template <> struct Raw<QR_FMT_F16> { uint32_t v; };
template <> struct Raw<QR_FMT_BF16> { uint32_t v; };
// ---- Q4_0, BlockDequantizer.cs:52-69: y[i] = d*((b[i]&15)-8), y[i+16] = d*((b[i]>>4)-8),
// 20-byte blocks (f16 d, 16 nibble bytes, 2 pad bytes)
template <> struct Raw<QR_FMT_Q4_0> { uint32_t d, q; };
// ---- Q8_0, BlockDequantizer.cs:71-84: y[i] = d * (sbyte)b[i], 34-byte blocks
template <> struct Raw<QR_FMT_Q8_0> { uint32_t d, q; };
// ---- Q4_K, BlockDequantizer.cs:155-196: y = (d*sc_j) * q - dmin*m_j over 8 sub-blocks of
// 32; 6-bit (sc, m) pairs packed in 12 bytes (sub-blocks 4..7 keep their high bits in the
// top two bits of bytes 0..7); nibbles of sub-blocks 2p and 2p+1 share bytes 32p..32p+31.
template <> struct Raw<QR_FMT_Q4_K> { uint32_t hdr, s0, s1, s2, q; };
// ---- Q6_K, BlockDequantizer.cs:228-256: y = (d*sc) * (q6 - 32); q6 = 4 low bits from ql |
// 2 high bits from qh; weight (half, m, l) of a 256-block uses ql[64 half + l + 32 (m&1)]
// (high nibble for m >= 2), qh[32 half + l] bits 2m..2m+1 and int8 scale 8 half + l/16 + 2m.
template <> struct Raw<QR_FMT_Q6_K> { uint32_t ql, qh, sc, d; };

template <int FMT, class Row> __device__ __forceinline__ Raw<FMT> raw(const Row& row, int k) {
    if constexpr (FMT == QR_FMT_F32) {
        return {row.f2(4 * k)};
    } else if constexpr (FMT == QR_FMT_F16 || FMT == QR_FMT_BF16) {
        return {row.u32(2 * k)};
    } else if constexpr (FMT == QR_FMT_Q4_0) {
        const int blk = (k >> 5) * 20;
        return {row.u16(blk), row.u16(blk + 2 + (k & 15))};
    } else if constexpr (FMT == QR_FMT_Q8_0) {
        const int blk = (k >> 5) * 34;
        return {row.u16(blk), row.u16(blk + 2 + (k & 31))};
    } else if constexpr (FMT == QR_FMT_Q4_K) {
        const int blk = (k >> 8) * 144;  // 144-byte blocks keep the 16-byte header aligned
        const u32x4_t h = row.u128(blk);
        const int sub = (k >> 5) & 7;
        return {h.x, h.y, h.z, h.w, row.u16(blk + 16 + (sub >> 1) * 32 + (k & 31))};
    } else {
        static_assert(FMT == QR_FMT_Q6_K, "format");
        const int blk = (k >> 8) * 210;
        const int w = k & 255, half = w >> 7, m = (w >> 5) & 3, l = w & 31;
        return {row.u16(blk + 64 * half + l + 32 * (m & 1)), row.u16(blk + 128 + 32 * half + l),
                row.u8(blk + 192 + 8 * half + (l >> 4) + 2 * m), row.u16(blk + 208)};
    }
}

template <int FMT> __device__ __forceinline__ float2 dec(const Raw<FMT>& r, int k);

template <> __device__ __forceinline__ float2 dec<QR_FMT_F32>(const Raw<QR_FMT_F32>& r, int) { return r.v; }

template <> __device__ __forceinline__ float2 dec<QR_FMT_F16>(const Raw<QR_FMT_F16>& r, int) {
    return make_float2(h2f(r.v & 0xFFFFu), h2f(r.v >> 16));
}

template <> __device__ __forceinline__ float2 dec<QR_FMT_BF16>(const Raw<QR_FMT_BF16>& r, int) {
    return make_float2(__uint_as_float(r.v << 16), __uint_as_float(r.v & 0xFFFF0000u));
}

template <> __device__ __forceinline__ float2 dec<QR_FMT_Q4_0>(const Raw<QR_FMT_Q4_0>& r, int k) {
    const int sh = (k & 31) >= 16 ? 4 : 0;
    return mul2(h2f(r.d), static_cast<int>((r.q >> sh) & 15u) - 8, static_cast<int>((r.q >> (8 + sh)) & 15u) - 8);
}

template <> __device__ __forceinline__ float2 dec<QR_FMT_Q8_0>(const Raw<QR_FMT_Q8_0>& r, int) {
    return mul2(h2f(r.d), static_cast<int8_t>(r.q & 0xFFu), static_cast<int8_t>((r.q >> 8) & 0xFFu));
}

template <> __device__ __forceinline__ float2 dec<QR_FMT_Q4_K>(const Raw<QR_FMT_Q4_K>& r, int k) {
    const int sub = (k >> 5) & 7;
    auto byte = [&](int j) {
        const uint32_t w = j < 4 ? r.s0 : j < 8 ? r.s1 : r.s2;
        return static_cast<int>((w >> (8 * (j & 3))) & 0xFFu);
    };
    int sc, m;
    if (sub < 4) {
        sc = byte(sub) & 63;
        m = byte(sub + 4) & 63;
    } else {
        sc = (byte(sub + 4) & 0xF) | ((byte(sub - 4) >> 6) << 4);
        m = (byte(sub + 4) >> 4) | ((byte(sub) >> 6) << 4);
    }
    const float a = mul_rn(h2f(r.hdr & 0xFFFFu), static_cast<float>(sc));
    const float mm = mul_rn(h2f(r.hdr >> 16), static_cast<float>(m));
    const int sh = (sub & 1) ? 4 : 0;
    return make_float2(sub_rn(mul_rn(a, static_cast<float>((r.q >> sh) & 15u)), mm),
                       sub_rn(mul_rn(a, static_cast<float>((r.q >> (8 + sh)) & 15u)), mm));
}

template <> __device__ __forceinline__ float2 dec<QR_FMT_Q6_K>(const Raw<QR_FMT_Q6_K>& r, int k) {
    const int m = (k >> 5) & 3;
    const float ds = mul_rn(h2f(r.d), static_cast<float>(static_cast<int8_t>(r.sc & 0xFFu)));
    const int lsh = m >= 2 ? 4 : 0, hsh = 2 * m;
    const int q0 = static_cast<int>(((r.ql >> lsh) & 15u) | (((r.qh >> hsh) & 3u) << 4)) - 32;
    const int q1 = static_cast<int>(((r.ql >> (8 + lsh)) & 15u) | (((r.qh >> (8 + hsh)) & 3u) << 4)) - 32;
    return mul2(ds, q0, q1);
}

template <int FMT>
__device__ __forceinline__ float2 deq2(const uint8_t* row, int k) {
    return dec<FMT>(raw<FMT>(PtrRow{row}, k), k);
}

}  // namespace qr
