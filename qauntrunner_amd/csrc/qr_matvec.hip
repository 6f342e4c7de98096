// qr_matvec.hip -- fused dequant + dot MatVec y = W x over block-quantized rows
// (DotKernels.MatVec / MatVecParallel, DotKernels.cs:599-633), in each format's own
// fp32 operation order (DotRow, DotKernels.cs:24-447) so that every y[r] equals the
// reference's bit for bit:
//   F32/BF16/F16  8 lane sums over k = 8c + L, then 0 + lane0 + ... + lane7
//                 (F16 decodes exponent 31 as a finite 2^16-scale value, as the
//                 reference's vector converter HalfBitsToFloat does, :86-100)
//   Q8_0          per block: lanes over q[L], q[8+L], q[16+L], q[24+L]; HSum; sum += d*dot
//   Q4_0          per block: lanes over lo/hi nibbles; sum += d*dotQ - 8*d*sumX
//   Q4_K          per sub-block: sum += a*(VecDot16 + VecDot16) - mm*SubSum(32)
//   Q6_K          per block: 256 products summed in (half, l, q1..q4) order; sum += d*dot
// Every product and sum is separately rounded (mul_rn / add_rn / sub_rn).
//
// Kernels (every weight byte is read once per input vector):
//   matvec_blk_persistent  Q4_K: x in registers per 64-column item, row tiles double
//                          buffered in registers, block terms per thread, in-order sums last
//   matvec_blk_ring        Q8_0: the same items with row tiles streamed through an LDS ring
//   matvec_fp_wave         F32/F16/BF16: one wave per 8 rows, lane = (row, DotF32 lane),
//                          1 KiB row segments through an LDS ring
//   matvec_kernel          everything else (Q4_0, Q6_K, unaligned rows): LDS tiles of R rows,
//                          block terms in parallel, one thread per row adds them in order
#include <algorithm>

#include "qr_matvec.hpp"
#include "qr_mfma.hpp"

namespace qr {

namespace {

constexpr int kMvThreads = 256;
constexpr int kMvSlabCols = 4096;     // x slab: 16 KiB of LDS
constexpr int kMvTileBytes = 32768;   // weight tile per slab
constexpr int kMvTermsPerRow = 128;   // block terms per row per slab (Q4_K: 16 blocks x 8)
constexpr int kMvMaxRows = 16;
constexpr int kMvStageBatch = 8;
constexpr int kMvXLoads = kMvSlabCols / 4 / kMvThreads;
constexpr int kMvTermStride = kMvTermsPerRow + 1;  // padded: the summing threads read distinct banks
constexpr int kMvPersistMaxCols = 16384;           // persistent form: x of up to 16K values in LDS
constexpr int kMvPersistXLoads = kMvPersistMaxCols / 4 / kMvThreads;

// x sits in LDS in groups of 32 values 36 words apart: every group starts 16-byte aligned
// (float4 reads) and threads reading the same offset of different groups hit different
// banks.  xwords: LDS words for the first n values.
constexpr int kXGroup = 36;
__device__ __forceinline__ int xpad(int k) { return k + 4 * (k >> 5); }
__host__ __device__ constexpr int xwords(int n) { return (n / 32 + 1) * kXGroup; }

// the 32 values of the group at xg (16-byte aligned LDS) into registers
__device__ __forceinline__ void load_group(const float* xg, float (&v)[32]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = reinterpret_cast<const float4*>(xg)[i];
        v[4 * i] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
}

template <int FMT>
struct MvFormat {
    static constexpr bool fp = FMT == QR_FMT_F32 || FMT == QR_FMT_F16 || FMT == QR_FMT_BF16;
    static constexpr int terms = FMT == QR_FMT_Q4_K ? 8 : 1;  // terms per block
};

struct MvLayout {
    int R;            // rows per workgroup
    int slab_cols;
    int stride;       // bytes per staged row (16-byte multiple, padded)
    int copy_bytes;   // 16, 4 or 2
    int persistent;   // one slab, 16-byte copies, one batch per tile: matvec_persistent
    int tstride;      // floats per row of the term buffer (persistent form; a multiple of 4)
    __host__ __device__ size_t lds_bytes() const {
        if (persistent)  // x rounded to whole float4 so that the term rows stay 16-byte aligned
            return static_cast<size_t>(R) * stride + static_cast<size_t>(xwords(slab_cols)) * 4 +
                   static_cast<size_t>(R) * tstride * 4 + static_cast<size_t>(slab_cols / 32) * 4;
        return static_cast<size_t>(R) * stride + static_cast<size_t>(xwords(slab_cols)) * 4 +
               static_cast<size_t>(R) * kMvTermStride * 4 + kMvTermsPerRow * 4;
    }
};

template <int G> struct MvWord;
template <> struct MvWord<16> { typedef u32x4_t type; };
template <> struct MvWord<4> { typedef uint32_t type; };
template <> struct MvWord<2> { typedef uint16_t type; };

__device__ __forceinline__ float hsum8(const float (&v)[8]) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = add_rn(s, v[i]);
    return s;
}

// DotKernels.cs:86-100 (HalfBitsToFloat): exact for finite halves; exponent 31 is
// re-biased like a normal exponent instead of becoming inf/NaN.
__device__ __forceinline__ float f16_dot_decode(uint32_t h) {
    if (((h >> 10) & 0x1Fu) == 0x1Fu) return __uint_as_float(((h & 0x8000u) << 16) | (143u << 23) | ((h & 0x3FFu) << 13));
    return f16_bits_to_f32(static_cast<uint16_t>(h));
}

__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// ---- block terms: the block at p (LDS or global memory), x of the block at xb (padded LDS)

// DotKernels.cs:183-230; xg: the block's x group (LDS)
__device__ __forceinline__ float term_q8_0(const uint8_t* p, const float* xg) {
    float xv[32];
    load_group(xg, xv);
    const float d = f16_bits_to_f32(static_cast<uint16_t>(ld16(p)));
    float acc[8];
#pragma unroll
    for (int L = 0; L < 8; ++L) acc[L] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int L = 0; L < 8; L += 2) {
            const uint32_t v = ld16(p + 2 + 8 * k + L);
            const float q0 = static_cast<float>(static_cast<int8_t>(v & 0xFFu));
            const float q1 = static_cast<float>(static_cast<int8_t>(v >> 8));
            acc[L] = add_rn(acc[L], mul_rn(q0, xv[8 * k + L]));
            acc[L + 1] = add_rn(acc[L + 1], mul_rn(q1, xv[8 * k + L + 1]));
        }
    }
    return mul_rn(d, hsum8(acc));
}

// DotKernels.cs:134-178; sum_x = HSum of the x lanes (precomputed per block)
__device__ __forceinline__ float term_q4_0(const uint8_t* p, const float* xg, float sum_x) {
    float xv[32];
    load_group(xg, xv);
    const float d = f16_bits_to_f32(static_cast<uint16_t>(ld16(p)));
    float acc[8];
#pragma unroll
    for (int L = 0; L < 8; L += 2) {
        const uint32_t b0 = ld16(p + 2 + L), b1 = ld16(p + 2 + 8 + L);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t v0 = (b0 >> (8 * e)) & 0xFFu, v1 = (b1 >> (8 * e)) & 0xFFu;
            float a = 0.0f;
            a = add_rn(a, mul_rn(static_cast<float>(v0 & 15u), xv[L + e]));
            a = add_rn(a, mul_rn(static_cast<float>(v1 & 15u), xv[8 + L + e]));
            a = add_rn(a, mul_rn(static_cast<float>(v0 >> 4), xv[16 + L + e]));
            a = add_rn(a, mul_rn(static_cast<float>(v1 >> 4), xv[24 + L + e]));
            acc[L + e] = a;
        }
    }
    const float dotq = hsum8(acc);
    return sub_rn(mul_rn(d, dotq), mul_rn(mul_rn(8.0f, d), sum_x));
}

// DotKernels.cs:361-373 (VecDot16) over 16 nibbles of bytes q[0..15] (shift 0/4) and the
// 16 values x[0..15] (registers)
__device__ __forceinline__ float vecdot16(const uint32_t (&q)[4], int sh, const float* x) {
    float acc[8];
#pragma unroll
    for (int L = 0; L < 8; ++L) {
        const float q0 = static_cast<float>((q[L >> 2] >> (8 * (L & 3) + sh)) & 15u);
        const float q1 = static_cast<float>((q[2 + (L >> 2)] >> (8 * (L & 3) + sh)) & 15u);
        acc[L] = add_rn(mul_rn(q0, x[L]), mul_rn(q1, x[8 + L]));
    }
    return hsum8(acc);
}

// DotKernels.cs:322-358: terms 2j and 2j+1 of one Q4_K block (the even sub-block over the
// low nibbles of bytes 32j..32j+31, the odd one over their high nibbles); xb: the block's
// first x group (LDS)
__device__ __forceinline__ void terms_q4_k_pair(const uint8_t* p, int j, const float* xb, const float* subsum,
                                                float* out) {
    float xv[2][32];
    load_group(xb + kXGroup * (2 * j), xv[0]);
    load_group(xb + kXGroup * (2 * j + 1), xv[1]);
    const u32x4_t h = *reinterpret_cast<const u32x4_t*>(p);
    const u32x4_t qa = *reinterpret_cast<const u32x4_t*>(p + 16 + 32 * j);
    const u32x4_t qb = *reinterpret_cast<const u32x4_t*>(p + 32 + 32 * j);
    const float d = f16_bits_to_f32(static_cast<uint16_t>(h.x & 0xFFFFu));
    const float dmin = f16_bits_to_f32(static_cast<uint16_t>(h.x >> 16));
    auto byte = [&](int i) {
        const uint32_t w = i < 4 ? h.y : i < 8 ? h.z : h.w;
        return static_cast<int>((w >> (8 * (i & 3))) & 0xFFu);
    };
    const uint32_t lo[4] = {qa.x, qa.y, qa.z, qa.w};
    const uint32_t hi[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int odd = 0; odd < 2; ++odd) {
        const int sub = 2 * j + odd;
        int sc, m;
        if (sub < 4) {
            sc = byte(sub) & 63;
            m = byte(sub + 4) & 63;
        } else {
            sc = (byte(sub + 4) & 0xF) | ((byte(sub - 4) >> 6) << 4);
            m = (byte(sub + 4) >> 4) | ((byte(sub) >> 6) << 4);
        }
        const float a = mul_rn(d, static_cast<float>(sc)), mm = mul_rn(dmin, static_cast<float>(m));
        const float v = add_rn(vecdot16(lo, 4 * odd, xv[odd]), vecdot16(hi, 4 * odd, xv[odd] + 16));
        out[odd] = sub_rn(mul_rn(a, v), mul_rn(mm, subsum[sub]));
    }
}

// all 8 terms of a Q4_K block, sub-blocks in order
__device__ __forceinline__ void terms_q4_k(const uint8_t* p, const float* xb, const float* subsum, float* out) {
#pragma unroll
    for (int j = 0; j < 4; ++j) terms_q4_k_pair(p, j, xb, subsum, out + 2 * j);
}

// DotKernels.cs:420-447; xb: the block's first x group (LDS).  Half n, lane-sum step l
// uses x[128n + 32m + l] for m = 0..3, i.e. offset l of groups 4n+m.
__device__ __forceinline__ float term_q6_k(const uint8_t* p, const float* xb) {
    const float d = f16_bits_to_f32(static_cast<uint16_t>(ld16(p + 208)));
    float dot = 0.0f;
    for (int n = 0; n < 2; ++n) {
        int sc[8];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const uint32_t v = ld16(p + 192 + 8 * n + i);
            sc[i] = static_cast<int8_t>(v & 0xFFu);
            sc[i + 1] = static_cast<int8_t>(v >> 8);
        }
        const uint8_t* ql = p + 64 * n;
        const uint8_t* qh = p + 128 + 32 * n;
        for (int l0 = 0; l0 < 32; l0 += 8) {
            float xv[4][8];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float4* g = reinterpret_cast<const float4*>(xb + kXGroup * (4 * n + m) + l0);
                const float4 f0 = g[0], f1 = g[1];
                xv[m][0] = f0.x; xv[m][1] = f0.y; xv[m][2] = f0.z; xv[m][3] = f0.w;
                xv[m][4] = f1.x; xv[m][5] = f1.y; xv[m][6] = f1.z; xv[m][7] = f1.w;
            }
#pragma unroll
            for (int l = 0; l < 8; l += 2) {
                const int ll = l0 + l;
                const uint32_t la = ld16(ql + ll), lb = ld16(ql + 32 + ll), hh = ld16(qh + ll);
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int is = (ll + e) >> 4;
                    const uint32_t a = (la >> (8 * e)) & 0xFFu, b = (lb >> (8 * e)) & 0xFFu, hb = (hh >> (8 * e)) & 0xFFu;
                    const int q1 = static_cast<int>((a & 15u) | (((hb >> 0) & 3u) << 4));
                    const int q2 = static_cast<int>((b & 15u) | (((hb >> 2) & 3u) << 4));
                    const int q3 = static_cast<int>((a >> 4) | (((hb >> 4) & 3u) << 4));
                    const int q4 = static_cast<int>((b >> 4) | (((hb >> 6) & 3u) << 4));
                    dot = add_rn(dot, mul_rn(static_cast<float>(sc[is + 0] * (q1 - 32)), xv[0][l + e]));
                    dot = add_rn(dot, mul_rn(static_cast<float>(sc[is + 2] * (q2 - 32)), xv[1][l + e]));
                    dot = add_rn(dot, mul_rn(static_cast<float>(sc[is + 4] * (q3 - 32)), xv[2][l + e]));
                    dot = add_rn(dot, mul_rn(static_cast<float>(sc[is + 6] * (q4 - 32)), xv[3][l + e]));
                }
            }
        }
    }
    return mul_rn(d, dot);
}

// ---- Q4_K, one thread per (row, sub-block pair): DotKernels.cs:322-373 with x in registers.
// Pair pc = 4*block + j covers x[64*pc .. 64*pc+63]: sub-block 2j over the low nibbles of
// quant bytes 32j..32j+31, sub-block 2j+1 over their high nibbles.

// w & 0x0F0F0F0F, opaque to the optimiser: it would otherwise fold the mask into one
// bit-field extract per nibble, where a byte-to-float conversion of the masked word
// (v_cvt_f32_ubyte0..3) takes one instruction per nibble.
__device__ __forceinline__ uint32_t nibble_mask(uint32_t w) {
    uint32_t m;
    asm("v_and_b32 %0, %1, %2" : "=v"(m) : "s"(0x0F0F0F0Fu), "v"(w));
    return m;
}

// VecDot16 (DotKernels.cs:361-373) over 16 nibbles already masked into bytes: q holds bytes
// 0..15 (the value of nibble L is byte L of q), x the 16 values
__device__ __forceinline__ float vecdot16_bytes(const uint32_t (&q)[4], const float* x) {
    float acc[8];
#pragma unroll
    for (int L = 0; L < 8; ++L) {
        const float q0 = static_cast<float>((q[L >> 2] >> (8 * (L & 3))) & 0xFFu);
        const float q1 = static_cast<float>((q[2 + (L >> 2)] >> (8 * (L & 3))) & 0xFFu);
        acc[L] = add_rn(mul_rn(q0, x[L]), mul_rn(q1, x[8 + L]));
    }
    return hsum8(acc);
}

// the two terms of pair j of the block whose header is h, quants qa (bytes 32j..32j+15)
// and qb (32j+16..32j+31), against x[0..63] and the two sub-block sums of x
// The 6-bit scale and min of sub-block 2j+odd from the 12 scale bytes s[0..11] (h.y, h.z,
// h.w) without a branch on j: with c = 16 (j & 1) + 8 odd, sub-blocks 0..3 (j < 2) take
// sc = s[j2] & 63 = bits c..c+5 of h.y and m = bits c..c+5 of h.z; sub-blocks 4..7 take
// sc = (s[8+j2] & 15) | (s[j2] >> 6) << 4 and m = (s[8+j2] >> 4) | (s[4+j2] >> 6) << 4,
// i.e. bit fields c..c+3 / c+4..c+7 of h.w and c+6..c+7 of h.y / h.z (j2 = 2 (j & 1) + odd).
__device__ __forceinline__ void q4k_scale_min(const u32x4_t h, int j, int odd, int& sc, int& m) {
    const uint32_t c = 16u * static_cast<uint32_t>(j & 1) + 8u * static_cast<uint32_t>(odd);
    const uint32_t lo_sc = __builtin_amdgcn_ubfe(h.y, c, 6), lo_m = __builtin_amdgcn_ubfe(h.z, c, 6);
    const uint32_t hi_sc = __builtin_amdgcn_ubfe(h.w, c, 4) | (__builtin_amdgcn_ubfe(h.y, c + 6, 2) << 4);
    const uint32_t hi_m = __builtin_amdgcn_ubfe(h.w, c + 4, 4) | (__builtin_amdgcn_ubfe(h.z, c + 6, 2) << 4);
    sc = static_cast<int>(j >= 2 ? hi_sc : lo_sc);
    m = static_cast<int>(j >= 2 ? hi_m : lo_m);
}

__device__ __forceinline__ void q4k_pair_terms(const u32x4_t h, const u32x4_t qa, const u32x4_t qb, int j,
                                               const float (&x)[64], float ss0, float ss1, float& t0, float& t1) {
    const float d = f16_bits_to_f32(static_cast<uint16_t>(h.x & 0xFFFFu));
    const float dmin = f16_bits_to_f32(static_cast<uint16_t>(h.x >> 16));
    const uint32_t a[4] = {qa.x, qa.y, qa.z, qa.w};
    const uint32_t b[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int odd = 0; odd < 2; ++odd) {
        int sc, m;
        q4k_scale_min(h, j, odd, sc, m);
        uint32_t na[4], nb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            na[i] = nibble_mask(odd ? a[i] >> 4 : a[i]);
            nb[i] = nibble_mask(odd ? b[i] >> 4 : b[i]);
        }
        const float as = mul_rn(d, static_cast<float>(sc)), mm = mul_rn(dmin, static_cast<float>(m));
        const float v = add_rn(vecdot16_bytes(na, x + 32 * odd), vecdot16_bytes(nb, x + 32 * odd + 16));
        const float t = sub_rn(mul_rn(as, v), mul_rn(mm, odd ? ss1 : ss0));
        if (odd) t1 = t;
        else t0 = t;
    }
}

// Persistent form of the block formats: workgroup w takes row tiles w, w + G, w + 2G, ...
// (G = the workgroups of its matrix, R rows a tile).  Thread (row group g, item column pc) owns one item of every
// row (Q4_K: a sub-block pair, 64 columns, two terms; Q8_0: a block pair, 64 columns, two
// terms): its x values stay in registers for all tiles, the next tile's weights are loaded
// while the current tile is computed (two register buffers, the loop unrolled by two so that
// each half waits only for its own loads), every tile's terms stay in LDS, and the in-order
// sums of all the workgroup's rows run at the end.  blockDim = rg * tpg threads.
// x row pitch in LDS: 64 values and 4 floats of padding
constexpr int kXRow = 68;

// In-order sum (left to right, from +0) of a row's nt terms (nt even, 16-byte aligned) in
// LDS.  Groups of 32 terms: the loads of the next group are issued before the adds of the
// current one (clamped to the row, so every iteration issues the same loads), so the chain
// of dependent adds waits for LDS once per row instead of once per group.
__device__ __forceinline__ float ordered_row_sum(const float* tr, int nt) {
    const float4* t4 = reinterpret_cast<const float4*>(tr);
    const int n4 = nt >> 2;
    const int last = max(n4 - 1, 0);
    float sum = 0.0f;
    auto add4 = [&](const float4 v) { sum = add_rn(add_rn(add_rn(add_rn(sum, v.x), v.y), v.z), v.w); };
    auto load8 = [&](float4 (&v)[8], int g0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = t4[min(g0 + j, last)];
    };
    float4 a[8], b[8];
    int g = 0;
    load8(a, 0);
    for (;;) {
        if (g + 8 > n4) break;
        load8(b, g + 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) add4(a[j]);
        g += 8;
        if (g + 8 > n4) break;
        load8(a, g + 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) add4(b[j]);
        g += 8;
    }
    for (; g < n4; ++g) add4(t4[g]);  // the last n4 % 8 groups
    if (nt & 2) sum = add_rn(add_rn(sum, tr[nt - 2]), tr[nt - 1]);
    return sum;
}

struct MvBlkP {
    int P, tpg, rg, R, tstride;
    int ntiles;   // ceil(rows / R)
};

// Matrices of one launch of the block kernels: workgroups start[m] .. start[m + 1] - 1 take
// matrix m (its own tiles, strided by its workgroup count), every matrix sharing the
// format, cols and x (a single MatVec is a group of one).
struct BlkGroup {
    int n;
    int start[kMatVecGroupMax + 1];
    int ntiles[kMatVecGroupMax];
    const uint8_t* w[kMatVecGroupMax];
    long long rows[kMatVecGroupMax];
    float* y[kMatVecGroupMax];
};

__device__ __forceinline__ int group_member(int n, const int (&start)[kMatVecGroupMax + 1]) {
    int m = 0;
#pragma unroll
    for (int i = 1; i < kMatVecGroupMax; ++i)
        if (i < n && static_cast<int>(blockIdx.x) >= start[i]) m = i;
    return m;
}

// Q4_K (DotKernels.cs:322-373): item pc = 4*block + j; loads: the block header and the two
// 16-byte quant vectors of pair j.
struct PolQ4K {
    static constexpr int kLoads = 3;
    static constexpr int kWords = 4;  // dwords per load
    struct Lane {
        int j;
        float ss0, ss1;
        float xv[64];
    };
    __device__ static void offsets(int pc, uint32_t (&o)[kLoads]) {
        const uint32_t b = static_cast<uint32_t>((pc >> 2) * 144);
        o[0] = b;
        o[1] = b + 16 + 32 * (pc & 3);
        o[2] = o[1] + 16;
    }
    __device__ static void prep(Lane& l, const float* xi, int pc) {  // xi: the item's 64 values
        l.j = pc & 3;
        const float4* x4 = reinterpret_cast<const float4*>(xi);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 f = x4[i];
            l.xv[4 * i] = f.x;
            l.xv[4 * i + 1] = f.y;
            l.xv[4 * i + 2] = f.z;
            l.xv[4 * i + 3] = f.w;
        }
        l.ss0 = 0.0f;  // SubSum over the 32 values of each sub-block, in order
        l.ss1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) l.ss0 = add_rn(l.ss0, l.xv[i]);
#pragma unroll
        for (int i = 32; i < 64; ++i) l.ss1 = add_rn(l.ss1, l.xv[i]);
    }
    __device__ static void terms(const Lane& l, const u32x4_t (&v)[kLoads], float& t0, float& t1) {
        q4k_pair_terms(v[0], v[1], v[2], l.j, l.xv, l.ss0, l.ss1, t0, t1);
    }
};

// Q8_0 (DotKernels.cs:183-230): item pc = block pair (blocks 2pc, 2pc+1: 68 bytes, 4-byte
// aligned when the row is); loads: the 17 dwords of the pair.  Per block: lane L sums
// q[L]x[L], q[8+L]x[8+L], q[16+L]x[16+L], q[24+L]x[24+L] in order, HSum, times d.
struct PolQ8 {
    static constexpr int kLoads = 17;
    static constexpr int kWords = 1;
    struct Lane {
        float xv[64];
    };
    __device__ static void offsets(int pc, uint32_t (&o)[kLoads]) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) o[i] = static_cast<uint32_t>(68 * pc + 4 * i);
    }
    __device__ static void prep(Lane& l, const float* xi, int) {  // xi: the item's 64 values
        const float4* x4 = reinterpret_cast<const float4*>(xi);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float4 f = x4[i];
            l.xv[4 * i] = f.x;
            l.xv[4 * i + 1] = f.y;
            l.xv[4 * i + 2] = f.z;
            l.xv[4 * i + 3] = f.w;
        }
    }
    // byte k of the pair
    __device__ static int sbyte(const uint32_t (&w)[kLoads], int k) {
        return static_cast<int8_t>((w[k >> 2] >> (8 * (k & 3))) & 0xFFu);
    }
    __device__ static float block(const uint32_t (&w)[kLoads], int b0, const float* x) {
        const uint32_t hb = (w[b0 >> 2] >> (8 * (b0 & 3))) & 0xFFFFu;  // b0 even: one dword
        const float d = f16_bits_to_f32(static_cast<uint16_t>(hb));
        float acc[8];
#pragma unroll
        for (int L = 0; L < 8; ++L) {
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                a = add_rn(a, mul_rn(static_cast<float>(sbyte(w, b0 + 2 + 8 * k + L)), x[8 * k + L]));
            acc[L] = a;
        }
        return mul_rn(d, hsum8(acc));
    }
    __device__ static void terms(const Lane& l, const uint32_t (&v)[kLoads], float& t0, float& t1) {
        t0 = block(v, 0, l.xv);
        t1 = block(v, 34, l.xv + 32);
    }
};

template <class Pol> struct PolLoad { typedef u32x4_t type; };
template <> struct PolLoad<PolQ8> { typedef uint32_t type; };

// Loads of one tile through a buffer resource made for it (uniform base and size), so that a
// tile costs scalar arithmetic only: the lane offsets (per row) are fixed for the whole kernel.
// Rows past the end of the matrix lie outside the resource and read as zero; their terms are
// never summed.
template <class Pol, int RPT>
__device__ __forceinline__ void blk_load(const MatVecArgs& a, const MvBlkP& k, int tile,
                                         const uint32_t (&off)[RPT][Pol::kLoads],
                                         typename PolLoad<Pol>::type (&v)[RPT][Pol::kLoads]) {
    // 32-bit uniform arithmetic (rows < 2^31 and R * row_bytes < 2^31 are checked on the host):
    // a 64-bit compare would be done in vector registers
    const int r0 = tile * k.R;
    const int nrec = min(k.R, static_cast<int>(a.rows) - r0) * static_cast<int>(a.row_bytes);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(a.w + static_cast<long long>(r0) * a.row_bytes), static_cast<short>(0), nrec,
        kBufferFlags);
    // default cache policy: these per-item loads measured slower as non-temporal (Q4_K layer
    // 48.3 -> 51.3 us), unlike the whole-line DMA of the ring and single-wave forms
#pragma unroll
    for (int r = 0; r < RPT; ++r)
#pragma unroll
        for (int i = 0; i < Pol::kLoads; ++i) {
            if constexpr (Pol::kWords == 4) v[r][i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[r][i], 0, 0);
            else v[r][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, off[r][i], 0, 0);
        }
}

template <class Pol, int RPT>
__global__ __launch_bounds__(512) void matvec_blk_persistent(MatVecArgs a, MvBlkP k, BlkGroup gr) {
    typedef typename PolLoad<Pol>::type V;
    extern __shared__ __align__(16) uint8_t mv_lds[];
    float* terms = reinterpret_cast<float*>(mv_lds);
    const int mg = group_member(gr.n, gr.start);  // this workgroup's matrix (uniform)
    a.w = gr.w[mg];
    a.rows = gr.rows[mg];
    a.y = gr.y[mg];
    k.ntiles = gr.ntiles[mg];
    const int bx = static_cast<int>(blockIdx.x) - gr.start[mg];
    const int t = threadIdx.x;
    const int g = t / k.tpg;
    const bool active = t - g * k.tpg < k.P;
    // lanes past the row's items load and compute item P-1 and store nothing: no branch
    // around the loads, so the wait counts stay exact
    const int pc = min(t - g * k.tpg, k.P - 1);
    const int G = gr.start[mg + 1] - gr.start[mg];
    const int q = blockIdx.y;
    const float* x = a.x + static_cast<long long>(q) * a.cols;
    const int last = k.ntiles - 1;

    uint32_t off[RPT][Pol::kLoads];
    {
        uint32_t o[Pol::kLoads];
        Pol::offsets(pc, o);
#pragma unroll
        for (int r = 0; r < RPT; ++r)
#pragma unroll
            for (int i = 0; i < Pol::kLoads; ++i) off[r][i] = static_cast<uint32_t>((g * RPT + r) * a.row_bytes) + o[i];
    }
    V vA[RPT][Pol::kLoads], vB[RPT][Pol::kLoads];
    int it = bx;
    blk_load<Pol, RPT>(a, k, it, off, vA);
    // x reaches the threads through LDS: one coalesced copy per workgroup (every thread of
    // every workgroup reading its 64 values from global memory made all CUs hit the same
    // lines of L2 at once), 64-value rows padded by 4 floats so that the rows the lanes read
    // start on distinct banks.  The area is the terms' area, written only after the barrier.
    float* xl = reinterpret_cast<float*>(mv_lds);
    for (int i = 4 * t; i < a.cols; i += 4 * static_cast<int>(blockDim.x))
        *reinterpret_cast<float4*>(xl + i + 4 * (i >> 6)) = *reinterpret_cast<const float4*>(x + i);
    __syncthreads();
    typename Pol::Lane lane;
    Pol::prep(lane, xl + kXRow * pc, pc);
    __syncthreads();
    auto compute = [&](const V (&v)[RPT][Pol::kLoads], int slot) {
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            float t0, t1;
            Pol::terms(lane, v[r], t0, t1);
            if (active)
                *reinterpret_cast<float2*>(terms + ((slot * k.R) + g * RPT + r) * k.tstride + 2 * pc) =
                    make_float2(t0, t1);
        }
    };
    int slot = 0;
    for (;;) {  // exits only through the breaks: the back-edge is the steady state
        const int n1 = it + G;
        blk_load<Pol, RPT>(a, k, min(n1, last), off, vB);
        compute(vA, slot++);
        if (n1 > last) break;
        it = n1;
        const int n2 = it + G;
        blk_load<Pol, RPT>(a, k, min(n2, last), off, vA);
        compute(vB, slot++);
        if (n2 > last) break;
        it = n2;
    }
    __syncthreads();
    // in-order sums: thread t takes row t % R of the workgroup's tile t / R
    const int nt = 2 * k.P;
    for (int i = t; i < slot * k.R; i += blockDim.x) {
        const int s = i / k.R, r = i - s * k.R;
        const long long row = static_cast<long long>(bx + s * G) * k.R + r;
        if (row >= a.rows) continue;
        a.y[static_cast<long long>(q) * a.rows + row] = ordered_row_sum(terms + i * k.tstride, nt);
    }
}

// Ring form of the block formats: the same items and in-order sums as matvec_blk_persistent,
// but row tiles stream into an LDS ring of kRingSlots slots by direct-to-LDS buffer loads
// (kRingSlots - 1 tiles in flight, explicit vmcnt waits), so the prefetch depth costs no
// registers.  A tile is R rows (R * row_bytes <= 4 KiB * U); wave w loads its 1 KiB units
// w, w + 4, ... of it.  Per tile: wait for this wave's units, barrier (every wave's units have
// landed and the slot refilled next has been read), refill, compute the tile's terms from LDS.
// Two slots: one tile in flight while one is read, and more workgroups per CU (measured
// per 8B layer of Q8_0 MatVecs: 82.9 us, against 87.4-88.8 with three slots; deeper rings
// slower still)
constexpr int kRingSlots = 2;

struct MvRing {
    int P, tpg, rg, R, tstride;
    int ntiles;
    int slot_bytes;  // 4096 * U
};

template <class Pol, int RPT>
__device__ __forceinline__ void ring_read(const char* tile, int row_bytes, int g, int pc,
                                          typename PolLoad<Pol>::type (&v)[RPT][Pol::kLoads]) {
    uint32_t o[Pol::kLoads];
    Pol::offsets(pc, o);
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const char* rowp = tile + (g * RPT + r) * row_bytes;
#pragma unroll
        for (int i = 0; i < Pol::kLoads; ++i) {
            if constexpr (Pol::kWords == 4) v[r][i] = *reinterpret_cast<const u32x4_t*>(rowp + o[i]);
            else v[r][i] = *reinterpret_cast<const uint32_t*>(rowp + o[i]);
        }
    }
}

template <class Pol, int RPT, int U>
__global__ __launch_bounds__(256) void matvec_blk_ring(MatVecArgs a, MvRing k, BlkGroup gr) {
    typedef typename PolLoad<Pol>::type V;
    extern __shared__ __align__(1024) char ring_lds[];
    float* terms = reinterpret_cast<float*>(ring_lds + kRingSlots * k.slot_bytes);
    const int mg = group_member(gr.n, gr.start);  // this workgroup's matrix (uniform)
    a.w = gr.w[mg];
    a.rows = gr.rows[mg];
    a.y = gr.y[mg];
    k.ntiles = gr.ntiles[mg];
    const int bx = static_cast<int>(blockIdx.x) - gr.start[mg];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // four waves
    const int g = t / k.tpg;
    const bool active = t - g * k.tpg < k.P;
    const int pc = min(t - g * k.tpg, k.P - 1);
    const int G = gr.start[mg + 1] - gr.start[mg];
    const int q = blockIdx.y;
    const float* x = a.x + static_cast<long long>(q) * a.cols;
    const int cnt = (k.ntiles - bx + G - 1) / G;  // tiles of this workgroup, >= 1

    // DMA of the workgroup's tile s (clamped to its last one, so every round issues U units
    // per wave) into ring slot s % kRingSlots; rows past the matrix read as zero
    auto dma = [&](int s) {
        s = min(s, cnt - 1);
        const int r0 = (bx + s * G) * k.R;
        const int nrec = min(k.R, static_cast<int>(a.rows) - r0) * static_cast<int>(a.row_bytes);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(a.w + static_cast<long long>(r0) * a.row_bytes), static_cast<short>(0), nrec,
            kBufferFlags);
        char* slot = ring_lds + (s % kRingSlots) * k.slot_bytes;
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int u = wave + 4 * i;
            // weights are read once per call: non-temporal (Q8_0 layer 68.3 -> 64.9 us)
            buffer_load_lds16<kCacheNt>(rs, slot + 1024 * u, static_cast<uint32_t>(16 * lane), static_cast<uint32_t>(1024 * u));
        }
    };
    // x first, awaited before any DMA is in flight: the compiler counts its loads but not the
    // DMAs, and a wait for x inside the loop would also wait for every tile in flight
    typename Pol::Lane pl;
    Pol::prep(pl, x + 64 * pc, pc);
    wait_vmcnt<0>();
#pragma unroll
    for (int s = 0; s < kRingSlots - 1; ++s) dma(s);
    for (int s = 0; s < cnt; ++s) {
        wait_vmcnt<(kRingSlots - 2) * U>();  // this wave's units of tile s have landed
        lds_barrier();                       // everyone's have; slot (s - 1) % kRingSlots is free
        dma(s + kRingSlots - 1);
        V v[RPT][Pol::kLoads];
        ring_read<Pol, RPT>(ring_lds + (s % kRingSlots) * k.slot_bytes, static_cast<int>(a.row_bytes), g, pc, v);
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            float t0, t1;
            Pol::terms(pl, v[r], t0, t1);
            if (active)
                *reinterpret_cast<float2*>(terms + ((s * k.R) + g * RPT + r) * k.tstride + 2 * pc) = make_float2(t0, t1);
        }
    }
    wait_dma();
    __syncthreads();
    const int nt = 2 * k.P;
    for (int i = t; i < cnt * k.R; i += blockDim.x) {
        const int s = i / k.R, r = i - s * k.R;
        const long long row = static_cast<long long>(bx + s * G) * k.R + r;
        if (row >= a.rows) continue;
        a.y[static_cast<long long>(q) * a.rows + row] = ordered_row_sum(terms + i * k.tstride, nt);
    }
}

// ---- F32 / F16 / BF16 (DotF32 order, DotKernels.cs:52-100).  Row r's lane L accumulates
// k = 8c + L over the chunks c in order, so every row is 8 serial chains.  A workgroup is one
// wave and R <= 8 rows, lane 8r + L the chain (row r, lane L).  The wave streams its rows in segments of 1 KiB per row through a
// ring of kFwSlots LDS slots filled by direct-to-LDS buffer loads (kFwSlots - 1 segments in
// flight; completion awaited with explicit vmcnt waits), and each lane walks its chain over
// the chunks of a segment: weight, x, product, add.  No barrier, no register prefetch.
// Two slots (one segment in flight while one is read): 20.6 KiB of LDS per one-wave
// workgroup, so 7 fit per CU and the 14336-row matrices of the 8B shape (1,792 workgroups)
// run in one round.  Measured per 8B layer of F16 MatVecs: 113.0 us, against 116.6-118.3
// with three slots and 125.9-127.0 with four.
constexpr int kFwSlots = 2;
constexpr int kFwRowPad = 1024 + 16;  // LDS bytes per row segment: rows land on distinct banks

template <int FMT, int R>
struct FwGeom {
    static constexpr int B = FMT == QR_FMT_F32 ? 32 : 16;     // bytes per chunk of 8 weights
    static constexpr int SEG = 1024 / B;                       // chunks per segment
    static constexpr int XBYTES = SEG * 32;                    // x bytes per segment
    static constexpr int XDMA = XBYTES / 1024;                 // DMAs of x per segment
    static constexpr int SLOT = R * kFwRowPad + XBYTES;        // bytes per slot
    static constexpr int DMAS = R + XDMA;                      // DMAs per segment
};

// The product of the weight at p (LDS) and x.  F16: fma(w, x, +0) in one v_fma_mix_f32 (the
// half converted exactly inside); it equals the rounded product w*x except that a -0 product
// becomes +0, which no chain can tell apart: a lane sum starts at +0 and never becomes -0
// (x + y is -0 only for two -0 operands), and for any other value v + (-0) = v + (+0).
template <int FMT>
__device__ __forceinline__ float fw_product(const char* p, float x) {
    if constexpr (FMT == QR_FMT_F32) return mul_rn(*reinterpret_cast<const float*>(p), x);
    else if constexpr (FMT == QR_FMT_BF16)
        return mul_rn(__uint_as_float(static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(p)) << 16), x);
    else return __builtin_fmaf(static_cast<float>(*reinterpret_cast<const _Float16*>(p)), x, 0.0f);
}

// Matrices of one launch: workgroups start[m] .. start[m + 1] - 1 take matrix m (a single
// MatVec is a group of one).  Every matrix shares the format, cols, row bytes and x.
struct FwGroup {
    int n;
    int start[kMatVecGroupMax + 1];
    const uint8_t* w[kMatVecGroupMax];
    long long rows[kMatVecGroupMax];
    float* y[kMatVecGroupMax];
};

template <int FMT, int R>
__global__ __launch_bounds__(64) void matvec_fp_wave(MatVecArgs a, FwGroup gr) {
    using Gm = FwGeom<FMT, R>;
    __shared__ __align__(16) char ring[kFwSlots][Gm::SLOT];
    const int lane = threadIdx.x;
    const int rr = lane >> 3, L = lane & 7;
    int mg = 0;  // this workgroup's matrix (uniform)
#pragma unroll
    for (int i = 1; i < kMatVecGroupMax; ++i)
        if (i < gr.n && static_cast<int>(blockIdx.x) >= gr.start[i]) mg = i;
    a.w = gr.w[mg];
    a.rows = gr.rows[mg];
    a.y = gr.y[mg];
    const long long r0 = static_cast<long long>(static_cast<int>(blockIdx.x) - gr.start[mg]) * R;
    const int q = blockIdx.y;
    const float* x = a.x + static_cast<long long>(q) * a.cols;
    const int nch = a.cols / 8;
    const int nseg = (nch + Gm::SEG - 1) / Gm::SEG;
    const int rbytes = nch * Gm::B;

    __amdgpu_buffer_rsrc_t rs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {  // rows past the matrix: an empty resource, read as zeros
        const bool in = r0 + r < a.rows;
        rs[r] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w + (in ? (r0 + r) * a.row_bytes : 0)),
                                                  static_cast<short>(0), in ? rbytes : 0, kBufferFlags);
    }
    const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), static_cast<short>(0),
                                                                        nch * 32, kBufferFlags);
    // segment s into slot s % kFwSlots; past the last segment the last one is read again, so
    // that every round issues the same number of DMAs
    auto issue = [&](int s) {
        s = min(s, nseg - 1);
        char* slot = ring[s % kFwSlots];
#pragma unroll
        for (int r = 0; r < R; ++r)
            // weights are read once per call: non-temporal (F16 layer 97.0 -> 93.8 us)
            buffer_load_lds16<kCacheNt>(rs[r], slot + r * kFwRowPad, static_cast<uint32_t>(16 * lane),
                                        static_cast<uint32_t>(s * 1024));
#pragma unroll
        for (int i = 0; i < Gm::XDMA; ++i)
            buffer_load_lds16(rsx, slot + R * kFwRowPad + 1024 * i, static_cast<uint32_t>(16 * lane),
                              static_cast<uint32_t>(s * Gm::XBYTES + 1024 * i));
    };

    float acc = 0.0f;
    const int wofs = rr * kFwRowPad + (FMT == QR_FMT_F32 ? 4 : 2) * L;
    const int xofs = R * kFwRowPad + 4 * L;
#pragma unroll
    for (int s = 0; s < kFwSlots - 1; ++s) issue(s);
    for (int s = 0; s < nseg; ++s) {
        // the slot refilled now was consumed in the previous round (this wave's own reads)
        issue(s + kFwSlots - 1);
        wait_vmcnt<(kFwSlots - 1) * Gm::DMAS>();  // segment s has landed
        asm volatile("" ::: "memory");
        const char* slot = ring[s % kFwSlots];
        const int n = min(Gm::SEG, nch - s * Gm::SEG);
        if (n == Gm::SEG) {
#pragma unroll 16
            for (int c = 0; c < Gm::SEG; ++c)
                acc = add_rn(acc, fw_product<FMT>(slot + wofs + c * Gm::B,
                                                  *reinterpret_cast<const float*>(slot + xofs + c * 32)));
        } else {
            for (int c = 0; c < n; ++c)
                acc = add_rn(acc, fw_product<FMT>(slot + wofs + c * Gm::B,
                                                  *reinterpret_cast<const float*>(slot + xofs + c * 32)));
        }
        asm volatile("" ::: "memory");  // this slot's reads stay before its refill
    }
    wait_dma();
    // HSum in lane order over the row's 8 lanes
    const int base = lane & ~7;
    float sum = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) sum = add_rn(sum, __shfl(acc, base + l, 64));
    const long long row = r0 + rr;
    if constexpr (FMT == QR_FMT_F16) {
        if (!isfinite(sum) && rr < R && row < a.rows) {
            // exact decode of the row's lane chain (HalfBitsToFloat, DotKernels.cs:86-100)
            const uint8_t* w = a.w + row * a.row_bytes;
            float e = 0.0f;
            for (int c = 0; c < nch; ++c) {
                const int k = 8 * c + L;
                e = add_rn(e, mul_rn(f16_dot_decode(*reinterpret_cast<const uint16_t*>(w + 2 * k)), x[k]));
            }
            sum = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; ++l) sum = add_rn(sum, __shfl(e, base + l, 64));
        }
    }
    if (L == 0 && rr < R && row < a.rows) a.y[static_cast<long long>(q) * a.rows + row] = sum;
}

// fp weight k of a staged row
template <int FMT>
__device__ __forceinline__ float fp_weight(const uint8_t* row, int k) {
    if constexpr (FMT == QR_FMT_F32) return *reinterpret_cast<const float*>(row + 4 * k);
    else if constexpr (FMT == QR_FMT_BF16) return __uint_as_float(ld16(row + 2 * k) << 16);
    else return f16_dot_decode(ld16(row + 2 * k));
}

// Copies bytes [0, bytes) of nrows rows (row r at src + r*row_bytes) into LDS rows of
// `stride` bytes: one batch of loads per thread is issued before its stores (indices
// past the end clamped to a valid address, not stored).
template <int G>
__device__ __forceinline__ void mv_stage(const uint8_t* src, long long row_bytes, int bytes, int nrows,
                                         uint8_t* lds, int stride, const float* xsrc, float* xlds, int xcols) {
    typedef typename MvWord<G>::type V;
    const int per_row = bytes / G;
    const int total = per_row * nrows;
    const int nx = xcols / 4;  // float4 of x
    for (int base = 0; base < total || base == 0; base += kMvThreads * kMvStageBatch) {
        V v[kMvStageBatch];
        int dst[kMvStageBatch];
#pragma unroll
        for (int s = 0; s < kMvStageBatch; ++s) {
            const int idx = base + threadIdx.x + s * kMvThreads;
            const int i = min(idx, total - 1);
            const int r = i / per_row, e = i - r * per_row;
            v[s] = *reinterpret_cast<const V*>(src + r * row_bytes + e * G);
            dst[s] = idx < total ? r * stride + e * G : -1;
        }
        if (base == 0) {  // the x slab: at most kMvSlabCols / 4 float4, issued with the first batch
            float4 xv[kMvXLoads];
#pragma unroll
            for (int s = 0; s < kMvXLoads; ++s)
                xv[s] = reinterpret_cast<const float4*>(xsrc)[min(static_cast<int>(threadIdx.x) + s * kMvThreads, nx - 1)];
#pragma unroll
            for (int s = 0; s < kMvXLoads; ++s) {
                const int i = static_cast<int>(threadIdx.x) + s * kMvThreads;
                if (i < nx) {
                    float* d = xlds + xpad(4 * i);
                    d[0] = xv[s].x;
                    d[1] = xv[s].y;
                    d[2] = xv[s].z;
                    d[3] = xv[s].w;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < kMvStageBatch; ++s)
            if (dst[s] >= 0) *reinterpret_cast<V*>(lds + dst[s]) = v[s];
        if (total <= kMvThreads * kMvStageBatch) break;
    }
}

template <int FMT, int G>
__device__ __forceinline__ void matvec_body(const MatVecArgs& a, const MvLayout& L, uint8_t* lds) {
    constexpr bool kFp = MvFormat<FMT>::fp;
    constexpr int T = MvFormat<FMT>::terms;
    FormatSpec fs;
    weight_format_spec(FMT, &fs);
    uint8_t* wt = lds;
    float* xs = reinterpret_cast<float*>(lds + L.R * L.stride);
    float* terms = xs + xwords(L.slab_cols);
    float* aux = terms + L.R * kMvTermStride;
    const long long r0 = static_cast<long long>(blockIdx.x) * L.R;
    const int nrows = static_cast<int>(min(static_cast<long long>(L.R), a.rows - r0));
    const int q = blockIdx.y;
    const float* x = a.x + static_cast<long long>(q) * a.cols;
    const int t = threadIdx.x;
    const uint8_t* W = a.w + r0 * a.row_bytes;

    float rowsum = 0.0f;  // Q formats: thread t < nrows
    float acc = 0.0f;     // fp formats: thread (row t / 8, lane t % 8)
    const int frow = min(t >> 3, nrows - 1), lane = t & 7;

    for (int c0 = 0; c0 < a.cols; c0 += L.slab_cols) {
        const int cols = min(L.slab_cols, a.cols - c0);
        const int nbs = cols / fs.block;
        const int sbytes = nbs * fs.bytes;
        if (c0 > 0) __syncthreads();  // the previous slab is consumed
        mv_stage<G>(W + static_cast<long long>(c0 / fs.block) * fs.bytes, a.row_bytes, sbytes, nrows, wt, L.stride,
                    x + c0, xs, cols);
        __syncthreads();

        if constexpr (kFp) {
            if ((t >> 3) < L.R) {
                const uint8_t* row = wt + frow * L.stride;
                for (int c = 0; c < cols; c += 64) {
                    float wv[8], xv[8];
#pragma unroll
                    for (int s = 0; s < 8; ++s) {
                        const int k = min(c + 8 * s, cols - 8) + lane;
                        wv[s] = fp_weight<FMT>(row, k);
                        xv[s] = xs[xpad(k)];
                    }
#pragma unroll
                    for (int s = 0; s < 8; ++s)
                        if (c + 8 * s < cols) acc = add_rn(acc, mul_rn(wv[s], xv[s]));
                }
            }
        } else {
            // x-only block sums
            if constexpr (FMT == QR_FMT_Q4_0) {
                for (int i = t; i < nbs; i += kMvThreads) {
                    const float* xb = xs + kXGroup * i;
                    float ax[8];
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        float s = 0.0f;
                        s = add_rn(s, xb[l]);
                        s = add_rn(s, xb[8 + l]);
                        s = add_rn(s, xb[16 + l]);
                        s = add_rn(s, xb[24 + l]);
                        ax[l] = s;
                    }
                    aux[i] = hsum8(ax);
                }
                __syncthreads();
            } else if constexpr (FMT == QR_FMT_Q4_K) {
                for (int i = t; i < nbs * 8; i += kMvThreads) {
                    const float* xg = xs + kXGroup * i;
                    float v[32];
#pragma unroll
                    for (int k = 0; k < 32; ++k) v[k] = xg[k];
                    float s = 0.0f;
#pragma unroll
                    for (int k = 0; k < 32; ++k) s = add_rn(s, v[k]);
                    aux[i] = s;
                }
                __syncthreads();
            }
            // rows vary fastest: threads of one block read the same x (broadcast)
            for (int i = t; i < nrows * nbs; i += kMvThreads) {
                const int blk = i / nrows, row = i - blk * nrows;
                const uint8_t* p = wt + row * L.stride + blk * fs.bytes;
                float* out = terms + row * kMvTermStride + blk * T;
                if constexpr (FMT == QR_FMT_Q8_0) out[0] = term_q8_0(p, xs + kXGroup * blk);
                else if constexpr (FMT == QR_FMT_Q4_0) out[0] = term_q4_0(p, xs + kXGroup * blk, aux[blk]);
                else if constexpr (FMT == QR_FMT_Q4_K) terms_q4_k(p, xs + kXGroup * 8 * blk, aux + 8 * blk, out);
                else out[0] = term_q6_k(p, xs + kXGroup * 8 * blk);
            }
            __syncthreads();
            if (t < nrows) {  // in order, reading 16 terms per batch
                const float* tr = terms + t * kMvTermStride;
                const int nt = nbs * T;
                for (int j = 0; j < nt; j += 16) {
                    float v[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) v[k] = tr[min(j + k, nt - 1)];
#pragma unroll
                    for (int k = 0; k < 16; ++k)
                        if (j + k < nt) rowsum = add_rn(rowsum, v[k]);
                }
            }
        }
    }

    float* y = a.y + static_cast<long long>(q) * a.rows + r0;
    if constexpr (kFp) {
        // HSum in lane order over the 8 consecutive threads of a row
        const int base = (threadIdx.x & 63) & ~7;
        float s = 0.0f;
#pragma unroll
        for (int l = 0; l < 8; ++l) s = add_rn(s, __shfl(acc, base + l, 64));
        if (lane == 0 && (t >> 3) < nrows) y[t >> 3] = s;
    } else {
        if (t < nrows) y[t] = rowsum;
    }
}

// Persistent form of matvec_body for one slab (cols <= kMvSlabCols) and 16-byte
// staging of at most one batch per tile: x and its block sums are staged once per
// workgroup, and the loads of tile i+grid are held in registers while tile i is computed.
template <int FMT>
__device__ __forceinline__ void matvec_persistent(const MatVecArgs& a, const MvLayout& L, uint8_t* lds) {
    typedef u32x4_t V;
    constexpr int T = MvFormat<FMT>::terms;
    constexpr int UPB = FMT == QR_FMT_Q4_K ? 4 : 1;  // work items per block (Q4_K: sub-block pairs)
    FormatSpec fs;
    weight_format_spec(FMT, &fs);
    uint8_t* wt = lds;
    float* xs = reinterpret_cast<float*>(lds + L.R * L.stride);
    float* terms = xs + xwords(L.slab_cols);
    float* aux = terms + L.R * L.tstride;
    const int t = threadIdx.x;
    const int q = blockIdx.y;
    const float* x = a.x + static_cast<long long>(q) * a.cols;
    const int nbs = a.cols / fs.block;
    const int per_row = nbs * fs.bytes / 16;
    const long long ntiles = (a.rows + L.R - 1) / L.R;

    V v[kMvStageBatch];
    int dst[kMvStageBatch];
    auto load_tile = [&](long long it) {
        const long long r0 = it * L.R;
        const int nrows = static_cast<int>(min(static_cast<long long>(L.R), a.rows - r0));
        const int total = per_row * nrows;
        const uint8_t* src = a.w + r0 * a.row_bytes;
#pragma unroll
        for (int s = 0; s < kMvStageBatch; ++s) {
            const int idx = t + s * kMvThreads;
            const int i = min(idx, total - 1);
            const int r = i / per_row, e = i - r * per_row;
            v[s] = *reinterpret_cast<const V*>(src + r * a.row_bytes + e * 16);
            dst[s] = idx < total ? r * L.stride + e * 16 : -1;
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int s = 0; s < kMvStageBatch; ++s)
            if (dst[s] >= 0) *reinterpret_cast<V*>(wt + dst[s]) = v[s];
    };

    long long it = blockIdx.x;
    if (it < ntiles) load_tile(it);
    {  // x, padded, with the first tile's loads in flight
        float4 xv[kMvPersistXLoads];
        const int nx = a.cols / 4;
#pragma unroll
        for (int s = 0; s < kMvPersistXLoads; ++s)
            xv[s] = reinterpret_cast<const float4*>(x)[min(t + s * kMvThreads, nx - 1)];
#pragma unroll
        for (int s = 0; s < kMvPersistXLoads; ++s) {
            const int i = t + s * kMvThreads;
            if (i < nx) {
                float* d = xs + xpad(4 * i);
                d[0] = xv[s].x;
                d[1] = xv[s].y;
                d[2] = xv[s].z;
                d[3] = xv[s].w;
            }
        }
    }
    if (it < ntiles) store_tile();
    __syncthreads();
    if constexpr (FMT == QR_FMT_Q4_0) {
        for (int i = t; i < nbs; i += kMvThreads) {
            const float* xb = xs + kXGroup * i;
            float ax[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                float sx = 0.0f;
                sx = add_rn(sx, xb[l]);
                sx = add_rn(sx, xb[8 + l]);
                sx = add_rn(sx, xb[16 + l]);
                sx = add_rn(sx, xb[24 + l]);
                ax[l] = sx;
            }
            aux[i] = hsum8(ax);
        }
        __syncthreads();
    } else if constexpr (FMT == QR_FMT_Q4_K) {
        for (int i = t; i < nbs * 8; i += kMvThreads) {
            const float* xg = xs + kXGroup * i;
            float vv[32];
#pragma unroll
            for (int k = 0; k < 32; ++k) vv[k] = xg[k];
            float sx = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; ++k) sx = add_rn(sx, vv[k]);
            aux[i] = sx;
        }
        __syncthreads();
    }

    for (; it < ntiles; it += gridDim.x) {
        const long long next = it + gridDim.x;
        if (next < ntiles) load_tile(next);  // in flight while this tile is computed
        const long long r0 = it * L.R;
        const int nrows = static_cast<int>(min(static_cast<long long>(L.R), a.rows - r0));
        const int nitems = nrows * nbs * UPB;
        for (int i = t; i < nitems; i += kMvThreads) {
            const int unit = i / nrows, row = i - unit * nrows;  // rows vary fastest
            const int blk = unit / UPB;
            const uint8_t* p = wt + row * L.stride + blk * fs.bytes;
            float* out = terms + row * L.tstride + blk * T;
            if constexpr (FMT == QR_FMT_Q8_0) out[0] = term_q8_0(p, xs + kXGroup * blk);
            else if constexpr (FMT == QR_FMT_Q4_0) out[0] = term_q4_0(p, xs + kXGroup * blk, aux[blk]);
            else if constexpr (FMT == QR_FMT_Q4_K) {
                const int j = unit - blk * UPB;
                terms_q4_k_pair(p, j, xs + kXGroup * 8 * blk, aux + 8 * blk, out + 2 * j);
            } else out[0] = term_q6_k(p, xs + kXGroup * 8 * blk);
        }
        __syncthreads();
        if (t < nrows) {  // in order, 64 terms (16 float4 reads) per batch
            const float4* tr = reinterpret_cast<const float4*>(terms + t * L.tstride);
            const int nt = nbs * T;
            float sum = 0.0f;
            for (int j = 0; j < nt; j += 64) {
                float4 vv[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) vv[k] = tr[min(j / 4 + k, (nt - 1) / 4)];
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const int base = j + 4 * k;
                    if (base + 0 < nt) sum = add_rn(sum, vv[k].x);
                    if (base + 1 < nt) sum = add_rn(sum, vv[k].y);
                    if (base + 2 < nt) sum = add_rn(sum, vv[k].z);
                    if (base + 3 < nt) sum = add_rn(sum, vv[k].w);
                }
            }
            a.y[static_cast<long long>(q) * a.rows + r0 + t] = sum;
        }
        if (next < ntiles) {
            __syncthreads();  // this tile's weights and terms are consumed
            store_tile();
            __syncthreads();
        }
    }
}

template <int FMT>
__global__ __launch_bounds__(kMvThreads) void matvec_kernel(MatVecArgs a, MvLayout L) {
    extern __shared__ __align__(16) uint8_t mv_lds[];
    if constexpr (!MvFormat<FMT>::fp) {
        if (L.persistent) {
            matvec_persistent<FMT>(a, L, mv_lds);
            return;
        }
    }
    if (L.copy_bytes == 16) matvec_body<FMT, 16>(a, L, mv_lds);
    else if (L.copy_bytes == 4) matvec_body<FMT, 4>(a, L, mv_lds);
    else matvec_body<FMT, 2>(a, L, mv_lds);
}


MvLayout mv_layout(const MatVecArgs& a) {
    FormatSpec fs;
    weight_format_spec(a.fmt, &fs);
    MvLayout L{};
    L.slab_cols = std::min(a.cols, kMvSlabCols);
    const int slab_bytes = L.slab_cols / fs.block * fs.bytes;
    const bool fp = a.fmt == QR_FMT_F32 || a.fmt == QR_FMT_F16 || a.fmt == QR_FMT_BF16;
    int R = std::max(1, std::min(kMvMaxRows, kMvTileBytes / slab_bytes));
    if (fp) R = std::min(R, kMvThreads / 8);
    // at least ~2 workgroups per CU when the rows allow it
    const long long want = 512 / std::max(1, a.nq);
    if (a.rows / want < R) R = static_cast<int>(std::max(1LL, a.rows / std::max(1LL, want)));
    R = static_cast<int>(std::min<long long>(R, a.rows));
    L.R = R;
    L.stride = (slab_bytes + 15) / 16 * 16 + 16;
    const uintptr_t base = reinterpret_cast<uintptr_t>(a.w);
    auto aligned = [&](int g) { return base % g == 0 && a.row_bytes % g == 0 && slab_bytes % g == 0; };
    L.copy_bytes = aligned(16) ? 16 : aligned(4) ? 4 : 2;
    L.persistent = 0;
    L.tstride = 0;
    const long long row_bytes = a.row_bytes;
    if (!fp && a.cols <= kMvPersistMaxCols && row_bytes % 16 == 0 && base % 16 == 0 &&
        row_bytes <= static_cast<long long>(kMvThreads) * kMvStageBatch * 16) {
        // the whole row is one slab; tiles of at most one batch of 16-byte copies, about two
        // or more per workgroup
        L.slab_cols = a.cols;
        const int rbytes = static_cast<int>(row_bytes);
        const int rmax = std::max(1, std::min(kMvMaxRows, kMvThreads * kMvStageBatch * 16 / rbytes));
        L.R = static_cast<int>(std::max(1LL, std::min<long long>(rmax, a.rows / 1024)));
        L.stride = (rbytes + 15) / 16 * 16 + 16;
        L.copy_bytes = 16;
        const int nt = a.cols / fs.block * (a.fmt == QR_FMT_Q4_K ? 8 : 1);
        L.tstride = (nt + 3) / 4 * 4 + 4;
        L.persistent = 1;
    }
    return L;
}

constexpr int kBlkRptQ4k = 2;  // Q4_K rows per thread and tile (Q8_0: 1, its 17 loads a row)
constexpr int kBlkWgPerCu = 2;  // workgroups of 256 threads per CU (measured: 1 and 3 slower for Q4_K)

template <int U>
hipError_t ring_launch_q8(const MatVecArgs& a, const MvRing& k, const BlkGroup& gr, dim3 grid, size_t lds,
                          hipStream_t stream) {
    static bool attr = false;  // dynamic LDS above 64 KiB must be allowed per kernel
    if (lds > 64 * 1024 && !attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&matvec_blk_ring<PolQ8, 1, U>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr = true;
    }
    hipLaunchKernelGGL((matvec_blk_ring<PolQ8, 1, U>), grid, dim3(kMvThreads), lds, stream, a, k, gr);
    return hipGetLastError();
}

// The ring form, used for Q8_0 (Q4_K is VALU-bound and measures faster in the persistent
// form): block pairs, rows of at most 256 pairs (16384 columns), tiles of at most 32 KiB;
// false when the shape does not fit.
// Workgroups of a group launch: `budget` split over the matrices in proportion to their
// tiles (at least one each, at most one per tile), doubled while the terms of a workgroup's
// tiles (`per_tile` bytes each, after `fixed` bytes) exceed `target` bytes of LDS.  Returns
// the LDS bytes; start[] gets the workgroup ranges.
size_t group_grid(BlkGroup& gr, int budget, size_t fixed, size_t per_tile, size_t target) {
    long long total = 0;
    for (int m = 0; m < gr.n; ++m) total += gr.ntiles[m];
    int G[kMatVecGroupMax];
    for (int m = 0; m < gr.n; ++m)
        G[m] = static_cast<int>(std::max<long long>(1, std::min<long long>(gr.ntiles[m], static_cast<long long>(budget) * gr.ntiles[m] / total)));
    size_t lds = 0;
    for (;;) {
        int tpw = 1;
        bool full = true;
        for (int m = 0; m < gr.n; ++m) {
            tpw = std::max(tpw, (gr.ntiles[m] + G[m] - 1) / G[m]);
            full = full && G[m] == gr.ntiles[m];
        }
        lds = fixed + static_cast<size_t>(tpw) * per_tile;
        if (lds <= target || full) break;
        for (int m = 0; m < gr.n; ++m) G[m] = std::min(gr.ntiles[m], 2 * G[m]);
    }
    gr.start[0] = 0;
    for (int m = 0; m < gr.n; ++m) gr.start[m + 1] = gr.start[m] + G[m];
    return lds;
}

BlkGroup group_of(const MatVecArgs* a, int n, int R) {
    BlkGroup gr{};
    gr.n = n;
    for (int m = 0; m < n; ++m) {
        gr.w[m] = a[m].w;
        gr.rows[m] = a[m].rows;
        gr.y[m] = a[m].y;
        gr.ntiles[m] = static_cast<int>((a[m].rows + R - 1) / R);
    }
    return gr;
}

// Q8_0 (block pairs, 4-byte aligned rows) in the ring form, for one matrix or a group that
// shares x: false when the shape does not fit it.
bool blk_ring_launch(const MatVecArgs* a, int n, hipStream_t stream, hipError_t* err) {
    for (int m = 0; m < n; ++m)
        if (a[m].fmt != QR_FMT_Q8_0 || reinterpret_cast<uintptr_t>(a[m].x) % 16 || a[m].cols % 64 ||
            reinterpret_cast<uintptr_t>(a[m].w) % 4 || a[m].row_bytes % 4 || a[m].rows < 1)
            return false;
    MvRing k{};
    k.P = a[0].cols / 64;
    if (k.P > 256) return false;
    k.tpg = k.P <= 64 ? 64 : k.P <= 128 ? 128 : 256;  // four waves always: U units per wave per tile
    k.rg = kMvThreads / k.tpg;
    k.R = k.rg;
    const long long tile = static_cast<long long>(k.R) * a[0].row_bytes;
    int U = static_cast<int>((tile + 4095) / 4096);
    if (U > 8) return false;
    if (U == 7) U = 8;
    k.slot_bytes = 4096 * U;
    k.tstride = (2 * k.P + 3) / 4 * 4 + 4;
    long long groups_total = 0;
    for (int m = 0; m < n; ++m) {
        if (a[m].rows >= (1LL << 31) - k.R) return false;
        groups_total += (a[m].rows + k.R - 1) / k.R;
    }
    if (groups_total >= (1LL << 31)) return false;
    BlkGroup gr = group_of(a, n, k.R);
    k.ntiles = gr.ntiles[0];
    // workgroups: two per CU when the LDS allows, the terms of all of a workgroup's tiles kept
    const size_t lds = group_grid(gr, 512, static_cast<size_t>(kRingSlots) * k.slot_bytes,
                                  static_cast<size_t>(k.R) * k.tstride * 4, 80 * 1024);
    if (lds > 160 * 1024) return false;
    const dim3 grid(static_cast<unsigned>(gr.start[n]), static_cast<unsigned>(a[0].nq));
    switch (U) {
    case 1: case 2: *err = ring_launch_q8<2>(a[0], k, gr, grid, lds, stream); break;
    case 3: *err = ring_launch_q8<3>(a[0], k, gr, grid, lds, stream); break;
    case 4: *err = ring_launch_q8<4>(a[0], k, gr, grid, lds, stream); break;
    case 5: *err = ring_launch_q8<5>(a[0], k, gr, grid, lds, stream); break;
    case 6: *err = ring_launch_q8<6>(a[0], k, gr, grid, lds, stream); break;
    default: *err = ring_launch_q8<8>(a[0], k, gr, grid, lds, stream); break;
    }
    return true;
}

// The persistent form for Q4_K (64-column items: rows of at most 512 items, 32768 columns) and
// Q8_0 (block pairs: whole pairs and 4-byte aligned rows): false when the shape does not fit or
// the terms of a workgroup's tiles would not fit in 64 KiB of LDS.
bool blk_persistent_launch(const MatVecArgs* a, int n, hipStream_t stream, hipError_t* err) {
    const bool q4k = a[0].fmt == QR_FMT_Q4_K, q8 = a[0].fmt == QR_FMT_Q8_0;
    long long rows_total = 0;
    for (int m = 0; m < n; ++m) {
        if (!(q4k || q8) || a[m].fmt != a[0].fmt || reinterpret_cast<uintptr_t>(a[m].x) % 16 || a[m].cols % 64 ||
            a[m].rows < 1)
            return false;
        if (q4k && (reinterpret_cast<uintptr_t>(a[m].w) % 16 || a[m].row_bytes % 16)) return false;
        if (q8 && (reinterpret_cast<uintptr_t>(a[m].w) % 4 || a[m].row_bytes % 4)) return false;
        rows_total += a[m].rows;
    }
    MvBlkP k{};
    k.P = a[0].cols / 64;
    if (k.P > 512) return false;
    k.tpg = (k.P + 63) / 64 * 64;
    k.rg = std::max(1, kMvThreads / k.tpg);
    // rows per thread and tile: loads of two tiles in flight stay within the 63 that vmcnt counts;
    // Q4_K launches with fewer than 1024 tiles of kBlkRptQ4k rows per thread take one row per
    // thread (twice the tiles: their runtime is the latency of a workgroup's few tiles; at the
    // 8B shape the wq/wk/wv group and wo: 46.4-47.1 us per layer against 47.4-49.8 with the
    // bound at 512 tiles)
    int rpt = 1;
    if (q4k) rpt = (rows_total + k.rg * kBlkRptQ4k - 1) / (k.rg * kBlkRptQ4k) < 1024 ? 1 : kBlkRptQ4k;
    k.R = k.rg * rpt;
    k.tstride = (2 * k.P + 3) / 4 * 4 + 4;
    for (int m = 0; m < n; ++m)
        if (static_cast<long long>(k.R) * a[m].row_bytes >= (1LL << 31) || a[m].rows >= (1LL << 31) - k.R) return false;
    if ((rows_total + k.R - 1) / k.R >= (1LL << 31)) return false;
    BlkGroup gr = group_of(a, n, k.R);
    k.ntiles = gr.ntiles[0];
    const int threads = k.rg * k.tpg;
    const int wg_per_cu = std::max(1, kBlkWgPerCu * 256 / threads);
    // LDS: the terms of the workgroup's tiles, or the padded copy of x that precedes them;
    // more workgroups (fewer tiles each) when the terms would not fit
    const size_t xbytes = static_cast<size_t>(k.P) * kXRow * 4;
    size_t lds = group_grid(gr, 256 * wg_per_cu, 0, static_cast<size_t>(k.R) * k.tstride * 4, 160 * 1024);
    lds = std::max(lds, xbytes);
    if (lds > 160 * 1024) return false;
    const int which = q4k ? (rpt == 1 ? 1 : 2) : 0;
    const void* fns[3] = {reinterpret_cast<const void*>(&matvec_blk_persistent<PolQ8, 1>),
                          reinterpret_cast<const void*>(&matvec_blk_persistent<PolQ4K, 1>),
                          reinterpret_cast<const void*>(&matvec_blk_persistent<PolQ4K, kBlkRptQ4k>)};
    static bool attr[3] = {false, false, false};  // dynamic LDS above 64 KiB must be allowed per kernel
    if (lds > 64 * 1024 && !attr[which]) {
        *err = hipFuncSetAttribute(fns[which], hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (*err != hipSuccess) return true;
        attr[which] = true;
    }
    const dim3 grid(static_cast<unsigned>(gr.start[n]), static_cast<unsigned>(a[0].nq));
    if (which == 2)
        hipLaunchKernelGGL((matvec_blk_persistent<PolQ4K, kBlkRptQ4k>), grid, dim3(threads), lds, stream, a[0], k, gr);
    else if (which == 1)
        hipLaunchKernelGGL((matvec_blk_persistent<PolQ4K, 1>), grid, dim3(threads), lds, stream, a[0], k, gr);
    else
        hipLaunchKernelGGL((matvec_blk_persistent<PolQ8, 1>), grid, dim3(threads), lds, stream, a[0], k, gr);
    *err = hipGetLastError();
    return true;
}

template <int FMT>
hipError_t launch_fmt(const MatVecArgs& a, hipStream_t stream) {
    const MvLayout L = mv_layout(a);
    static bool attr_set = false;  // dynamic LDS above 64 KiB must be allowed per kernel
    if (L.lds_bytes() > 65536 && !attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&matvec_kernel<FMT>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const long long tiles = (a.rows + L.R - 1) / L.R;
    // persistent: as many workgroups as stay resident (LDS-bound), at most two per CU
    const long long resident = 256LL * std::max<long long>(1, std::min<long long>(2, 160 * 1024 / L.lds_bytes()));
    const dim3 grid(static_cast<unsigned>(L.persistent ? std::min(tiles, resident) : tiles), static_cast<unsigned>(a.nq));
    hipLaunchKernelGGL((matvec_kernel<FMT>), grid, dim3(kMvThreads), L.lds_bytes(), stream, a, L);
    return hipGetLastError();
}

}  // namespace

bool matvec_shape_ok(int fmt, int cols) {
    FormatSpec fs;
    if (!weight_format_spec(fmt, &fs) || cols < 1 || cols % fs.block) return false;
    const bool fp = fmt == QR_FMT_F32 || fmt == QR_FMT_F16 || fmt == QR_FMT_BF16;
    return !fp || cols % 8 == 0;
}

// The single-wave fp form needs 16-byte aligned rows and x.
bool fp_wave_fits(const MatVecArgs& a) {
    return reinterpret_cast<uintptr_t>(a.w) % 16 == 0 && a.row_bytes % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && a.cols % 8 == 0;
}

template <int FMT>
hipError_t launch_fp_group(const MatVecArgs& a, const FwGroup& g, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(g.start[g.n]), static_cast<unsigned>(a.nq));
    hipLaunchKernelGGL((matvec_fp_wave<FMT, 8>), grid, dim3(64), 0, stream, a, g);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_fp(const MatVecArgs& a, hipStream_t stream) {
    if (!fp_wave_fits(a)) return launch_fmt<FMT>(a, stream);
    FwGroup g{};
    g.n = 1;
    g.start[1] = static_cast<int>((a.rows + 7) / 8);
    g.w[0] = a.w;
    g.rows[0] = a.rows;
    g.y[0] = a.y;
    return launch_fp_group<FMT>(a, g, stream);
}

hipError_t launch_matvec(const MatVecArgs& a, hipStream_t stream) {
    if (a.nq == 0 || a.rows == 0) return hipSuccess;
    switch (a.fmt) {
    case QR_FMT_F32: return launch_fp<QR_FMT_F32>(a, stream);
    case QR_FMT_F16: return launch_fp<QR_FMT_F16>(a, stream);
    case QR_FMT_BF16: return launch_fp<QR_FMT_BF16>(a, stream);
    case QR_FMT_Q4_0: return launch_fmt<QR_FMT_Q4_0>(a, stream);
    case QR_FMT_Q8_0: {
        hipError_t e;
        if (blk_ring_launch(&a, 1, stream, &e)) return e;
        if (blk_persistent_launch(&a, 1, stream, &e)) return e;
        return launch_fmt<QR_FMT_Q8_0>(a, stream);
    }
    case QR_FMT_Q4_K: {
        hipError_t e;
        if (blk_persistent_launch(&a, 1, stream, &e)) return e;
        return launch_fmt<QR_FMT_Q4_K>(a, stream);
    }
    case QR_FMT_Q6_K: return launch_fmt<QR_FMT_Q6_K>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec_group(const MatVecArgs* a, int n, hipStream_t stream) {
    // F32/F16/BF16 rows in the single-wave form: one launch for the group
    bool one = n > 1 && (a[0].fmt == QR_FMT_F32 || a[0].fmt == QR_FMT_F16 || a[0].fmt == QR_FMT_BF16);
    long long wgs = 0;
    for (int m = 0; one && m < n; ++m) {
        one = fp_wave_fits(a[m]) && a[m].fmt == a[0].fmt && a[m].cols == a[0].cols &&
              a[m].row_bytes == a[0].row_bytes && a[m].x == a[0].x && a[m].nq == a[0].nq && a[m].rows > 0;
        wgs += (a[m].rows + 7) / 8;
    }
    if (!one && n > 1 && a[0].nq > 0) {
        // Q8_0 / Q4_K matrices of one x: one launch of the ring or persistent form
        bool same = true;
        for (int m = 1; m < n; ++m)
            same = same && a[m].fmt == a[0].fmt && a[m].cols == a[0].cols && a[m].row_bytes == a[0].row_bytes &&
                   a[m].x == a[0].x && a[m].nq == a[0].nq;
        hipError_t e = hipSuccess;
        if (same && a[0].fmt == QR_FMT_Q8_0 && (blk_ring_launch(a, n, stream, &e) || blk_persistent_launch(a, n, stream, &e)))
            return e;
        if (same && a[0].fmt == QR_FMT_Q4_K && blk_persistent_launch(a, n, stream, &e)) return e;
    }
    if (!one || a[0].nq == 0 || wgs >= (1LL << 31)) {
        for (int m = 0; m < n; ++m) {
            const hipError_t e = launch_matvec(a[m], stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    FwGroup g{};
    g.n = n;
    for (int m = 0; m < n; ++m) {
        g.w[m] = a[m].w;
        g.rows[m] = a[m].rows;
        g.y[m] = a[m].y;
        g.start[m + 1] = g.start[m] + static_cast<int>((a[m].rows + 7) / 8);
    }
    switch (a[0].fmt) {
    case QR_FMT_F32: return launch_fp_group<QR_FMT_F32>(a[0], g, stream);
    case QR_FMT_F16: return launch_fp_group<QR_FMT_F16>(a[0], g, stream);
    default: return launch_fp_group<QR_FMT_BF16>(a[0], g, stream);
    }
}

}  // namespace qr
