// qr_mla.hip -- MLA absorbed attention over the paged latent cache (gfx950).
//
// Replaces the score -> softmax -> latent-sum loops of StreamingEngine.MlaLayer
// (StreamingEngine.cs:531-568).  Latent pages are token-major rows of
// kv_lora + rope elements ([c_kv | k_pe], StreamingEngine.cs:494-506).
//
// mla_mfma_kernel (bf16/f16 latents, kv_lora 512, rope 0 or 64): MFMA tiles, see
//   below; splits merged by mla_combine_wide_kernel.
// mla_split_generic_kernel: one workgroup per (split of 256 positions, head).
//   Scores of the split are staged in LDS; the split's partial (max, sum,
//   unnormalised u) is merged across splits by mla_combine_kernel.  This path
//   serves every other shape and the fp32 cache.
#include "qr_mla.hpp"

#include <algorithm>
#include <type_traits>

namespace qr {
namespace {

constexpr int kThreads = 256;
constexpr int kGenericSplit = kPageTokens;

struct MlaK {
    const char* pool;
    const int* page_table;
    int dtype;
    int kv_lora, rope, width;
    int heads;
    int seq_len;
    int split_tokens;
    int splits;
    const float* q_tilde;
    const float* q_rope;
    float* u;
    float* part_u;     // [heads][splits][kv_lora]
    float2* part_ml;   // [heads][splits]
    float qscale;      // scale * log2(e)
};

__device__ __forceinline__ float load_elem(const char* pool, int dtype, long long i) {
    switch (dtype) {
        case QR_DTYPE_F32: return reinterpret_cast<const float*>(pool)[i];
        case QR_DTYPE_F16: return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(pool)[i]);
        default: return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(pool)[i]);
    }
}

__device__ __forceinline__ long long row_base(const MlaK& p, int t) {
    const long long phys = p.page_table[t >> kPageShift];
    return (phys * kPageTokens + (t & (kPageTokens - 1))) * p.width;
}

__global__ void __launch_bounds__(kThreads) mla_split_generic_kernel(const MlaK p) {
    const int split = blockIdx.x;
    const int h = blockIdx.y;
    const int t0 = split * p.split_tokens;
    const int t1 = min(p.seq_len, t0 + p.split_tokens);
    const int n = t1 - t0;

    __shared__ float sq[kMlaMaxLora + kMlaMaxRope];
    __shared__ float sp[kGenericSplit];
    __shared__ float red[kThreads];

    for (int k = threadIdx.x; k < p.width; k += kThreads)
        sq[k] = (k < p.kv_lora ? p.q_tilde[static_cast<size_t>(h) * p.kv_lora + k]
                               : p.q_rope[static_cast<size_t>(h) * p.rope + (k - p.kv_lora)]) * p.qscale;
    __syncthreads();

    // scores (log2 units) of this split, one position per thread
    float s = -INFINITY;
    if (static_cast<int>(threadIdx.x) < n) {
        const long long base = row_base(p, t0 + threadIdx.x);
        float d = 0.f;
        for (int k = 0; k < p.width; ++k) d = fmaf(sq[k], load_elem(p.pool, p.dtype, base + k), d);
        s = d;
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    const float m = red[0];
    __syncthreads();
    const float e = (static_cast<int>(threadIdx.x) < n) ? fast_exp2(s - m) : 0.f;
    if (threadIdx.x < kGenericSplit) sp[threadIdx.x] = e;
    red[threadIdx.x] = e;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float l = red[0];

    // unnormalised latent sum over the split
    const size_t slot = static_cast<size_t>(h) * p.splits + split;
    for (int k = threadIdx.x; k < p.kv_lora; k += kThreads) {
        float acc = 0.f;
        for (int i = 0; i < n; ++i) acc = fmaf(sp[i], load_elem(p.pool, p.dtype, row_base(p, t0 + i) + k), acc);
        if (p.splits == 1) p.u[static_cast<size_t>(h) * p.kv_lora + k] = acc / l;
        else p.part_u[slot * p.kv_lora + k] = acc;
    }
    if (threadIdx.x == 0 && p.splits > 1) p.part_ml[slot] = make_float2(m, l);
}

__global__ void __launch_bounds__(kThreads) mla_combine_kernel(const MlaK p) {
    const int h = blockIdx.x;
    const size_t base = static_cast<size_t>(h) * p.splits;
    __shared__ float w[4096];
    __shared__ float red[kThreads];
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < p.splits; s += kThreads) mx = fmaxf(mx, p.part_ml[base + s].x);
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();
    float ls = 0.f;
    for (int s = threadIdx.x; s < p.splits; s += kThreads) {
        const float2 ml = p.part_ml[base + s];
        const float c = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - M);
        w[s] = c;
        ls += ml.y * c;
    }
    red[threadIdx.x] = ls;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float L = red[0];
    for (int k = threadIdx.x; k < p.kv_lora; k += kThreads) {
        float o = 0.f;
        for (int s = 0; s < p.splits; ++s) o = fmaf(p.part_u[(base + s) * p.kv_lora + k], w[s], o);
        p.u[static_cast<size_t>(h) * p.kv_lora + k] = o / L;
    }
}

// ---------------------------------------------------------------------------
// MFMA path for 16-bit latents (kv_lora 512, rope 0 or 64).
//
// Workgroup = 4 waves = 64 heads (16 per wave) over one split of the sequence.
// The split is walked in tiles of 32 positions; each tile is staged in LDS twice:
// row-major [token][kv_lora+rope] (QK operand) and transposed [dim][token] over the
// first kv_lora dims (PV operand), so every MFMA operand is one or two vector LDS
// reads.  v_mfma_f32_16x16x32_{bf16,f16} lane layout (verified on gfx950):
//   A[m = lane%16][k = 8*(lane/16)+i], B[k = 8*(lane/16)+i][n = lane%16],
//   D[m = 4*(lane/16)+r][n = lane%16].
//   QK: S^T[token][head] = C[token][dims] . q~^T[dims][head]      (M tokens, N heads)
//   PV: U^T[dim][head]  += C^T[dim][tokens] . P^T[tokens][head]    (M dims,   N heads)
// In PV the 8 k-slots of lane quarter q are tokens {4q..4q+3, 16+4q..16+4q+3}: exactly
// the 8 scores that lane holds after QK, so P goes from the QK result straight into
// the B operand.  Each lane owns one head (lane%16) in both results, so the online
// softmax rescale of its U tiles is lane-local.
// Operands are fp16 for both 16-bit cache types: bf16 latents are widened to fp16
// while the tile is staged (exact for |x| in the fp16 range, 2^-24..65504), which
// keeps 11 mantissa bits for q~ and P instead of bf16's 8.  q~ is pre-multiplied per
// head by a power of two that brings its largest element to at most 2^14 (exact) and
// the scores are scaled back, so q~ never overflows fp16.
constexpr int kTileTok = 32;
constexpr int kMfmaLora = 512;
constexpr int kMfmaHeads = 64;  // per workgroup

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma16;
template <> struct Mfma16<__bf16> {
    using vec = bf16x8_t;
    __device__ static f32x4_t mma(vec a, vec b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
    __device__ static __bf16 from_f32(float x) { return static_cast<__bf16>(x); }  // round to nearest even
    __device__ static float to_f32(__bf16 x) { return static_cast<float>(x); }
};
template <> struct Mfma16<_Float16> {
    using vec = f16x8_t;
    __device__ static f32x4_t mma(vec a, vec b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
    __device__ static _Float16 from_f32(float x) { return static_cast<_Float16>(x); }
    __device__ static float to_f32(_Float16 x) { return static_cast<float>(x); }
};

struct MlaMK {
    const char* pool;
    const int* page_table;
    int heads;
    int seq_len;
    int split_tokens;
    int splits;
    const float* q_tilde;
    const float* q_rope;
    float* u;
    float* part_u;     // [heads][splits][kv_lora]
    float2* part_ml;   // [heads][splits]
    float qscale;      // scale * log2(e)
};

template <bool SRC_BF16, int KR>
__global__ void __launch_bounds__(256) mla_mfma_kernel(const MlaMK p) {
    using T = _Float16;
    using M = Mfma16<T>;
    using V = typename M::vec;
    constexpr int KL = kMfmaLora;
    constexpr int W = KL + KR;             // latent width
    constexpr int NK = W / 32;              // QK k-steps
    constexpr int NT = KL / 16;             // PV dim tiles
    constexpr int RS = W * 2 + 16;          // row-major LDS row stride (bytes), padded
    constexpr int TS = kTileTok * 2 + 8;    // transposed LDS row stride (bytes), padded
    constexpr int CHUNKS = kTileTok * W / 8; // 16-byte chunks per tile
    constexpr int CPT = (CHUNKS + 255) / 256;

    __shared__ __attribute__((aligned(16))) char lds_rm[kTileTok * RS];
    __shared__ __attribute__((aligned(16))) char lds_tr[KL * TS];

    const int split = blockIdx.x;
    const int hg = blockIdx.y;
    const int t_begin = split * p.split_tokens;
    const int t_end = min(p.seq_len, t_begin + p.split_tokens);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int q4 = lane >> 4;                // lane quarter
    const int hl = lane & 15;
    const int head = hg * kMfmaHeads + wave * 16 + hl;
    const int hq = min(head, p.heads - 1);

    // ---- q~ (and q_rope) as B operands: lane holds dims 32*kk + 8*q4 .. +8 of head hl,
    // scaled by 2^-e so the head's largest |element| is at most 2^14
    float qf[NK][8];
    float amax = 0.f;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int d = 32 * kk + 8 * q4 + i;
            const float x = d < KL ? p.q_tilde[static_cast<size_t>(hq) * KL + d]
                                   : p.q_rope[static_cast<size_t>(hq) * KR + (d - KL)];
            qf[kk][i] = x;
            amax = fmaxf(amax, fabsf(x));
        }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    int qexp = 0;
    if (amax > 16384.f) qexp = static_cast<int>(ceilf(log2f(amax / 16384.f)));
    const float qdown = ldexpf(1.f, -qexp);
    const float sscale = p.qscale * ldexpf(1.f, qexp);  // score scale, undoing the q~ scaling
    V qv[NK];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[kk][i] = M::from_f32(qf[kk][i] * qdown);

    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    // ---- staging of one tile: thread loads CPT 16-byte chunks
    auto load_tile = [&](int t0, U32x4 (&r)[CPT]) {
        const long long phys = p.page_table[t0 >> kPageShift];
        const char* base = p.pool + (phys * kPageTokens + (t0 & (kPageTokens - 1))) * W * 2;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int gi = c * 256 + threadIdx.x;
            if (gi < CHUNKS) {
                const int tok = gi / (W / 8);
                const int col = gi - tok * (W / 8);
                r[c] = (t0 + tok < t_end) ? load16(base + static_cast<long long>(tok) * W * 2 + col * 16)
                                          : U32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&](const U32x4 (&r)[CPT]) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int gi = c * 256 + threadIdx.x;
            if (gi < CHUNKS) {
                const int tok = gi / (W / 8);
                const int col = gi - tok * (W / 8);
                U32x4 v = r[c];
                if (SRC_BF16) {  // widen bf16 -> fp32 -> fp16 (exact inside the fp16 range)
                    uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const _Float16 lo = static_cast<_Float16>(__uint_as_float(w4[i] << 16));
                        const _Float16 hi = static_cast<_Float16>(__uint_as_float(w4[i] & 0xFFFF0000u));
                        w4[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
                                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
                    }
                    v = U32x4{w4[0], w4[1], w4[2], w4[3]};
                }
                *reinterpret_cast<U32x4*>(lds_rm + tok * RS + col * 16) = v;
                if (col * 8 < KL) {
                    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const uint16_t e = static_cast<uint16_t>(w4[i >> 1] >> ((i & 1) * 16));
                        *reinterpret_cast<uint16_t*>(lds_tr + (col * 8 + i) * TS + tok * 2) = e;
                    }
                }
            }
        }
    };

    const int ntiles = (t_end - t_begin + kTileTok - 1) / kTileTok;
    U32x4 stage[CPT];
    load_tile(t_begin, stage);
    for (int it = 0; it < ntiles; ++it) {
        const int t0 = t_begin + it * kTileTok;
        __syncthreads();  // previous tile's readers are done
        store_tile(stage);
        __syncthreads();
        if (it + 1 < ntiles) load_tile(t0 + kTileTok, stage);  // in flight during the MFMAs

        // QK: two 16-token M tiles
        f32x4_t sc[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            sc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            const char* row = lds_rm + (16 * mt + hl) * RS + 8 * q4 * 2;
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) {
                const V a = *reinterpret_cast<const V*>(row + 64 * kk);
                sc[mt] = M::mma(a, qv[kk], sc[mt]);
            }
        }
        // online softmax for head hl over this tile's 32 tokens
        float s[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = t0 + 16 * mt + 4 * q4 + r;
                const float v = tok < t_end ? sc[mt][r] * sscale : -INFINITY;
                s[4 * mt + r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        if (tmax > m) {
            const float corr = m == -INFINITY ? 0.f : fast_exp2(m - tmax);
            l *= corr;
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] *= corr;
            m = tmax;
        }
        const float mref = m == -INFINITY ? 0.f : m;
        V pb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float e = fast_exp2(s[i] - mref);
            l += e;
            pb[i] = M::from_f32(e);
        }
        // PV: one 32-token k step per 16-dim tile
        const char* col = lds_tr + hl * TS + 4 * q4 * 2;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const char* rp = col + 16 * t * TS;
            const uint2 lo = *reinterpret_cast<const uint2*>(rp);
            const uint2 hi = *reinterpret_cast<const uint2*>(rp + 32);
            V a;
            const uint32_t w4[4] = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                a[i] = __builtin_bit_cast(T, static_cast<uint16_t>(w4[i >> 1] >> ((i & 1) * 16)));
            acc[t] = M::mma(a, pb, acc[t]);
        }
    }

    // l: sum over the four lane quarters that share the head
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (head >= p.heads) return;
    if (p.splits == 1) {
        float* out = p.u + static_cast<size_t>(head) * KL;
        const float inv = 1.f / l;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 v = make_float4(acc[t][0] * inv, acc[t][1] * inv, acc[t][2] * inv, acc[t][3] * inv);
            *reinterpret_cast<float4*>(out + 16 * t + 4 * q4) = v;
        }
        return;
    }
    const size_t slot = static_cast<size_t>(head) * p.splits + split;
    float* out = p.part_u + slot * KL;
#pragma unroll
    for (int t = 0; t < NT; ++t)
        *reinterpret_cast<float4*>(out + 16 * t + 4 * q4) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    if (q4 == 0) p.part_ml[slot] = make_float2(m, l);
}

// Split merge for the MFMA path: one workgroup per (head, 128-dim block); a thread
// owns one float4 column and every 8th split, loading 8 partials at a time.
__global__ void __launch_bounds__(256) mla_combine_wide_kernel(const MlaMK p) {
    constexpr int KL = kMfmaLora;
    const int h = blockIdx.x;
    const int blk = blockIdx.y;             // 128-dim block
    const int c4 = threadIdx.x & 31;        // float4 column inside the block
    const int grp = threadIdx.x >> 5;       // 8 split groups
    const size_t base = static_cast<size_t>(h) * p.splits;
    const int d = blk * 128 + c4 * 4;
    float m = -INFINITY, l = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = grp; s0 < p.splits; s0 += 64) {
        float4 a[8];
        float2 ml[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int s = s0 + 8 * i;
            const bool in = s < p.splits;
            a[i] = in ? *reinterpret_cast<const float4*>(p.part_u + (base + s) * KL + d) : make_float4(0.f, 0.f, 0.f, 0.f);
            ml[i] = in ? p.part_ml[base + s] : make_float2(-INFINITY, 0.f);
        }
        float mb = m;
#pragma unroll
        for (int i = 0; i < 8; ++i) mb = fmaxf(mb, ml[i].x);
        const float cm = m == -INFINITY ? 0.f : fast_exp2(m - mb);
        l *= cm;
        o.x *= cm; o.y *= cm; o.z *= cm; o.w *= cm;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float c = ml[i].x == -INFINITY ? 0.f : fast_exp2(ml[i].x - mb);
            l = fmaf(ml[i].y, c, l);
            o.x = fmaf(a[i].x, c, o.x);
            o.y = fmaf(a[i].y, c, o.y);
            o.z = fmaf(a[i].z, c, o.z);
            o.w = fmaf(a[i].w, c, o.w);
        }
        m = mb;
    }
    __shared__ float rm[256], rl[256];
    __shared__ float4 ro[256];
    rm[threadIdx.x] = m;
    rl[threadIdx.x] = l;
    ro[threadIdx.x] = o;
    __syncthreads();
    if (threadIdx.x < 32) {
        float M = -INFINITY;
        for (int g = 0; g < 8; ++g) M = fmaxf(M, rm[g * 32 + threadIdx.x]);
        float L = 0.f;
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int g = 0; g < 8; ++g) {
            const int k = g * 32 + threadIdx.x;
            const float c = rm[k] == -INFINITY ? 0.f : fast_exp2(rm[k] - M);
            L = fmaf(rl[k], c, L);
            t.x = fmaf(ro[k].x, c, t.x);
            t.y = fmaf(ro[k].y, c, t.y);
            t.z = fmaf(ro[k].z, c, t.z);
            t.w = fmaf(ro[k].w, c, t.w);
        }
        *reinterpret_cast<float4*>(p.u + static_cast<size_t>(h) * KL + d) =
            make_float4(t.x / L, t.y / L, t.z / L, t.w / L);
    }
}

bool mfma_eligible(const MlaArgs& a) {
    return a.dtype != QR_DTYPE_F32 && a.kv_lora == kMfmaLora && (a.rope == 0 || a.rope == 64);
}

int cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            n = prop.multiProcessorCount;
        if (n <= 0) n = 256;
    }
    return n;
}

}  // namespace

MlaPlan plan_mla(const MlaArgs& a) {
    MlaPlan pl{};
    if (mfma_eligible(a)) {
        // about one workgroup per CU: (64-head group) x split, splits of whole 32-token tiles
        const int groups = (a.heads + kMfmaHeads - 1) / kMfmaHeads;
        const int tiles = (a.seq_len + kTileTok - 1) / kTileTok;
        int want = std::max(1, cus() / groups);
        want = std::min(want, tiles);
        const int tiles_per_split = (tiles + want - 1) / want;
        pl.split_tokens = tiles_per_split * kTileTok;
    } else {
        pl.split_tokens = kGenericSplit;
    }
    pl.splits = (a.seq_len + pl.split_tokens - 1) / pl.split_tokens;
    pl.workspace_bytes = pl.splits > 1
        ? static_cast<size_t>(a.heads) * pl.splits * (static_cast<size_t>(a.kv_lora) * 4 + 8)
        : 0;
    return pl;
}

namespace {
template <bool SRC_BF16, int KR>
hipError_t launch_mfma(const MlaMK& k, int groups, hipStream_t stream) {
    hipLaunchKernelGGL((mla_mfma_kernel<SRC_BF16, KR>), dim3(k.splits, groups), dim3(256), 0, stream, k);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_mla(const MlaArgs& a, const MlaPlan& pl, void* workspace, hipStream_t stream) {
    if (pl.splits > 4096) return hipErrorInvalidValue;
    const size_t slots = static_cast<size_t>(a.heads) * pl.splits;
    if (mfma_eligible(a)) {
        MlaMK k{};
        k.pool = static_cast<const char*>(a.pool);
        k.page_table = a.page_table;
        k.heads = a.heads;
        k.seq_len = a.seq_len;
        k.split_tokens = pl.split_tokens;
        k.splits = pl.splits;
        k.q_tilde = a.q_tilde;
        k.q_rope = a.q_rope;
        k.u = a.u;
        k.part_u = static_cast<float*>(workspace);
        k.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + slots * a.kv_lora * 4);
        k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
        const int groups = (a.heads + kMfmaHeads - 1) / kMfmaHeads;
        hipError_t e;
        const bool bf = a.dtype == QR_DTYPE_BF16;
        if (a.rope) e = bf ? launch_mfma<true, 64>(k, groups, stream) : launch_mfma<false, 64>(k, groups, stream);
        else e = bf ? launch_mfma<true, 0>(k, groups, stream) : launch_mfma<false, 0>(k, groups, stream);
        if (e != hipSuccess || pl.splits == 1) return e;
        hipLaunchKernelGGL(mla_combine_wide_kernel, dim3(a.heads, kMfmaLora / 128), dim3(256), 0, stream, k);
        return hipGetLastError();
    }
    MlaK k{};
    k.pool = static_cast<const char*>(a.pool);
    k.page_table = a.page_table;
    k.dtype = a.dtype;
    k.kv_lora = a.kv_lora;
    k.rope = a.rope;
    k.width = a.kv_lora + a.rope;
    k.heads = a.heads;
    k.seq_len = a.seq_len;
    k.split_tokens = pl.split_tokens;
    k.splits = pl.splits;
    k.q_tilde = a.q_tilde;
    k.q_rope = a.q_rope;
    k.u = a.u;
    k.part_u = static_cast<float*>(workspace);
    k.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + slots * a.kv_lora * 4);
    k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
    hipLaunchKernelGGL(mla_split_generic_kernel, dim3(pl.splits, a.heads), dim3(kThreads), 0, stream, k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.splits == 1) return e;
    hipLaunchKernelGGL(mla_combine_kernel, dim3(a.heads), dim3(kThreads), 0, stream, k);
    return hipGetLastError();
}

}  // namespace qr
