// qr_decode.hip -- split-K (flash-decoding) GQA decode attention for gfx950.
//
// Replaces the two-pass, fully materialised PagedKvCache.Attention
// (PagedKvCache.cs:83-136) with:
//   decode_split_kernel   one workgroup per (entry, kv head [x head chunk], split of
//                         split_tokens positions).  K/V rows of the split are read
//                         from HBM once and shared by every query head of the group.
//   decode_combine_kernel log-sum-exp merge of the per-split partials.
//
// Lane layout (wave64): a token row of head_dim elements is spread over
// LPT = head_dim/16 consecutive lanes, 16 elements per lane, taken as 16-byte
// chunks c = sub + LPT*j (sub = lane % LPT).  One load instruction of a wave
// therefore reads LPT*16 contiguous bytes from each of 64/LPT consecutive rows;
// rows of one (page, kv head) are contiguous, so a wave reads one contiguous run.
// Per-token dot products are finished with DPP butterflies inside the LPT lanes.
//
// Softmax: each token group (the LPT lanes that share a token stream) keeps
// its T scores per head in registers, takes their max, exponentiates relative
// to it and accumulates p*V.  Token groups, waves and splits are then merged
// with the log-sum-exp rule, so no accumulator is rescaled inside the stream.
// Scores are kept in log2 units: q is pre-multiplied by scale*log2(e) and
// exponentials use v_exp_f32 (exp2).
#include "qr_kernels.hpp"

#include <algorithm>
#include <cmath>

namespace qr {
namespace {

constexpr int kWaves = 4;            // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kTokensPerGroup = 8;   // T: tokens each token group handles per split
constexpr int kMaxCombineSplits = 4096;

struct DecodeK {
    const char* pool;
    const int* page_table;
    long long page_elems;
    long long plane_elems;
    int head_dim;
    int lpt_shift;       // log2(head_dim / 16)
    int kv_heads;
    int heads;
    int group;           // heads / kv_heads (uniform GQA)
    int head_chunks;     // ceil(group / GMAX)
    int per_head;        // 1: one query head per workgroup (kv_heads does not divide heads)
    const float* q;
    float* out;
    float* part_acc;     // [nb][heads][max_splits][head_dim]
    float2* part_ml;     // [nb][heads][max_splits] (max in log2 units, sum)
    float qscale;        // scale * log2(e)
    int split_tokens;
    int max_splits;
    int seq_len[kMaxDecodeBatch];
    int pt_off[kMaxDecodeBatch];
};

__device__ __forceinline__ float exp2_or_zero(float x_minus_m, float m) {
    return m == -INFINITY ? 0.f : fast_exp2(x_minus_m);
}

template <typename KT, int GMAX, int T>
__global__ void __launch_bounds__(kThreads) decode_split_kernel(const DecodeK p) {
    using C = Chunk<KT>;
    constexpr int EPC = C::kElems;  // elements per 16-byte chunk
    constexpr int NC = 16 / EPC;    // chunks per lane
    constexpr int ESZ = 16 / EPC;   // bytes per element

    const int split = blockIdx.x;
    const int unit = blockIdx.y;
    const int b = blockIdx.z;
    const int seq = p.seq_len[b];
    const int t_begin = split * p.split_tokens;
    if (t_begin >= seq) return;
    const int t_end = min(seq, t_begin + p.split_tokens);

    const int D = p.head_dim;
    const int lsh = p.lpt_shift;
    const int LPT = 1 << lsh;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane & (LPT - 1);
    const int tpw = 64 >> lsh;
    const int ntg = kWaves * tpw;
    const int tg = wave * tpw + (lane >> lsh);

    int kvh, h0, G;
    if (p.per_head) {
        h0 = unit;
        kvh = static_cast<int>(static_cast<long long>(unit) * p.kv_heads / p.heads);
        G = 1;
    } else {
        const int c = unit % p.head_chunks;
        kvh = unit / p.head_chunks;
        h0 = kvh * p.group + c * GMAX;
        G = min(GMAX, p.group - c * GMAX);
    }

    // ---- query slice of this lane, pre-scaled into log2 units
    float q[GMAX][16];
    const float* qb = p.q + static_cast<size_t>(b) * p.heads * D;
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
#pragma unroll
        for (int j = 0; j < NC; ++j)
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
                const int dim = (sub + LPT * j) * EPC + e;
                q[g][j * EPC + e] = (g < G) ? qb[static_cast<size_t>(h0 + g) * D + dim] * p.qscale : 0.f;
            }

    const int* pt = p.page_table + p.pt_off[b];
    const long long head_off = static_cast<long long>(kvh) * kPageTokens * D;

    // ---- scores of this token group's T positions
    float s[T][GMAX];
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int t = t_begin + tg + i * ntg;
        const bool valid = t < t_end;
        const int tc = valid ? t : t_end - 1;
        const long long phys = pt[tc >> kPageShift];
        const char* row = p.pool + (phys * p.page_elems + head_off +
                                    static_cast<long long>(tc & (kPageTokens - 1)) * D) * ESZ;
        float k[16];
#pragma unroll
        for (int j = 0; j < NC; ++j) C::widen(load16(row + (sub + LPT * j) * 16), &k[j * EPC]);
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) d = fmaf(q[g][e], k[e], d);
            d = group_sum(d, LPT);
            s[i][g] = valid ? d : -INFINITY;
        }
    }

    // ---- local softmax numerators
    float m[GMAX], l[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        m[g] = s[0][g];
#pragma unroll
        for (int i = 1; i < T; ++i) m[g] = fmaxf(m[g], s[i][g]);
        const float mref = (m[g] == -INFINITY) ? 0.f : m[g];
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < T; ++i) {
            s[i][g] = fast_exp2(s[i][g] - mref);
            l[g] += s[i][g];
        }
    }

    // ---- p . V
    float acc[GMAX][16];
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[g][e] = 0.f;
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int t = t_begin + tg + i * ntg;
        const int tc = t < t_end ? t : t_end - 1;
        const long long phys = pt[tc >> kPageShift];
        const char* row = p.pool + (phys * p.page_elems + p.plane_elems + head_off +
                                    static_cast<long long>(tc & (kPageTokens - 1)) * D) * ESZ;
        float v[16];
#pragma unroll
        for (int j = 0; j < NC; ++j) C::widen(load16(row + (sub + LPT * j) * 16), &v[j * EPC]);
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[g][e] = fmaf(s[i][g], v[e], acc[g][e]);
    }

    // ---- merge the token groups of this wave (lanes with equal `sub`)
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            const float m2 = __shfl_xor(m[g], off);
            const float l2 = __shfl_xor(l[g], off);
            const float M = fmaxf(m[g], m2);
            const float c1 = exp2_or_zero(m[g] - M, m[g]);
            const float c2 = exp2_or_zero(m2 - M, m2);
            l[g] = l[g] * c1 + l2 * c2;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[g][e] = acc[g][e] * c1 + __shfl_xor(acc[g][e], off) * c2;
            m[g] = M;
        }
    }

    // ---- merge the waves through LDS and write the split's partial
    __shared__ float sm_acc[kWaves][GMAX][256];
    __shared__ float sm_m[kWaves][GMAX];
    __shared__ float sm_l[kWaves][GMAX];
    if ((lane >> lsh) == 0) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
#pragma unroll
            for (int j = 0; j < NC; ++j)
#pragma unroll
                for (int e = 0; e < EPC; ++e) sm_acc[wave][g][(sub + LPT * j) * EPC + e] = acc[g][j * EPC + e];
            if (sub == 0) {
                sm_m[wave][g] = m[g];
                sm_l[wave][g] = l[g];
            }
        }
    }
    __syncthreads();

    const bool single = (t_begin == 0 && t_end == seq);
    for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
        const int g = idx / D;
        const int d = idx - g * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][g]);
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float c = exp2_or_zero(sm_m[w][g] - M, sm_m[w][g]);
            L += sm_l[w][g] * c;
            o += sm_acc[w][g][d] * c;
        }
        const int h = h0 + g;
        if (single) {
            p.out[(static_cast<size_t>(b) * p.heads + h) * D + d] = o / L;
        } else {
            const size_t slot = (static_cast<size_t>(b) * p.heads + h) * p.max_splits + split;
            p.part_acc[slot * D + d] = o;
            if (d == 0) p.part_ml[slot] = make_float2(M, L);
        }
    }
}

// One workgroup per (head, entry).  Weights of the splits go through LDS, then
// head_dim/4 lanes x (256*4/head_dim) split groups read the partials as float4.
__global__ void __launch_bounds__(kThreads) decode_combine_kernel(const DecodeK p) {
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int seq = p.seq_len[b];
    const int nsplit = (seq + p.split_tokens - 1) / p.split_tokens;
    if (nsplit <= 1) return;
    const int D = p.head_dim;
    const size_t base = (static_cast<size_t>(b) * p.heads + h) * p.max_splits;

    __shared__ float w[kMaxCombineSplits];
    __shared__ float red[kThreads];
    __shared__ float4 red4[kThreads];

    // global max of the split maxima
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < nsplit; s += kThreads) {
        const float ms = p.part_ml[base + s].x;
        w[s] = ms;
        mx = fmaxf(mx, ms);
    }
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();

    // split weights and the total denominator
    float lsum = 0.f;
    for (int s = threadIdx.x; s < nsplit; s += kThreads) {
        const float c = exp2_or_zero(w[s] - M, w[s]);
        w[s] = c;
        lsum += p.part_ml[base + s].y * c;
    }
    red[threadIdx.x] = lsum;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float L = red[0];

    // weighted sum of the partial accumulators
    const int d4n = D >> 2;
    const int groups = kThreads / d4n;
    const int d4 = threadIdx.x % d4n;
    const int grp = threadIdx.x / d4n;
    float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4* acc4 = reinterpret_cast<const float4*>(p.part_acc + base * D);
#pragma unroll 8
    for (int s = grp; s < nsplit; s += groups) {
        const float4 a = acc4[static_cast<size_t>(s) * d4n + d4];
        const float c = w[s];
        o4.x = fmaf(a.x, c, o4.x);
        o4.y = fmaf(a.y, c, o4.y);
        o4.z = fmaf(a.z, c, o4.z);
        o4.w = fmaf(a.w, c, o4.w);
    }
    red4[threadIdx.x] = o4;
    __syncthreads();
    if (threadIdx.x < d4n) {
        float4 t = red4[threadIdx.x];
        for (int gi = 1; gi < groups; ++gi) {
            const float4 u = red4[gi * d4n + threadIdx.x];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        float* out = p.out + (static_cast<size_t>(b) * p.heads + h) * D + threadIdx.x * 4;
        out[0] = t.x / L;
        out[1] = t.y / L;
        out[2] = t.z / L;
        out[3] = t.w / L;
    }
}

int pick_gmax(int group) {
    if (group <= 1) return 1;
    if (group <= 2) return 2;
    if (group <= 4) return 4;
    return 8;
}

template <typename KT, int GMAX>
hipError_t launch_split(const DecodeK& k, dim3 grid, hipStream_t stream) {
    hipLaunchKernelGGL((decode_split_kernel<KT, GMAX, kTokensPerGroup>), grid, dim3(kThreads), 0,
                       stream, k);
    return hipGetLastError();
}

template <typename KT>
hipError_t dispatch_gmax(int gmax, const DecodeK& k, dim3 grid, hipStream_t stream) {
    switch (gmax) {
        case 1: return launch_split<KT, 1>(k, grid, stream);
        case 2: return launch_split<KT, 2>(k, grid, stream);
        case 4: return launch_split<KT, 4>(k, grid, stream);
        default: return launch_split<KT, 8>(k, grid, stream);
    }
}

int log2_exact(int v) {
    int s = 0;
    while ((1 << s) < v) ++s;
    return s;
}

}  // namespace

DecodePlan plan_decode(const DecodeArgs& a) {
    DecodePlan pl{};
    const int D = a.geom.head_dim;
    const int lpt = D / 16;
    const int ntg = kWaves * (64 / lpt);
    pl.split_tokens = kTokensPerGroup * ntg;
    int max_len = 0;
    for (int i = 0; i < a.nb; ++i) max_len = std::max(max_len, a.seq_len[i]);
    pl.max_splits = std::max(1, (max_len + pl.split_tokens - 1) / pl.split_tokens);
    const int kvh = a.geom.kv_heads;
    if (a.heads % kvh == 0) {
        const int group = a.heads / kvh;
        const int gmax = pick_gmax(group);
        pl.units = kvh * ((group + gmax - 1) / gmax);
    } else {
        pl.units = a.heads;
    }
    pl.workspace_bytes = pl.max_splits > 1
        ? static_cast<size_t>(a.nb) * a.heads * pl.max_splits * (static_cast<size_t>(D) * 4 + 8)
        : 0;
    return pl;
}

hipError_t launch_decode(const DecodeArgs& a, const DecodePlan& pl, void* workspace,
                         hipStream_t stream) {
    DecodeK k{};
    k.pool = static_cast<const char*>(a.pool);
    k.page_table = a.page_table;
    k.page_elems = a.geom.page_elems();
    k.plane_elems = a.geom.plane_elems();
    k.head_dim = a.geom.head_dim;
    k.lpt_shift = log2_exact(a.geom.head_dim / 16);
    k.kv_heads = a.geom.kv_heads;
    k.heads = a.heads;
    int gmax = 1;
    if (a.heads % a.geom.kv_heads == 0) {
        k.group = a.heads / a.geom.kv_heads;
        gmax = pick_gmax(k.group);
        k.head_chunks = (k.group + gmax - 1) / gmax;
        k.per_head = 0;
    } else {
        k.group = 1;
        k.head_chunks = 1;
        k.per_head = 1;
    }
    k.q = a.q;
    k.out = a.out;
    const size_t slots = static_cast<size_t>(a.nb) * a.heads * pl.max_splits;
    k.part_acc = static_cast<float*>(workspace);
    k.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + slots * a.geom.head_dim * 4);
    k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
    k.split_tokens = pl.split_tokens;
    k.max_splits = pl.max_splits;
    for (int i = 0; i < a.nb; ++i) {
        k.seq_len[i] = a.seq_len[i];
        k.pt_off[i] = a.pt_off[i];
    }
    if (pl.max_splits > kMaxCombineSplits) return hipErrorInvalidValue;

    const dim3 grid(pl.max_splits, pl.units, a.nb);
    hipError_t e;
    switch (a.dtype) {
        case QR_DTYPE_F32: e = dispatch_gmax<float>(gmax, k, grid, stream); break;
        case QR_DTYPE_F16: e = dispatch_gmax<F16Tag>(gmax, k, grid, stream); break;
        default: e = dispatch_gmax<BF16Tag>(gmax, k, grid, stream); break;
    }
    if (e != hipSuccess || pl.max_splits == 1) return e;
    hipLaunchKernelGGL(decode_combine_kernel, dim3(a.heads, a.nb), dim3(kThreads), 0, stream, k);
    return hipGetLastError();
}

}  // namespace qr
