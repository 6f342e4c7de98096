// qr_chunk.hip -- causal multi-query attention over the paged cache on MFMA tiles
// (chunked prefill and speculative verify), gfx950.
//
// Semantics: query i of the chunk sits at position pos0+i and attends positions
// 0..pos0+i, which is what nq sequential PagedKvCache.Attention calls with
// interleaved appends compute (StreamingEngine.cs:831-836, SpeculativeRunner.cs:85-93).
//
// A row is one (query, query head) pair; the G = heads/kv_heads heads of one kv
// head and a block of consecutive queries form the rows of a workgroup, so every
// K/V tile staged in LDS serves them all.  Workgroup = 4 waves x NT x 16 rows.
// v_mfma_f32_16x16x32_f16 (lane layout verified on gfx950):
//   A[m = lane%16][k = 8*(lane/16)+i], B[k = 8*(lane/16)+i][n = lane%16],
//   D[m = 4*(lane/16)+r][n = lane%16].
//   QK: S^T[token][row] = K[token][dims] . Q^T[dims][row]      (M tokens, N rows)
//   PV: O^T[dim][row]  += V^T[dim][tokens] . P^T[tokens][row]   (M dims,   N rows)
// The 8 PV k-slots of lane quarter q are tokens {4q..4q+3, 16+4q..16+4q+3} of the
// 32-token tile: the 8 scores that lane already holds for its row after QK.  Each
// lane owns one row in both results, so the causal mask and the online-softmax
// rescale are lane-local.  K tiles are staged row-major; V tiles are copied from the
// dims-major V block of the page, which already is the V^T operand layout.
// Operands are fp16 (bf16 caches are widened to fp16 while staged, exact inside the
// fp16 range); accumulation and softmax are fp32.
#include "qr_chunk.hpp"

#include <algorithm>

namespace qr {
namespace {

constexpr int kTok = 32;  // tokens per tile

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mma16(f16x8_t a, f16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t widen_bf16_pair(uint32_t w) {
    const _Float16 lo = static_cast<_Float16>(__uint_as_float(w << 16));
    const _Float16 hi = static_cast<_Float16>(__uint_as_float(w & 0xFFFF0000u));
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

__device__ __forceinline__ float load_q(const void* q, int dtype, size_t i) {
    switch (dtype) {
        case QR_DTYPE_F32: return static_cast<const float*>(q)[i];
        case QR_DTYPE_F16: return f16_bits_to_f32(static_cast<const uint16_t*>(q)[i]);
        default: return bf16_bits_to_f32(static_cast<const uint16_t*>(q)[i]);
    }
}

struct ChunkK {
    const char* pool;
    const int* page_table;   // row of (sequence, layer)
    long long page_elems;
    long long plane_elems;
    int kv_heads;
    int heads;
    int group;
    int group_shift;         // log2(group)
    int pos0;
    int nq;
    int q_dtype;
    const void* q;           // [nq][heads][D]
    float* out;              // [nq][heads][D]
    float* part_acc;         // [nq*heads][splits][D]
    float2* part_ml;         // [nq*heads][splits]
    float qscale;            // scale * log2(e)
    int queries_per_block;
    int split_tokens;
    int splits;
};

template <bool SRC_BF16, int D, int NT>
__global__ void __launch_bounds__(256) chunk_mfma_kernel(const ChunkK p) {
    constexpr int NK = D / 32;             // QK k-steps
    constexpr int NDT = D / 16;            // PV dim tiles
    constexpr int RS = D * 2 + 16;         // K row stride in LDS (bytes), padded
    constexpr int TS = kTok * 2 + 16;      // V^T row stride in LDS (bytes), padded, 16-byte aligned
    constexpr int TILE_BYTES = kTok * D * 2;          // per plane
    constexpr int CPT = 2 * TILE_BYTES / 16 / 256;    // 16-byte chunks per thread (K then V)
    static_assert(CPT >= 1 && 2 * TILE_BYTES % (16 * 256) == 0, "tile must split evenly over 256 threads");

    __shared__ __attribute__((aligned(16))) char lds_k[2][kTok * RS];
    __shared__ __attribute__((aligned(16))) char lds_v[2][D * TS];

    const int split = blockIdx.x;
    const int qblk = blockIdx.y;
    const int kvh = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int q4 = lane >> 4;
    const int col = lane & 15;

    // rows of this lane, one per N tile
    const int q_first = qblk * p.queries_per_block;
    int row_q[NT], row_h[NT];
    bool row_on[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int rho = wave * 16 * NT + j * 16 + col;
        row_q[j] = q_first + (rho >> p.group_shift);
        row_h[j] = kvh * p.group + (rho & (p.group - 1));
        row_on[j] = row_q[j] < p.nq && (rho >> p.group_shift) < p.queries_per_block;
    }
    const int q_last = min(p.nq, q_first + p.queries_per_block) - 1;
    const int t_begin = split * p.split_tokens;
    const int t_end = min(t_begin + p.split_tokens, p.pos0 + q_last + 1);  // causal bound of the block

    // Q^T operands (fp16), rows beyond the chunk read row 0 and are never written
    f16x8_t qv[NT][NK];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const size_t qrow = (static_cast<size_t>(row_on[j] ? row_q[j] : 0) * p.heads + row_h[j]) * D;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                qv[j][kk][i] = static_cast<_Float16>(load_q(p.q, p.q_dtype, qrow + 32 * kk + 8 * q4 + i));
    }

    f32x4_t acc[NT][NDT];
    float m[NT], l[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.f;
#pragma unroll
        for (int t = 0; t < NDT; ++t) acc[j][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    const long long head_off = static_cast<long long>(kvh) * kPageTokens * D;
    // K rows are token-major; the V block of the page is dims-major ([dim][256 positions]),
    // so a tile's V^T is D rows of 64 contiguous bytes
    auto load_tile = [&](int t0, U32x4 (&r)[CPT]) {
        const long long phys = p.page_table[t0 >> kPageShift];
        const int slot0 = t0 & (kPageTokens - 1);
        const char* kb = p.pool + (phys * p.page_elems + head_off + static_cast<long long>(slot0) * D) * 2;
        const char* vb = p.pool + (phys * p.page_elems + p.plane_elems + head_off + slot0) * 2;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int gi = c * 256 + threadIdx.x;          // chunk index over K then V
            const int plane = gi / (TILE_BYTES / 16);
            const int ci = gi - plane * (TILE_BYTES / 16);
            r[c] = plane ? load16(vb + ((ci >> 2) * kPageTokens + 8 * (ci & 3)) * 2) : load16(kb + ci * 16);
        }
    };
    auto store_tile = [&](const U32x4 (&r)[CPT], int buf, int t0) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int gi = c * 256 + threadIdx.x;
            const int plane = gi / (TILE_BYTES / 16);
            const int ci = gi - plane * (TILE_BYTES / 16);
            U32x4 v = r[c];
            if (SRC_BF16) v = U32x4{widen_bf16_pair(v.x), widen_bf16_pair(v.y), widen_bf16_pair(v.z), widen_bf16_pair(v.w)};
            if (plane == 0) {
                const int tok = ci / (D / 8);
                *reinterpret_cast<U32x4*>(lds_k[buf] + tok * RS + (ci - tok * (D / 8)) * 16) = v;
            } else {
                // dim ci/4, positions t0 + 8(ci%4) .. +7; positions past t_end may hold stale
                // rows and are zeroed so that a zero weight cannot meet a NaN
                const int first = t0 + 8 * (ci & 3);
                if (first + 8 > t_end) {
                    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (first + i >= t_end) w[i >> 1] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                    v = U32x4{w[0], w[1], w[2], w[3]};
                }
                *reinterpret_cast<U32x4*>(lds_v[buf] + (ci >> 2) * TS + 16 * (ci & 3)) = v;
            }
        }
    };

    const int ntiles = t_end > t_begin ? (t_end - t_begin + kTok - 1) / kTok : 0;
    U32x4 stage[CPT];
    if (ntiles > 0) {
        load_tile(t_begin, stage);
        store_tile(stage, 0, t_begin);
    }
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int buf = it & 1;
        const int t0 = t_begin + it * kTok;
        if (it + 1 < ntiles) load_tile(t0 + kTok, stage);  // in flight during the MFMAs

        // QK
        f32x4_t sc[NT][2];
#pragma unroll
        for (int j = 0; j < NT; ++j) sc[j][0] = sc[j][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const char* row = lds_k[buf] + (16 * mt + col) * RS + 16 * q4;
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) {
                const f16x8_t a = *reinterpret_cast<const f16x8_t*>(row + 64 * kk);
#pragma unroll
                for (int j = 0; j < NT; ++j) sc[j][mt] = mma16(a, qv[j][kk], sc[j][mt]);
            }
        }
        // causal mask + online softmax, one row per lane and N tile
        f16x8_t pb[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int qpos = p.pos0 + row_q[j];
            float s[8];
            float tmax = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = t0 + 16 * mt + 4 * q4 + r;
                    const float v = (tok < t_end && tok <= qpos) ? sc[j][mt][r] * p.qscale : -INFINITY;
                    s[4 * mt + r] = v;
                    tmax = fmaxf(tmax, v);
                }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            if (tmax > m[j]) {
                const float corr = m[j] == -INFINITY ? 0.f : fast_exp2(m[j] - tmax);
                l[j] *= corr;
#pragma unroll
                for (int t = 0; t < NDT; ++t) acc[j][t] *= corr;
                m[j] = tmax;
            }
            const float mref = m[j] == -INFINITY ? 0.f : m[j];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float e = fast_exp2(s[i] - mref);
                l[j] += e;
                pb[j][i] = static_cast<_Float16>(e);
            }
        }
        // PV
        const char* vcol = lds_v[buf] + col * TS + 8 * q4;
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
            const char* rp = vcol + 16 * t * TS;
            const uint2 lo = *reinterpret_cast<const uint2*>(rp);
            const uint2 hi = *reinterpret_cast<const uint2*>(rp + 32);
            const uint32_t w4[4] = {lo.x, lo.y, hi.x, hi.y};
            f16x8_t a;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                a[i] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(w4[i >> 1] >> ((i & 1) * 16)));
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[j][t] = mma16(a, pb[j], acc[j][t]);
        }
        if (it + 1 < ntiles) store_tile(stage, buf ^ 1, t0 + kTok);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < NT; ++j) {
        l[j] += __shfl_xor(l[j], 16);
        l[j] += __shfl_xor(l[j], 32);
        if (!row_on[j]) continue;
        const size_t r = static_cast<size_t>(row_q[j]) * p.heads + row_h[j];
        if (p.splits == 1) {
            float* o = p.out + r * D;
            const float inv = 1.f / l[j];
#pragma unroll
            for (int t = 0; t < NDT; ++t)
                *reinterpret_cast<float4*>(o + 16 * t + 4 * q4) =
                    make_float4(acc[j][t][0] * inv, acc[j][t][1] * inv, acc[j][t][2] * inv, acc[j][t][3] * inv);
        } else {
            const size_t slot = r * p.splits + split;
            float* o = p.part_acc + slot * D;
#pragma unroll
            for (int t = 0; t < NDT; ++t)
                *reinterpret_cast<float4*>(o + 16 * t + 4 * q4) =
                    make_float4(acc[j][t][0], acc[j][t][1], acc[j][t][2], acc[j][t][3]);
            if (q4 == 0) p.part_ml[slot] = make_float2(m[j], l[j]);
        }
    }
}

// Merge of the splits: one wave per (query, head) row.  Splits past the query's
// causal bound hold m = -inf and weigh zero.
template <int D>
__global__ void __launch_bounds__(64) chunk_combine_kernel(const ChunkK p) {
    const size_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const size_t base = r * p.splits;
    float mx = -INFINITY;
#pragma unroll 8
    for (int s = 0; s < p.splits; ++s) mx = fmaxf(mx, p.part_ml[base + s].x);
    float L = 0.f;
    float o[D / 64];
#pragma unroll
    for (int i = 0; i < D / 64; ++i) o[i] = 0.f;
#pragma unroll 8
    for (int s = 0; s < p.splits; ++s) {
        const float2 ml = p.part_ml[base + s];
        const float c = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - mx);
        L = fmaf(ml.y, c, L);
#pragma unroll
        for (int i = 0; i < D / 64; ++i) o[i] = fmaf(p.part_acc[(base + s) * D + lane + 64 * i], c, o[i]);
    }
#pragma unroll
    for (int i = 0; i < D / 64; ++i) p.out[r * D + lane + 64 * i] = o[i] / L;
}

int cu_total() {
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

template <bool BF, int D>
hipError_t launch_nt(const ChunkK& k, int nt, dim3 grid, hipStream_t s) {
    switch (nt) {
        case 1: hipLaunchKernelGGL((chunk_mfma_kernel<BF, D, 1>), grid, dim3(256), 0, s, k); break;
        case 2: hipLaunchKernelGGL((chunk_mfma_kernel<BF, D, 2>), grid, dim3(256), 0, s, k); break;
        default: hipLaunchKernelGGL((chunk_mfma_kernel<BF, D, 4>), grid, dim3(256), 0, s, k); break;
    }
    return hipGetLastError();
}

}  // namespace

bool chunk_mfma_eligible(int kv_dtype, int head_dim, int heads, int kv_heads) {
    if (kv_dtype == QR_DTYPE_F32 || (head_dim != 64 && head_dim != 128) || heads % kv_heads) return false;
    const int g = heads / kv_heads;
    return g <= 64 && (g & (g - 1)) == 0;
}

ChunkPlan plan_chunk(const ChunkArgs& a) {
    ChunkPlan pl{};
    const int g = a.heads / a.geom.kv_heads;
    const int total = a.pos0 + a.nq;  // tokens attended by the last query
    // rows per workgroup: up to 256 (4 queries' worth of heads per wave and N tile)
    int nt = 4;
    while (nt > 1 && (64 * nt) / g > std::max(1, a.nq)) nt >>= 1;
    pl.nt = nt;
    pl.queries_per_block = std::max(1, 64 * nt / g);
    const int qblocks = (a.nq + pl.queries_per_block - 1) / pl.queries_per_block;
    const int units = qblocks * a.geom.kv_heads;
    // split the keys when there are too few (query block, kv head) units to fill the GPU
    int splits = 1;
    if (units < cu_total()) splits = std::min((cu_total() + units - 1) / units, (total + kTok - 1) / kTok);
    int split_tokens = ((total + splits - 1) / splits + kTok - 1) / kTok * kTok;
    splits = (total + split_tokens - 1) / split_tokens;
    pl.splits = splits;
    pl.split_tokens = split_tokens;
    pl.qblocks = qblocks;
    pl.workspace_bytes = splits > 1
        ? static_cast<size_t>(a.nq) * a.heads * splits * (static_cast<size_t>(a.geom.head_dim) * 4 + 8)
        : 0;
    return pl;
}

hipError_t launch_chunk(const ChunkArgs& a, const ChunkPlan& pl, void* workspace, hipStream_t stream,
                        hipEvent_t after_split) {
    ChunkK k{};
    k.pool = static_cast<const char*>(a.pool);
    k.page_table = a.page_table;
    k.page_elems = a.geom.page_elems();
    k.plane_elems = a.geom.plane_elems();
    k.kv_heads = a.geom.kv_heads;
    k.heads = a.heads;
    k.group = a.heads / a.geom.kv_heads;
    int gs = 0;
    while ((1 << gs) < k.group) ++gs;
    k.group_shift = gs;
    k.pos0 = a.pos0;
    k.nq = a.nq;
    k.q_dtype = a.q_dtype;
    k.q = a.q;
    k.out = a.out;
    const size_t rows = static_cast<size_t>(a.nq) * a.heads;
    k.part_acc = static_cast<float*>(workspace);
    k.part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + rows * pl.splits * a.geom.head_dim * 4);
    k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
    k.queries_per_block = pl.queries_per_block;
    k.split_tokens = pl.split_tokens;
    k.splits = pl.splits;
    const dim3 grid(pl.splits, pl.qblocks, a.geom.kv_heads);
    const bool bf = a.kv_dtype == QR_DTYPE_BF16;
    hipError_t e;
    if (a.geom.head_dim == 128) e = bf ? launch_nt<true, 128>(k, pl.nt, grid, stream) : launch_nt<false, 128>(k, pl.nt, grid, stream);
    else e = bf ? launch_nt<true, 64>(k, pl.nt, grid, stream) : launch_nt<false, 64>(k, pl.nt, grid, stream);
    if (e != hipSuccess) return e;
    if (after_split && (e = hipEventRecord(after_split, stream)) != hipSuccess) return e;
    if (pl.splits == 1) return hipSuccess;
    if (a.geom.head_dim == 128) hipLaunchKernelGGL((chunk_combine_kernel<128>), dim3(rows), dim3(64), 0, stream, k);
    else hipLaunchKernelGGL((chunk_combine_kernel<64>), dim3(rows), dim3(64), 0, stream, k);
    return hipGetLastError();
}

}  // namespace qr
