// qr_append.hip -- in-place row append into HBM pages, and the debug copy-out.
//
// Append replaces PagedKvCache.Append / MlaLatentCache.Append
// (PagedKvCache.cs:62-69, MlaLatentCache.cs:45-51): a token row of
// kv_heads*head_dim elements is scattered into its page, one contiguous
// head_dim run per kv head, converted to the cache dtype on the way.
#include "qr_kernels.hpp"

namespace qr {
namespace {

__device__ __forceinline__ float load_f32(const void* src, int dtype, long long i) {
    switch (dtype) {
        case QR_DTYPE_F32: return static_cast<const float*>(src)[i];
        case QR_DTYPE_F16: return f16_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
        default: return bf16_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
    }
}

// Converts element i of src (src_dtype) into slot j of dst (dst_dtype).  A
// 16-bit value copied into a cache of the same type keeps its exact bits.
__device__ __forceinline__ void convert_store(void* dst, int dst_dtype, long long j, const void* src,
                                              int src_dtype, long long i) {
    if (dst_dtype != QR_DTYPE_F32 && src_dtype == dst_dtype) {
        static_cast<uint16_t*>(dst)[j] = static_cast<const uint16_t*>(src)[i];
        return;
    }
    const float x = load_f32(src, src_dtype, i);
    switch (dst_dtype) {
        case QR_DTYPE_F32: static_cast<float*>(dst)[j] = x; break;
        case QR_DTYPE_F16: static_cast<uint16_t*>(dst)[j] = f32_to_f16_bits_ref(x); break;
        default: static_cast<uint16_t*>(dst)[j] = f32_to_bf16_bits_ref(x); break;
    }
}

__device__ __forceinline__ long long page_offset(const PageGeom& g, long long phys, int plane,
                                                 int slot, int col) {
    const int kvh = col / g.head_dim;
    return g.offset(phys, plane, kvh, slot, col - kvh * g.head_dim);
}

__global__ void __launch_bounds__(256) append_kernel(const AppendArgs a) {
    int pos0 = a.pos0;
    if (a.pos_dev) {  // device-side position: written only where the pages of all rows were claimed
        pos0 = *a.pos_dev;
        if (pos0 < 0 || pos0 > a.max_seq - a.n || ((pos0 + a.n - 1) >> kPageShift) >= *a.held_dev) return;
    }
    const int width = a.geom.kv_heads * a.geom.head_dim;
    const long long per_plane = static_cast<long long>(a.n) * width;
    const long long total = per_plane * a.geom.planes;
    for (long long idx = blockIdx.x * 256LL + threadIdx.x; idx < total;
         idx += static_cast<long long>(gridDim.x) * 256) {
        const int plane = static_cast<int>(idx / per_plane);
        const long long rem = idx - plane * per_plane;
        const int r = static_cast<int>(rem / width);
        const int col = static_cast<int>(rem - static_cast<long long>(r) * width);
        if (col >= a.row_len[plane]) continue;
        const int t = pos0 + r;
        const long long phys = a.page_table[t >> kPageShift];
        convert_store(a.pool, a.dtype, page_offset(a.geom, phys, plane, t & (kPageTokens - 1), col),
                      a.src[plane], a.src_dtype, static_cast<long long>(r) * a.src_stride + col);
    }
}

__global__ void __launch_bounds__(256) gather_kernel(const GatherArgs a) {
    const int width = a.geom.kv_heads * a.geom.head_dim;
    const long long per_plane = static_cast<long long>(a.n) * width;
    const long long total = per_plane * a.geom.planes;
    const int esz = dtype_size(a.dtype);
    for (long long idx = blockIdx.x * 256LL + threadIdx.x; idx < total;
         idx += static_cast<long long>(gridDim.x) * 256) {
        const int plane = static_cast<int>(idx / per_plane);
        const long long rem = idx - plane * per_plane;
        const int r = static_cast<int>(rem / width);
        const int col = static_cast<int>(rem - static_cast<long long>(r) * width);
        const int t = a.pos0 + r;
        const long long phys = a.page_table[t >> kPageShift];
        const long long off = page_offset(a.geom, phys, plane, t & (kPageTokens - 1), col);
        if (a.to_f32) {
            static_cast<float*>(a.dst[plane])[rem] = load_f32(a.pool, a.dtype, off);
        } else if (esz == 4) {
            static_cast<float*>(a.dst[plane])[rem] = static_cast<const float*>(a.pool)[off];
        } else {
            static_cast<uint16_t*>(a.dst[plane])[rem] = static_cast<const uint16_t*>(a.pool)[off];
        }
    }
}

// Workgroup = kRopeRows positions.  The cos/sin of (position, i) for i < head_dim/2 are
// computed once into LDS; then every thread takes 4 consecutive dim pairs (d..d+3,
// d+D/2..d+D/2+3) of one head: K heads are rotated and stored in the cache dtype with
// the same dims of V, q heads are rotated in place.  Products and sums are separately
// rounded as in the reference (x0 c - x1 s, x0 s + x1 c).
constexpr int kRopeRows = 1;
constexpr int kVTileTpt = 8;       // V tile: tokens per thread (one 16-byte chunk per dim)

// 4 consecutive dims of one cache row (d a multiple of 4): one 16- or 8-byte store when
// they are contiguous (token-major planes and MFMA-layout K), element stores for an
// MFMA-layout V plane.
__device__ __forceinline__ void store4(void* pool, int dtype, const PageGeom& g, long long phys, int plane, int kvh,
                                       int slot, int d, const float (&x)[4]) {
    const bool rows = !(plane == 1 && g.mfma_layout);
    if (dtype == QR_DTYPE_F32 && rows) {
        *reinterpret_cast<float4*>(static_cast<float*>(pool) + g.offset(phys, plane, kvh, slot, d)) =
            make_float4(x[0], x[1], x[2], x[3]);
        return;
    }
    uint16_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) b[e] = dtype == QR_DTYPE_F16 ? f32_to_f16_bits_ref(x[e]) : f32_to_bf16_bits_ref(x[e]);
    uint16_t* base = static_cast<uint16_t*>(pool);
    if (rows) {
        *reinterpret_cast<uint2*>(base + g.offset(phys, plane, kvh, slot, d)) =
            make_uint2(b[0] | (static_cast<uint32_t>(b[1]) << 16), b[2] | (static_cast<uint32_t>(b[3]) << 16));
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) base[g.offset(phys, plane, kvh, slot, d + e)] = b[e];
}

// An MFMA-layout V plane keeps 8 aligned consecutive tokens of one dim contiguous, so a
// position's V row lands as scattered 2-byte stores.  V tiles write it instead: a
// workgroup owns an aligned run of T tokens of one kv head (T divides kPageTokens, so
// the run lies in one page), each thread 2 dims x TPT consecutive tokens, and a chunk of
// 8 tokens of one dim is one 16-byte store.  Source rows outside [pos0, pos0 + n) are
// clamped loads whose values are never stored; chunks at the ends of the range store
// only their in-range tokens.
__host__ __device__ constexpr int v_tile_tokens(int head_dim, int tpt) { return 2 * kRopeThreads / head_dim * tpt; }

template <int TPT>
__device__ __forceinline__ void v_tile_store(const AppendArgs& g, int pos0, int vb) {
    static_assert(TPT == 8, "one 16-byte chunk (8 aligned tokens of one dim) per thread and dim");
    const int D = g.geom.head_dim;
    const int pairs = D >> 1;  // 32 or 64
    const int T = v_tile_tokens(D, TPT);
    const int kvh = vb % g.geom.kv_heads;
    const int tbase = (pos0 / T + vb / g.geom.kv_heads) * T;
    if (tbase >= pos0 + g.n) return;  // a tile past the rows (device positions launch the most tiles n rows can span)
    const int dp = threadIdx.x & (pairs - 1);
    const int t0 = tbase + (threadIdx.x / pairs) * TPT;
    const float* src = static_cast<const float*>(g.src[1]) + kvh * D + 2 * dp;
    float2 v[TPT];
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
        const int r = min(max(t0 + k - pos0, 0), g.n - 1);
        v[k] = *reinterpret_cast<const float2*>(src + static_cast<long long>(r) * g.src_stride);
    }
    const long long phys = g.page_table[tbase >> kPageShift];
    const int slot0 = t0 & (kPageTokens - 1);
    const bool whole = t0 >= pos0 && t0 + TPT <= pos0 + g.n;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        uint16_t b[TPT];
#pragma unroll
        for (int k = 0; k < TPT; ++k) {
            const float x = e ? v[k].y : v[k].x;
            b[k] = g.dtype == QR_DTYPE_F16 ? f32_to_f16_bits_ref(x) : f32_to_bf16_bits_ref(x);
        }
        uint16_t* p = static_cast<uint16_t*>(g.pool) + g.geom.offset(phys, 1, kvh, slot0, 2 * dp + e);
        if (whole) {
#pragma unroll
            for (int c = 0; c < TPT / 8; ++c) {
                uint32_t w[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) w[j] = b[8 * c + 2 * j] | (static_cast<uint32_t>(b[8 * c + 2 * j + 1]) << 16);
                *reinterpret_cast<uint4*>(p + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < TPT; ++k)
                if (t0 + k >= pos0 && t0 + k < pos0 + g.n) p[k] = b[k];
        }
    }
}

// Same work with the loads of all of a thread's items issued before the cos/sin of the
// position are computed: the libm calls overlap the memory latency instead of preceding it.
// IPT = items per thread (heads * head_dim / 8 <= kRopeThreads * IPT).  With TPT > 0 the first
// nv workgroups are V tiles and the position workgroups leave V alone.
template <int IPT, int TPT>
__global__ void __launch_bounds__(kRopeThreads) rope_append_items_kernel(const RopeAppendArgs a, int nv) {
    const AppendArgs& g = a.app;
    int pos0 = g.pos0;
    if (g.pos_dev) {  // device-side position: written only where the pages of all rows were claimed
        pos0 = *g.pos_dev;
        if (pos0 < 0 || pos0 > g.max_seq - g.n || ((pos0 + g.n - 1) >> kPageShift) >= *g.held_dev) return;
    }
    if (TPT > 0 && static_cast<int>(blockIdx.x) < nv) {
        v_tile_store<TPT ? TPT : 8>(g, pos0, blockIdx.x);
        return;
    }
    const int D = g.geom.head_dim;
    const int half = D >> 1;
    const int kv_heads = g.geom.kv_heads;
    const int q_heads = a.q ? a.q_width / D : 0;
    const int heads = kv_heads + q_heads;
    const int per_head = half / 4;
    const int nitems = heads * per_head;
    const long long row = static_cast<int>(blockIdx.x) - (TPT > 0 ? nv : 0);  // one position per workgroup
    float4 x0[IPT], x1[IPT], w0[IPT], w1[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = min(static_cast<int>(threadIdx.x) + kRopeThreads * k, nitems - 1);  // past the end: a valid item, not stored
        const int h = it / per_head;
        const int d = 4 * (it - h * per_head);
        const float* src = h < kv_heads ? static_cast<const float*>(g.src[0]) + row * g.src_stride + h * D
                                        : a.q + row * a.q_width + (h - kv_heads) * D;
        x0[k] = *reinterpret_cast<const float4*>(src + d);
        x1[k] = *reinterpret_cast<const float4*>(src + d + half);
        if (TPT == 0) {
            const float* v = static_cast<const float*>(g.src[1]) + row * g.src_stride + min(h, kv_heads - 1) * D;
            w0[k] = *reinterpret_cast<const float4*>(v + d);
            w1[k] = *reinterpret_cast<const float4*>(v + d + half);
        }
    }
    __shared__ float cs[2][kMaxRopeHalf];
    for (int i = threadIdx.x; i < half; i += kRopeThreads) {
        const float ang = mul_rn(static_cast<float>(pos0 + row), a.freq[i]);
        cs[0][i] = cosf(ang);
        cs[1][i] = sinf(ang);
    }
    __syncthreads();
    const int t = pos0 + static_cast<int>(row);
    const long long phys = g.page_table[t >> kPageShift];
    const int slot = t & (kPageTokens - 1);
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = threadIdx.x + kRopeThreads * k;
        if (it >= nitems) break;
        const int h = it / per_head;
        const int d = 4 * (it - h * per_head);
        const float4 c = *reinterpret_cast<const float4*>(&cs[0][d]);
        const float4 sn = *reinterpret_cast<const float4*>(&cs[1][d]);
        const float cc[4] = {c.x, c.y, c.z, c.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
        const float a0[4] = {x0[k].x, x0[k].y, x0[k].z, x0[k].w}, a1[4] = {x1[k].x, x1[k].y, x1[k].z, x1[k].w};
        float y0[4], y1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            y0[e] = sub_rn(mul_rn(a0[e], cc[e]), mul_rn(a1[e], ss[e]));
            y1[e] = add_rn(mul_rn(a0[e], ss[e]), mul_rn(a1[e], cc[e]));
        }
        if (h < kv_heads) {
            store4(g.pool, g.dtype, g.geom, phys, 0, h, slot, d, y0);
            store4(g.pool, g.dtype, g.geom, phys, 0, h, slot, d + half, y1);
            if (TPT == 0) {
                const float v0[4] = {w0[k].x, w0[k].y, w0[k].z, w0[k].w}, v1[4] = {w1[k].x, w1[k].y, w1[k].z, w1[k].w};
                store4(g.pool, g.dtype, g.geom, phys, 1, h, slot, d, v0);
                store4(g.pool, g.dtype, g.geom, phys, 1, h, slot, d + half, v1);
            }
        } else {
            float* q = a.q + row * a.q_width + (h - kv_heads) * D;
            *reinterpret_cast<float4*>(q + d) = make_float4(y0[0], y0[1], y0[2], y0[3]);
            *reinterpret_cast<float4*>(q + d + half) = make_float4(y1[0], y1[1], y1[2], y1[3]);
        }
    }
}

__global__ void __launch_bounds__(256) rope_append_kernel(const RopeAppendArgs a) {
    const AppendArgs& g = a.app;
    const int D = g.geom.head_dim;
    const int half = D >> 1;
    const int kv_heads = g.geom.kv_heads;
    const int q_heads = a.q ? a.q_width / D : 0;
    const int r0 = blockIdx.x * kRopeRows;
    __shared__ float cs[kRopeRows][2][kMaxRopeHalf];
    for (int idx = threadIdx.x; idx < kRopeRows * half; idx += 256) {
        const int r = idx / half, i = idx - r * half;
        const float ang = mul_rn(static_cast<float>(g.pos0 + r0 + r), a.freq[i]);
        cs[r][0][i] = cosf(ang);
        cs[r][1][i] = sinf(ang);
    }
    __syncthreads();
    const int per_head = half / 4;
    const int heads = kv_heads + q_heads;
    for (int it = threadIdx.x; it < kRopeRows * heads * per_head; it += 256) {
        const int r = it / (heads * per_head);
        const int rem = it - r * heads * per_head;
        const int h = rem / per_head;
        const int d = 4 * (rem - h * per_head);
        if (r0 + r >= g.n) continue;
        const float4 c = *reinterpret_cast<const float4*>(&cs[r][0][d]);
        const float4 sn = *reinterpret_cast<const float4*>(&cs[r][1][d]);
        const float cc[4] = {c.x, c.y, c.z, c.w}, ss[4] = {sn.x, sn.y, sn.z, sn.w};
        const long long row = r0 + r;
        const float* src = h < kv_heads ? static_cast<const float*>(g.src[0]) + row * g.src_stride + h * D
                                        : a.q + row * a.q_width + (h - kv_heads) * D;
        const float4 a0 = *reinterpret_cast<const float4*>(src + d);
        const float4 a1 = *reinterpret_cast<const float4*>(src + d + half);
        const float x0[4] = {a0.x, a0.y, a0.z, a0.w}, x1[4] = {a1.x, a1.y, a1.z, a1.w};
        float y0[4], y1[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            y0[e] = sub_rn(mul_rn(x0[e], cc[e]), mul_rn(x1[e], ss[e]));
            y1[e] = add_rn(mul_rn(x0[e], ss[e]), mul_rn(x1[e], cc[e]));
        }
        if (h < kv_heads) {
            const int t = g.pos0 + r0 + r;
            const long long phys = g.page_table[t >> kPageShift];
            const int slot = t & (kPageTokens - 1);
            store4(g.pool, g.dtype, g.geom, phys, 0, h, slot, d, y0);
            store4(g.pool, g.dtype, g.geom, phys, 0, h, slot, d + half, y1);
            const float* v = static_cast<const float*>(g.src[1]) + row * g.src_stride + h * D;
            const float4 b0 = *reinterpret_cast<const float4*>(v + d);
            const float4 b1 = *reinterpret_cast<const float4*>(v + d + half);
            const float v0[4] = {b0.x, b0.y, b0.z, b0.w}, v1[4] = {b1.x, b1.y, b1.z, b1.w};
            store4(g.pool, g.dtype, g.geom, phys, 1, h, slot, d, v0);
            store4(g.pool, g.dtype, g.geom, phys, 1, h, slot, d + half, v1);
        } else {
            float* q = a.q + row * a.q_width + (h - kv_heads) * D;
            *reinterpret_cast<float4*>(q + d) = make_float4(y0[0], y0[1], y0[2], y0[3]);
            *reinterpret_cast<float4*>(q + d + half) = make_float4(y1[0], y1[1], y1[2], y1[3]);
        }
    }
}

// A float into the cache dtype (the append codecs).
__device__ __forceinline__ void store1(void* pool, int dtype, long long j, float x) {
    switch (dtype) {
        case QR_DTYPE_F32: static_cast<float*>(pool)[j] = x; break;
        case QR_DTYPE_F16: static_cast<uint16_t*>(pool)[j] = f32_to_f16_bits_ref(x); break;
        default: static_cast<uint16_t*>(pool)[j] = f32_to_bf16_bits_ref(x); break;
    }
}

// Any head size the item kernels do not take (not a multiple of 8, or above 256): one
// workgroup per position, one thread per rotation pair (i, i + D/2) of a head, with the same
// separately rounded products and sums; an odd head size leaves dim D - 1 unrotated, as the
// reference rotates i < D/2 only (TransformerOps.cs:78-87).  V rows (and dim D - 1 of
// each K row) are copied in a second loop.
__global__ void __launch_bounds__(256) rope_append_generic_kernel(const RopeAppendArgs a) {
    const AppendArgs& g = a.app;
    int pos0 = g.pos0;
    if (g.pos_dev) {  // device-side position: written only where the pages of all rows were claimed
        pos0 = *g.pos_dev;
        if (pos0 < 0 || pos0 > g.max_seq - g.n || ((pos0 + g.n - 1) >> kPageShift) >= *g.held_dev) return;
    }
    const int D = g.geom.head_dim;
    const int half = D >> 1;
    const int kv_heads = g.geom.kv_heads;
    const int q_heads = a.q ? a.q_width / D : 0;
    const long long row = blockIdx.x;
    const int t = pos0 + static_cast<int>(row);
    __shared__ float cs[2][kMaxRopeHalf];
    for (int i = threadIdx.x; i < half; i += 256) {
        const float ang = mul_rn(static_cast<float>(t), a.freq[i]);
        cs[0][i] = cosf(ang);
        cs[1][i] = sinf(ang);
    }
    __syncthreads();
    const long long phys = g.page_table[t >> kPageShift];
    const int slot = t & (kPageTokens - 1);
    const float* krow = static_cast<const float*>(g.src[0]) + row * g.src_stride;
    const float* vrow = static_cast<const float*>(g.src[1]) + row * g.src_stride;
    const int pairs = (kv_heads + q_heads) * half;
    for (int it = threadIdx.x; it < pairs; it += 256) {
        const int h = it / half;
        const int i = it - h * half;
        float* q = h < kv_heads ? nullptr : a.q + row * a.q_width + (h - kv_heads) * D;
        const float* src = q ? q : krow + h * D;
        const float x0 = src[i], x1 = src[i + half];
        const float c = cs[0][i], sn = cs[1][i];
        const float y0 = sub_rn(mul_rn(x0, c), mul_rn(x1, sn));
        const float y1 = add_rn(mul_rn(x0, sn), mul_rn(x1, c));
        if (q) {
            q[i] = y0;
            q[i + half] = y1;
        } else {
            store1(g.pool, g.dtype, g.geom.offset(phys, 0, h, slot, i), y0);
            store1(g.pool, g.dtype, g.geom.offset(phys, 0, h, slot, i + half), y1);
        }
    }
    for (int it = threadIdx.x; it < kv_heads * D; it += 256) {
        const int h = it / D;
        const int d = it - h * D;
        store1(g.pool, g.dtype, g.geom.offset(phys, 1, h, slot, d), vrow[h * D + d]);
        if (d == 2 * half) store1(g.pool, g.dtype, g.geom.offset(phys, 0, h, slot, d), krow[h * D + d]);  // odd D
    }
}

__global__ void __launch_bounds__(256) widen_kernel(const void* src, int dtype, float* dst, long long n) {
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += static_cast<long long>(gridDim.x) * 256)
        dst[i] = load_f32(src, dtype, i);
}

unsigned grid_for(long long total) {
    long long blocks = (total + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 8192) blocks = 8192;
    return static_cast<unsigned>(blocks);
}

}  // namespace

hipError_t launch_append(const AppendArgs& a, hipStream_t stream) {
    const long long total = static_cast<long long>(a.n) * a.geom.kv_heads * a.geom.head_dim * a.geom.planes;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(append_kernel, dim3(grid_for(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

// One thread: the pages a device-side position needs, from the pool's device counter.
__global__ void __launch_bounds__(64) page_claim_kernel(const PageClaimArgs a) {
    if (threadIdx.x != 0) return;
    const int pos = *a.pos_dev;
    if (pos < 0 || pos > a.max_seq - a.n) {
        atomicOr(&a.state[1], 2);
        return;
    }
    const int need = ((pos + a.n - 1) >> kPageShift) + 1;
    const int held = a.state[a.held_index];
    if (need > held) {
        const int cnt = need - held;
        const int first = atomicAdd(&a.state[0], cnt);
        if (first + cnt > a.capacity) {
            atomicSub(&a.state[0], cnt);
            atomicOr(&a.state[1], 1);
            return;
        }
        for (int i = 0; i < cnt; ++i) a.page_table[held + i] = first + i;
        a.state[a.held_index] = need;
    }
    atomicMax(&a.state[a.seq_index], pos + a.n);  // PagedKvCache.cs:68
}

hipError_t launch_page_claim(const PageClaimArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(page_claim_kernel, dim3(1), dim3(64), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_gather(const GatherArgs& a, hipStream_t stream) {
    const long long total = static_cast<long long>(a.n) * a.geom.kv_heads * a.geom.head_dim * a.geom.planes;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_rope_append(const RopeAppendArgs& a, hipStream_t stream) {
    if (a.app.n == 0) return hipSuccess;
    const int D = a.app.geom.head_dim;
    if (rope_generic(D)) {
        if (D > 2 * kMaxRopeHalf) return hipErrorInvalidValue;
        hipLaunchKernelGGL(rope_append_generic_kernel, dim3(a.app.n), dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    const int heads = a.app.geom.kv_heads + (a.q ? a.q_width / D : 0);
    const int ipt = rope_items_per_thread(heads, D);
    // V tiles: 16-bit MFMA-layout V plane (head_dim 64 or 128), kVTileTpt tokens per thread
    const bool tiles = a.app.geom.mfma_layout && a.app.geom.planes == 2 && (D == 64 || D == 128) &&
                       a.app.dtype != QR_DTYPE_F32;
    int nv = 0;
    if (tiles) {
        const int T = v_tile_tokens(D, kVTileTpt);
        // with a device position, the most tiles n rows can span (those past the rows return)
        nv = (a.app.pos_dev ? (a.app.n + T - 2) / T + 1 : (a.app.pos0 + a.app.n - 1) / T - a.app.pos0 / T + 1) *
             a.app.geom.kv_heads;
    }
    const dim3 grid(static_cast<unsigned>(a.app.n + nv));
#define QR_ROPE_ITEMS(I)                                                                               \
    do {                                                                                               \
        if (tiles) hipLaunchKernelGGL((rope_append_items_kernel<I, kVTileTpt>), grid, dim3(kRopeThreads), 0, stream, a, nv); \
        else hipLaunchKernelGGL((rope_append_items_kernel<I, 0>), grid, dim3(kRopeThreads), 0, stream, a, 0);             \
    } while (0)
    switch (ipt) {
    case 1: QR_ROPE_ITEMS(1); break;
    case 2: QR_ROPE_ITEMS(2); break;
    case 3: QR_ROPE_ITEMS(3); break;
    case 4: QR_ROPE_ITEMS(4); break;
    case 5: QR_ROPE_ITEMS(5); break;
    case 6: QR_ROPE_ITEMS(6); break;
    case 7: case 8: QR_ROPE_ITEMS(8); break;
    default:
        if (a.app.pos_dev) return hipErrorInvalidValue;  // device positions: the item kernel only
        hipLaunchKernelGGL(rope_append_kernel, dim3((a.app.n + kRopeRows - 1) / kRopeRows), dim3(256), 0, stream, a);
    }
#undef QR_ROPE_ITEMS
    return hipGetLastError();
}

hipError_t launch_widen(const void* src, int src_dtype, float* dst, long long n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(widen_kernel, dim3(grid_for(n)), dim3(256), 0, stream, src, src_dtype, dst, n);
    return hipGetLastError();
}

namespace {
__global__ void __launch_bounds__(64) positions_kernel(int* out, const int* pos0_dev, int n) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i < n) out[i] = *pos0_dev + i;
}
}  // namespace

hipError_t launch_positions(int* out, const int* pos0_dev, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(positions_kernel, dim3((n + 63) / 64), dim3(64), 0, stream, out, pos0_dev, n);
    return hipGetLastError();
}

}  // namespace qr
