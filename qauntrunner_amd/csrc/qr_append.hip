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
        const int t = a.pos0 + r;
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

hipError_t launch_gather(const GatherArgs& a, hipStream_t stream) {
    const long long total = static_cast<long long>(a.n) * a.geom.kv_heads * a.geom.head_dim * a.geom.planes;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_widen(const void* src, int src_dtype, float* dst, long long n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(widen_kernel, dim3(grid_for(n)), dim3(256), 0, stream, src, src_dtype, dst, n);
    return hipGetLastError();
}

}  // namespace qr
