// qr_mla.hip -- MLA absorbed attention over the paged latent cache (gfx950).
//
// Replaces the score -> softmax -> latent-sum loops of StreamingEngine.MlaLayer
// (StreamingEngine.cs:531-568).  Latent pages are token-major rows of
// kv_lora + rope elements ([c_kv | k_pe], StreamingEngine.cs:494-506).
//
// mla_split_generic_kernel: one workgroup per (split of 256 positions, head).
//   Scores of the split are staged in LDS; the split's partial (max, sum,
//   unnormalised u) is merged across splits by mla_combine_kernel.  This path
//   serves every cache dtype.
#include "qr_mla.hpp"

#include <algorithm>

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

}  // namespace

MlaPlan plan_mla(const MlaArgs& a) {
    MlaPlan pl{};
    pl.split_tokens = kGenericSplit;
    pl.splits = (a.seq_len + pl.split_tokens - 1) / pl.split_tokens;
    pl.workspace_bytes = pl.splits > 1
        ? static_cast<size_t>(a.heads) * pl.splits * (static_cast<size_t>(a.kv_lora) * 4 + 8)
        : 0;
    return pl;
}

hipError_t launch_mla(const MlaArgs& a, const MlaPlan& pl, void* workspace, hipStream_t stream) {
    if (pl.splits > 4096) return hipErrorInvalidValue;
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
    const size_t slots = static_cast<size_t>(a.heads) * pl.splits;
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
