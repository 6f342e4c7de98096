// qr_proj.hip -- MLA q-absorb (W_UK) and W_UV up-projection with on-the-fly dequant of
// the kvb rows (StreamingEngine.cs:517-529, :569-576), in the reference's fp32
// operation order so that the results equal the reference's bit for bit:
//   absorb  q~_h[k] = (((0 + q_h[0] W[h,0,k]) + q_h[1] W[h,1,k]) + ...)   j ascending
//   W_UV    out_h[j] = DotF32(W_UV,h[j], u_h): 8 lane sums over k = 8c + L (c ascending),
//           then 0 + lane0 + ... + lane7 (SimdMath.cs:17-22, :34-53)
// Products and sums are separately rounded (mul_rn / add_rn: no FMA contraction).
// Both are HBM-bound weight streams (one pass over heads*(nope+vdim) rows per call).
#include <algorithm>

#include "qr_mfma.hpp"
#include "qr_proj.hpp"

namespace qr {

namespace {

// ------------------------------------------------------------------ q-absorb
// One wave per (128-column slice, head, batch tile); each lane owns columns k, k+1
// and walks the nope rows of its head in order.  Rows go in blocks of AbsRows<FMT>,
// double buffered as raw loads: the loads of block i+1 are in flight while block i is
// decoded and summed.
constexpr int kAbsThreads = 64;

template <int FMT>
struct AbsRows {  // rows per block: 32 load instructions, so that a wait for one block can
                  // leave the next block's loads outstanding (vmcnt counts at most 63)
    static constexpr int loads = FMT == QR_FMT_Q6_K ? 4 : (FMT == QR_FMT_Q4_0 || FMT == QR_FMT_Q8_0 || FMT == QR_FMT_Q4_K) ? 2 : 1;
    static constexpr int value = 32 / loads;
};

// q[b][h][64 g + lane] for the four 64-row groups g of nope <= 256, in named fields (an
// array indexed by the uniform group would be moved to LDS by the compiler).
struct QGroups {
    float g0, g1, g2, g3;
    __device__ __forceinline__ float pick(int g) const { return g == 0 ? g0 : g == 1 ? g1 : g == 2 ? g2 : g3; }
};
static_assert(kMlaProjMaxNope == 256, "QGroups holds four 64-row groups");

template <int FMT, int NBT>
__global__ __launch_bounds__(kAbsThreads) void mla_absorb_kernel(MlaProjArgs a) {
    constexpr int U = AbsRows<FMT>::value;
    const int h = blockIdx.y;
    const int b0 = blockIdx.z * NBT;
    const int nb = NBT == 1 ? 1 : min(NBT, a.nq - b0);
    const int lane = threadIdx.x;
    const int nope = a.nope;
    const int qk = nope + a.rope;
    const long long qrow = static_cast<long long>(a.heads) * qk;
    const float* q = a.in + b0 * qrow + static_cast<long long>(h) * qk;
    const int k = 2 * (blockIdx.x * kAbsThreads + lane);
    const int kk = k < a.kv_lora ? k : 0;  // lanes past the end load a valid column and drop it
    // The head's W_UK rows as one buffer: a row is selected by a scalar offset.
    const uint8_t* W = a.w + static_cast<long long>(h) * (nope + a.vdim) * a.row_bytes;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(W), static_cast<short>(0), static_cast<int>(nope * a.row_bytes), kBufferFlags);
    const uint32_t rb = static_cast<uint32_t>(a.row_bytes);

    // q[b][h][64 s + lane] in lane `lane` of qv[b][s]; rows read it back with readlane.
    // Indices are clamped (lanes past nope hold a copy that no row reads), so the loads
    // need no branches.
    QGroups qv[NBT];
#pragma unroll
    for (int b = 0; b < NBT; ++b) {
        const float* qb = q + min(b, nb - 1) * qrow;
        qv[b].g0 = qb[min(lane, nope - 1)];
        qv[b].g1 = qb[min(64 + lane, nope - 1)];
        qv[b].g2 = qb[min(128 + lane, nope - 1)];
        qv[b].g3 = qb[min(192 + lane, nope - 1)];
    }

    float ax[NBT], ay[NBT];
#pragma unroll
    for (int b = 0; b < NBT; ++b) ax[b] = ay[b] = 0.0f;

    auto load = [&](Raw<FMT>* buf, int j) {
#pragma unroll
        for (int u = 0; u < U; ++u) buf[u] = raw<FMT>(BufRow{rsrc, (j + u) * rb}, kk);
    };
    // rows j..j+U-1 lie in one 64-row group of q (U divides 64 and j is a multiple of U)
    auto compute = [&](const Raw<FMT>* buf, int j) {
        float qs[NBT];
#pragma unroll
        for (int b = 0; b < NBT; ++b) qs[b] = qv[b].pick(j >> 6);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float2 w = dec<FMT>(buf[u], kk);
#pragma unroll
            for (int b = 0; b < NBT; ++b) {
                if (b < nb) {
                    const float qval = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qs[b]), (j & 63) + u));
                    ax[b] = add_rn(ax[b], mul_rn(qval, w.x));
                    ay[b] = add_rn(ay[b], mul_rn(qval, w.y));
                }
            }
        }
    };

    const int nfull = nope / U;
    Raw<FMT> bufA[U], bufB[U];
    if (nfull > 0) load(bufA, 0);
    for (int i = 0; i < nfull; i += 2) {
        if (i + 1 < nfull) load(bufB, (i + 1) * U);
        compute(bufA, i * U);
        if (i + 1 >= nfull) break;
        if (i + 2 < nfull) load(bufA, (i + 2) * U);
        compute(bufB, (i + 1) * U);
    }
    for (int j = nfull * U; j < nope; ++j) {
        const float2 w = dec<FMT>(raw<FMT>(BufRow{rsrc, j * rb}, kk), kk);
#pragma unroll
        for (int b = 0; b < NBT; ++b) {
            if (b < nb) {
                const float qval = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qv[b].pick(j >> 6)), j & 63));
                ax[b] = add_rn(ax[b], mul_rn(qval, w.x));
                ay[b] = add_rn(ay[b], mul_rn(qval, w.y));
            }
        }
    }

    if (k < a.kv_lora) {
#pragma unroll
        for (int b = 0; b < NBT; ++b) {
            if (b < nb) {
                float* o = a.out + (static_cast<long long>(b0 + b) * a.heads + h) * a.kv_lora + k;
                *reinterpret_cast<float2*>(o) = make_float2(ax[b], ay[b]);
            }
        }
    }
    if (a.q_rope && blockIdx.x == 0) {
        for (int i = lane; i < nb * a.rope; i += kAbsThreads) {
            const int b = i / a.rope, r = i - b * a.rope;
            a.q_rope[(static_cast<long long>(b0 + b) * a.heads + h) * a.rope + r] = q[b * qrow + nope + r];
        }
    }
}

// q-absorb of one query with nope <= kAbsSumRows, block formats: workgroup = 4 waves =
// (128-column slice, head).  Wave w loads rows j = w, w + 4, ... of the head's W_UK, all at
// once, and lane l writes the products q_j W[h,j,k] of its columns k = 2l, 2l + 1 to LDS;
// then thread c adds column c's products in row order from 0 -- the reference's sequence,
// the same bits as the one-wave kernel, whose rows stream in blocks with one block in
// flight.  Four times the waves carry the block formats' decode: Q8_0 kvb at the C5 shape
// 9.0 -> 7.9 us; bf16 kvb, whose decode is a shift, 6.6 -> 7.0 us, so the fp formats keep
// the one-wave form.
constexpr int kAbsSumRows = 128;

template <int FMT>
__global__ __launch_bounds__(256) void mla_absorb_sum_kernel(MlaProjArgs a) {
    constexpr int RPW = kAbsSumRows / 4;  // rows per wave
    __shared__ float prod[kAbsSumRows][2 * kAbsThreads];
    const int h = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nope = a.nope;
    const int qk = nope + a.rope;
    const float* q = a.in + static_cast<long long>(h) * qk;
    const int k = 2 * (blockIdx.x * kAbsThreads + lane);
    const int kk = k < a.kv_lora ? k : 0;  // lanes past the end load a valid column and drop it
    const uint8_t* W = a.w + static_cast<long long>(h) * (nope + a.vdim) * a.row_bytes;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(W), static_cast<short>(0), static_cast<int>(nope * a.row_bytes), kBufferFlags);
    const uint32_t rb = static_cast<uint32_t>(a.row_bytes);
    Raw<FMT> buf[RPW];
    float qj[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int j = min(w + 4 * i, nope - 1);  // rows past nope: a valid row, not stored
        buf[i] = raw<FMT>(BufRow{rsrc, j * rb}, kk);
        qj[i] = q[j];
    }
    // every load is issued before the first product (the compiler would otherwise walk
    // the rows one round trip at a time in a few registers)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int j = w + 4 * i;
        if (j >= nope) break;
        const float2 wv = dec<FMT>(buf[i], kk);
        *reinterpret_cast<float2*>(&prod[j][2 * lane]) = make_float2(mul_rn(qj[i], wv.x), mul_rn(qj[i], wv.y));
    }
    __syncthreads();
    if (threadIdx.x < 2 * kAbsThreads) {
        const int c = threadIdx.x;
        const int kc = 2 * blockIdx.x * kAbsThreads + c;
        float acc = 0.0f;
        int j = 0;
        for (; j + 16 <= nope; j += 16) {  // 16 reads in flight, then their adds in order
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = prod[j + u][c];
#pragma unroll
            for (int u = 0; u < 16; ++u) acc = add_rn(acc, v[u]);
        }
        for (; j < nope; ++j) acc = add_rn(acc, prod[j][c]);
        if (kc < a.kv_lora) a.out[static_cast<long long>(h) * a.kv_lora + kc] = acc;
    }
    if (a.q_rope && blockIdx.x == 0) {
        for (int i = threadIdx.x; i < a.rope; i += 256) a.q_rope[static_cast<long long>(h) * a.rope + i] = q[nope + i];
    }
}

// ------------------------------------------------------------------ W_UV
// One workgroup per (32 rows of W_UV,h, head, batch tile).  The rows are one contiguous
// byte range of kvb, taken in column slabs of <= kSlabBytes per row.  A slab is copied
// into LDS with coalesced loads (its u values alongside, all issued before any is
// stored), then thread (row r, pair p) decodes weights 8c+2p, 8c+2p+1 -- DotF32 lanes
// 2p and 2p+1 -- and keeps the two lane sums of each query.  (Double buffering the slabs
// measured slower: the C5 rows fit one slab.)
constexpr int kWuvRows = 32;
constexpr int kWuvThreads = 4 * kWuvRows;
constexpr int kSlabBytes = 1024;
constexpr int kMaxSlabCols = 1024;
constexpr int kStageBatch = kWuvRows * kSlabBytes / (16 * kWuvThreads);  // one batch of 16-byte copies per slab

struct WuvLayout {
    int slab_cols;   // columns per slab (multiple of 8 and of the block)
    int lds_stride;  // bytes per staged row (16-byte multiple, padded)
    int copy_bytes;  // 16, 4 or 2: width of the staging copies
    int dma;         // slabs of whole 1 KiB rows, 16-byte aligned: staged by direct-to-LDS loads
    __host__ __device__ size_t tile_bytes(int nbt) const {
        return static_cast<size_t>(kWuvRows) * lds_stride + static_cast<size_t>(nbt) * slab_cols * 4;
    }
    __host__ __device__ size_t lds_bytes(int nbt) const { return tile_bytes(nbt); }
};

template <int G> struct CopyWord;
template <> struct CopyWord<16> { typedef u32x4_t type; };
template <> struct CopyWord<4> { typedef uint32_t type; };
template <> struct CopyWord<2> { typedef uint16_t type; };

// One slab in flight in registers: the first batch of weight copies and the u values,
// each with its LDS destination (-1: an index past the end, clamped to a valid address).
template <int G, int KU>
struct SlabRegs {
    typename CopyWord<G>::type v[kStageBatch];
    int dst[kStageBatch];
    float2 u[KU];
    int udst[KU];
};

// Where slab s lives.  Row index = i / per_row as a multiply-high by magic =
// floor((2^32 - 1) / per_row) + 1, exact for every i < 2^16 and 2 <= per_row <= 4096 (a
// slab holds at most kWuvRows * kSlabBytes / 2 accesses); per_row 1 takes i itself.
struct SlabGeom {
    const uint8_t* src;  // first staged byte of row 0
    const float* u_src;  // u[b0][h][c0]
    int cols, per_row, total;
    uint32_t magic;
};

template <int FMT, int NBT, int G>
__device__ __forceinline__ void wuv_body(const MlaProjArgs& a, const WuvLayout& L, uint8_t* lds) {
    constexpr int KU = NBT * kMaxSlabCols / 2 / kWuvThreads;  // float2 u loads per thread per slab
    constexpr int kSteps = 8;                                   // 8-column chunks per batch of reads
    typedef typename CopyWord<G>::type V;
    FormatSpec fs;
    weight_format_spec(FMT, &fs);
    const int h = blockIdx.y, j0 = blockIdx.x * kWuvRows;
    const int nrows = min(kWuvRows, a.vdim - j0);
    const int b0 = blockIdx.z * NBT;
    const int nb = NBT == 1 ? 1 : min(NBT, a.nq - b0);
    const int t = threadIdx.x, r = t >> 2, p = t & 3;
    const int rr = min(r, nrows - 1);  // rows past the end compute on a valid row and drop it
    const uint8_t* W = a.w + (static_cast<long long>(h) * (a.nope + a.vdim) + a.nope + j0) * a.row_bytes;
    const float* U0 = a.in + (static_cast<long long>(b0) * a.heads + h) * a.kv_lora;
    const long long u_stride = static_cast<long long>(a.heads) * a.kv_lora;
    const int ns = (a.kv_lora + L.slab_cols - 1) / L.slab_cols;

    auto geom = [&](int s) {
        SlabGeom g;
        const int c0 = s * L.slab_cols;
        g.cols = min(L.slab_cols, a.kv_lora - c0);
        g.src = W + static_cast<long long>(c0 / fs.block) * fs.bytes;
        g.u_src = U0 + c0;
        g.per_row = g.cols / fs.block * fs.bytes / G;
        g.total = g.per_row * nrows;
        g.magic = 0xFFFFFFFFu / static_cast<uint32_t>(g.per_row) + 1u;
        return g;
    };
    auto row_of = [](int i, const SlabGeom& g) {
        return g.per_row == 1 ? i : static_cast<int>(__umulhi(static_cast<uint32_t>(i), g.magic));
    };
    auto copy_batch = [&](SlabRegs<G, KU>& R, const SlabGeom& g, int base) {
#pragma unroll
        for (int s = 0; s < kStageBatch; ++s) {
            const int idx = base + t + s * kWuvThreads;
            const int i = min(idx, g.total - 1);
            const int rw = row_of(i, g), e = i - rw * g.per_row;
            R.v[s] = *reinterpret_cast<const V*>(g.src + rw * a.row_bytes + e * G);
            R.dst[s] = idx < g.total ? rw * L.lds_stride + e * G : -1;
        }
    };
    auto store_batch = [&](const SlabRegs<G, KU>& R, uint8_t* tl) {
#pragma unroll
        for (int s = 0; s < kStageBatch; ++s)
            if (R.dst[s] >= 0) *reinterpret_cast<V*>(tl + R.dst[s]) = R.v[s];
    };
    // issue: the slab's first copy batch and its u values, no waits
    auto issue = [&](SlabRegs<G, KU>& R, int s) {
        const SlabGeom g = geom(s);
        copy_batch(R, g, 0);
        const int half = g.cols / 2, un = nb * half;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int idx = t + k * kWuvThreads;
            const int i = min(idx, un - 1);
            const int b = i / half, e = i - b * half;
            R.u[k] = *reinterpret_cast<const float2*>(g.u_src + b * u_stride + 2 * e);
            R.udst[k] = idx < un ? b * L.slab_cols + 2 * e : -1;
        }
    };
    // land: store slab s, then copy any further batches one at a time
    auto land = [&](SlabRegs<G, KU>& R, int s) {
        uint8_t* tl = lds;
        float* ul = reinterpret_cast<float*>(tl + kWuvRows * L.lds_stride);
        store_batch(R, tl);
#pragma unroll
        for (int k = 0; k < KU; ++k)
            if (R.udst[k] >= 0) *reinterpret_cast<float2*>(ul + R.udst[k]) = R.u[k];
        const SlabGeom g = geom(s);
        for (int base = kWuvThreads * kStageBatch; base < g.total; base += kWuvThreads * kStageBatch) {
            copy_batch(R, g, base);
            store_batch(R, tl);
        }
    };

    float acc0[NBT], acc1[NBT];
#pragma unroll
    for (int b = 0; b < NBT; ++b) acc0[b] = acc1[b] = 0.0f;

    auto compute = [&](int s) {
        const uint8_t* tl = lds;
        const float* ul = reinterpret_cast<const float*>(tl + kWuvRows * L.lds_stride);
        const uint8_t* row = tl + rr * L.lds_stride;
        const int cols = min(L.slab_cols, a.kv_lora - s * L.slab_cols);
        // whole groups of kSteps chunks: fixed offsets from the row, no clamps and no
        // per-chunk conditions on the chains
        int c = 0;
        for (; c + 8 * kSteps <= cols; c += 8 * kSteps) {
            float2 w[kSteps];
#pragma unroll
            for (int k = 0; k < kSteps; ++k) w[k] = deq2<FMT>(row, c + 8 * k + 2 * p);
#pragma unroll
            for (int b = 0; b < NBT; ++b) {
                if (b < nb) {
                    float2 uu[kSteps];
#pragma unroll
                    for (int k = 0; k < kSteps; ++k)
                        uu[k] = *reinterpret_cast<const float2*>(ul + b * L.slab_cols + c + 8 * k + 2 * p);
#pragma unroll
                    for (int k = 0; k < kSteps; ++k) {
                        acc0[b] = add_rn(acc0[b], mul_rn(w[k].x, uu[k].x));
                        acc1[b] = add_rn(acc1[b], mul_rn(w[k].y, uu[k].y));
                    }
                }
            }
        }
        for (; c < cols; c += 8) {  // the last cols % (8 kSteps) columns, one chunk at a time
            const float2 w = deq2<FMT>(row, c + 2 * p);
#pragma unroll
            for (int b = 0; b < NBT; ++b) {
                if (b < nb) {
                    const float2 uu = *reinterpret_cast<const float2*>(ul + b * L.slab_cols + c + 2 * p);
                    acc0[b] = add_rn(acc0[b], mul_rn(w.x, uu.x));
                    acc1[b] = add_rn(acc1[b], mul_rn(w.y, uu.y));
                }
            }
        }
    };

    // Direct-to-LDS staging (1 KiB slab rows): one buffer-load DMA per weight row into its
    // padded LDS row and one per KiB of u, split over the waves; rows past the matrix lie
    // outside the buffer and land as zeros.  No address arithmetic or stores per copy.
    auto dma_slab = [&](int s) {
        const SlabGeom g = geom(s);
        const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
        const uint32_t voff = 16u * static_cast<uint32_t>(t & 63);
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(g.src), static_cast<short>(0), nrows * static_cast<int>(a.row_bytes), kBufferFlags);
        for (int r = wave; r < kWuvRows; r += kWuvThreads / 64)
            buffer_load_lds16<kCacheNt>(rw, reinterpret_cast<const char*>(lds) + r * L.lds_stride, voff,
                              static_cast<uint32_t>(r * a.row_bytes));
        const char* ul = reinterpret_cast<const char*>(lds) + kWuvRows * L.lds_stride;
        const int pieces = g.cols * 4 / 1024;
#pragma unroll
        for (int b = 0; b < NBT; ++b) {
            const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(g.u_src + min(b, nb - 1) * u_stride), static_cast<short>(0), g.cols * 4, kBufferFlags);
            for (int i = wave; i < pieces; i += kWuvThreads / 64)
                buffer_load_lds16(ru, ul + b * L.slab_cols * 4 + 1024 * i, voff, static_cast<uint32_t>(1024 * i));
        }
    };

    SlabRegs<G, KU> R;
    for (int s = 0; s < ns; ++s) {
        if (s > 0) __syncthreads();  // the previous slab's reads are done
        if (G == 16 && L.dma) {
            dma_slab(s);
            wait_dma();
        } else {
            issue(R, s);
            land(R, s);
        }
        __syncthreads();
        compute(s);
    }

    // HSum in lane order: the four threads of a row hold lanes (0,1) (2,3) (4,5) (6,7).
    const int lane0 = (threadIdx.x & 63) & ~3;
#pragma unroll
    for (int b = 0; b < NBT; ++b) {
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            sum = add_rn(sum, __shfl(acc0[b], lane0 + q, 64));
            sum = add_rn(sum, __shfl(acc1[b], lane0 + q, 64));
        }
        if (b < nb && p == 0 && r < nrows)
            a.out[(static_cast<long long>(b0 + b) * a.heads + h) * a.vdim + j0 + r] = sum;
    }
}

template <int FMT, int NBT>
__global__ __launch_bounds__(kWuvThreads) void mla_wuv_kernel(MlaProjArgs a, WuvLayout L) {
    extern __shared__ __align__(16) uint8_t wuv_lds[];
    if (L.copy_bytes == 16)
        wuv_body<FMT, NBT, 16>(a, L, wuv_lds);
    else if (L.copy_bytes == 4)
        wuv_body<FMT, NBT, 4>(a, L, wuv_lds);
    else
        wuv_body<FMT, NBT, 2>(a, L, wuv_lds);
}

WuvLayout wuv_layout(const MlaProjArgs& a) {
    FormatSpec fs;
    weight_format_spec(a.fmt, &fs);
    const int unit_cols = fs.block >= 8 ? fs.block : 8;  // 32 and 256 are multiples of 8
    const int unit_bytes = unit_cols / fs.block * fs.bytes;
    const int units = a.kv_lora / unit_cols;
    int per_slab = std::min(units, std::max(1, std::min(kSlabBytes / unit_bytes, kMaxSlabCols / unit_cols)));
    // prefer a slab whose byte size keeps 16-byte copies (whole rows when they fit)
    for (int n = per_slab; n > per_slab / 2 && per_slab < units; --n)
        if (n * unit_bytes % 16 == 0) { per_slab = n; break; }
    WuvLayout L{};
    L.slab_cols = per_slab * unit_cols;
    const int slab_bytes = L.slab_cols / fs.block * fs.bytes;
    L.lds_stride = (slab_bytes + 15) / 16 * 16 + 16;
    const uintptr_t base = reinterpret_cast<uintptr_t>(a.w);
    auto aligned = [&](int g) { return base % g == 0 && a.row_bytes % g == 0 && slab_bytes % g == 0; };
    L.copy_bytes = aligned(16) ? 16 : aligned(4) ? 4 : 2;
    L.dma = L.copy_bytes == 16 && slab_bytes == 1024 && a.kv_lora % L.slab_cols == 0 && L.slab_cols % 256 == 0 &&
            reinterpret_cast<uintptr_t>(a.in) % 16 == 0;
    return L;
}

template <int FMT>
hipError_t launch_absorb_fmt(const MlaProjArgs& a, hipStream_t stream) {
    const dim3 block(kAbsThreads);
    const int gx = (a.kv_lora / 2 + kAbsThreads - 1) / kAbsThreads;
    constexpr bool fp = FMT == QR_FMT_F32 || FMT == QR_FMT_F16 || FMT == QR_FMT_BF16;
    if (!fp && a.nq == 1 && a.nope <= kAbsSumRows) {
        hipLaunchKernelGGL((mla_absorb_sum_kernel<FMT>), dim3(gx, a.heads, 1), dim3(256), 0, stream, a);
    } else if (a.nq == 1) {
        hipLaunchKernelGGL((mla_absorb_kernel<FMT, 1>), dim3(gx, a.heads, 1), block, 0, stream, a);
    } else {
        hipLaunchKernelGGL((mla_absorb_kernel<FMT, 4>), dim3(gx, a.heads, (a.nq + 3) / 4), block, 0, stream, a);
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_wuv_fmt(const MlaProjArgs& a, hipStream_t stream) {
    const WuvLayout L = wuv_layout(a);
    const int gx = (a.vdim + kWuvRows - 1) / kWuvRows;
    if (a.nq == 1) {
        hipLaunchKernelGGL((mla_wuv_kernel<FMT, 1>), dim3(gx, a.heads, 1), dim3(kWuvThreads), L.lds_bytes(1),
                           stream, a, L);
    } else {
        hipLaunchKernelGGL((mla_wuv_kernel<FMT, 4>), dim3(gx, a.heads, (a.nq + 3) / 4), dim3(kWuvThreads),
                           L.lds_bytes(4), stream, a, L);
    }
    return hipGetLastError();
}

}  // namespace

bool mla_proj_shape_ok(int fmt, int kv_lora) {
    FormatSpec fs;
    return weight_format_spec(fmt, &fs) && kv_lora >= 8 && kv_lora % 8 == 0 && kv_lora % fs.block == 0;
}

hipError_t launch_mla_absorb(const MlaProjArgs& a, hipStream_t stream) {
    if (a.nq == 0) return hipSuccess;
    switch (a.fmt) {
    case QR_FMT_F32: return launch_absorb_fmt<QR_FMT_F32>(a, stream);
    case QR_FMT_F16: return launch_absorb_fmt<QR_FMT_F16>(a, stream);
    case QR_FMT_BF16: return launch_absorb_fmt<QR_FMT_BF16>(a, stream);
    case QR_FMT_Q4_0: return launch_absorb_fmt<QR_FMT_Q4_0>(a, stream);
    case QR_FMT_Q8_0: return launch_absorb_fmt<QR_FMT_Q8_0>(a, stream);
    case QR_FMT_Q4_K: return launch_absorb_fmt<QR_FMT_Q4_K>(a, stream);
    case QR_FMT_Q6_K: return launch_absorb_fmt<QR_FMT_Q6_K>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_mla_wuv(const MlaProjArgs& a, hipStream_t stream) {
    if (a.nq == 0) return hipSuccess;
    switch (a.fmt) {
    case QR_FMT_F32: return launch_wuv_fmt<QR_FMT_F32>(a, stream);
    case QR_FMT_F16: return launch_wuv_fmt<QR_FMT_F16>(a, stream);
    case QR_FMT_BF16: return launch_wuv_fmt<QR_FMT_BF16>(a, stream);
    case QR_FMT_Q4_0: return launch_wuv_fmt<QR_FMT_Q4_0>(a, stream);
    case QR_FMT_Q8_0: return launch_wuv_fmt<QR_FMT_Q8_0>(a, stream);
    case QR_FMT_Q4_K: return launch_wuv_fmt<QR_FMT_Q4_K>(a, stream);
    case QR_FMT_Q6_K: return launch_wuv_fmt<QR_FMT_Q6_K>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace qr
