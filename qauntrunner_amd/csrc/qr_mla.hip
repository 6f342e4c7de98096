// qr_mla.hip -- MLA absorbed attention over the paged latent cache (gfx950).
//
// Replaces the score -> softmax -> latent-sum loops of StreamingEngine.MlaLayer
// (StreamingEngine.cs:531-568).  Latent pages are token-major rows of
// kv_lora + rope elements ([c_kv | k_pe], StreamingEngine.cs:494-506).
//
// mla_tile_kernel (bf16/f16 latents, kv_lora 512, rope 0 or 64): MFMA tiles, see
//   below; splits merged by mla_combine_wide_kernel.
// mla_split_generic_kernel: one workgroup per (split of 256 positions, head).
//   Scores of the split are staged in LDS; the split's partial (max, sum,
//   unnormalised u) is merged across splits by mla_combine_kernel.  This path
//   serves every other shape and the fp32 cache.
#include "qr_mla.hpp"
#include "qr_mfma.hpp"

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
    const int* pos_dev;  // device position (seq = pos + 1, clamped to [1, seq_len]) when set
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

// Positions attended: seq_len, or a device position + 1 bounded by it (a scalar load: no
// kernel here writes positions).
__device__ __forceinline__ int device_seq(const int* pos_dev, int seq_len) {
    if (!pos_dev) return seq_len;
    const int pos = reinterpret_cast<const __attribute__((address_space(4))) int*>(
        reinterpret_cast<uintptr_t>(pos_dev))[0];
    return __builtin_amdgcn_readfirstlane(min(max(pos + 1, 1), seq_len));
}

__device__ __forceinline__ long long row_base(const MlaK& p, int t) {
    const long long phys = p.page_table[t >> kPageShift];
    return (phys * kPageTokens + (t & (kPageTokens - 1))) * p.width;
}

__global__ void __launch_bounds__(kThreads) mla_split_generic_kernel(const MlaK p) {
    const int split = blockIdx.x;
    const int h = blockIdx.y;
    const int t0 = split * p.split_tokens;
    const int t1 = min(device_seq(p.pos_dev, p.seq_len), t0 + p.split_tokens);
    const int n = t1 - t0;  // <= 0 past a device position: a zero partial of weight 0

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
// Workgroup = 8 waves (two per SIMD) = 32 heads over one split of the sequence,
// walked in tiles of 32 positions.  Waves 0-3 compute scores, waves 4-7 the softmax
// and PV, so on every SIMD one wave's MFMAs run beside the other's softmax and loads.
// A tile (32 latent rows, contiguous inside one page) is loaded into registers of
// the PV waves two tiles ahead of its use and written to one of three LDS buffers.
//   QK  wave w < 4 scores positions 16(w%2)..16(w%2)+15 of the tile for all 32 heads
//       over half of the latent's dims (k-steps of half w/2): S^T[pos][head] =
//       C[pos][dims] . q~^T[dims][head]; A is read from the row-major tile once per
//       k-step and feeds four MFMAs (two head tiles, hi + lo), B = the wave's half of q~
//       (hi + lo) stays in registers.  Raw partial scores of each half go to LDS.
//       (Waves owning 16 heads over all dims read every A operand twice per tile: C5
//       24.0 vs 23.8 us per call.)
//   Softmax (log2 units, online): PV wave v owns heads 8v..8v+7; it adds the two halves'
//   scores, keeps their (m, l)
//   and writes P (hi + lo parts) and the accumulator rescale factor of each head to
//   LDS.
//   PV  wave 4 + v owns latent dims 128v..128v+127 for all 32 heads:
//       U^T[dim][head] += C^T[dim][pos] . P^T[pos][head]; the C^T operand is read
//       from the same row-major tile with ds_read_b64_tr_b16.
// Two waves per SIMD because a single wave keeps too few LDS reads in flight: on
// gfx950 one wave per SIMD reads ~100 bytes/clk per CU from LDS, two reach ~190.
// Step t, two barriers: the QK waves score tile t+1 while the PV waves run the
// softmax of tile t (scores written in step t-1); a barrier publishes P; the PV waves
// accumulate tile t and store tile t+2 into LDS; the barrier that ends the step
// publishes the scores of tile t+1 and tile t+2, and frees P and the buffer of tile t.
// v_mfma_f32_16x16x32_f16 lane layout (checked on gfx950):
//   A[m = lane%16][k = 8*(lane/16)+i], B[k = 8*(lane/16)+i][n = lane%16],
//   D[m = 4*(lane/16)+r][n = lane%16].
// ds_read_b64_tr_b16 (checked on gfx950): inside each group of 16 lanes, lane j
//   receives element i (0..3) from the 8 bytes addressed by lane 4i + j/4, at
//   element j%4 of them.
// In PV the 8 k-slots of lane quarter q are the positions {4q..4q+3, 16+4q..16+4q+3}
// of the tile, so each half of a transposed read touches 8 distinct rows.
// Both products run in the cache's own 16-bit type, so the latent enters every MFMA
// unconverted and any finite latent value is handled exactly.  QK: q~ is split into
// hi + lo parts of that type (two MFMAs per k-step), keeping about 16 (bf16) or 22
// (fp16) significant bits; for fp16 caches q~ is first multiplied per head by the
// power of two that brings its largest element to at most 2^14 (exact, scores scaled
// back), so it cannot overflow.  PV: P (at most 2^8 with the lazy rescale below) also
// enters as hi + lo parts of the cache type.  Split partials (the unnormalised
// accumulators) are stored in fp16 times a power of two per (head, split, 128-dim
// block) chosen from the block's largest value, so they neither overflow nor lose their
// small values whatever the latent's range (a bf16 latent may hold values far outside
// fp16's range).
// LDS tile layout: blocks of 8 logical 16-byte chunks (128 bytes) x 32 rows; inside
// a block, chunk c of row r sits at slot (c % 8) ^ f(r), where f(r) is the 3-bit
// reversal of (r >> 1) & 7, so the 16 rows of a QK read and the 8 rows of half a
// transposed read fall on distinct banks.
constexpr int kMTile = 32;                 // positions per tile
constexpr int kMHeads = 32;                // heads per workgroup
constexpr int kMWaves = 8;
constexpr int kMfmaLora = 512;
constexpr int kScoreStride = kMTile + 4;   // floats per head row of a score buffer
constexpr float kRescaleSlack = 8.f;       // log2 units
constexpr int kQkAhead = 4;                // QK k-steps whose A operands are read ahead

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t* lds_i16x4_ptr;

__device__ __forceinline__ int row_swizzle(int r) {
    const int x = (r >> 1) & 7;
    return ((x & 1) << 2) | (x & 2) | (x >> 2);
}

// MFMA operands in the cache's own 16-bit type.
template <bool SRC_BF16> struct PvType;
template <> struct PvType<false> {
    typedef _Float16 elem;
    typedef f16x8_t vec;
    __device__ static f32x4_t mma(vec a, vec b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <> struct PvType<true> {
    typedef __bf16 elem;
    typedef __bf16 vec __attribute__((ext_vector_type(8)));
    __device__ static f32x4_t mma(vec a, vec b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

struct MlaMK {
    const char* pool;
    const int* page_table;
    int heads;
    int seq_len;
    const int* pos_dev;  // device position (seq = pos + 1, clamped to [1, seq_len]) when set
    int split_tokens;  // multiple of kMTile
    int splits;
    int groups;        // head groups of kMHeads
    int per_xcd;       // launch slots per XCD
    const float* q_tilde;
    const float* q_rope;
    float* u;
    void* part_u;      // [heads][splits][kv_lora] fp16: acc_s / 2^e (unnormalised)
    float2* part_ml;   // [heads][splits] (m, l)
    signed char* part_e;  // [heads][splits][4] e of each 128-dim block
    float qscale;      // scale * log2(e)
};

// Positions per split: the plan's; with a device position (the plan was made for the
// bound) the tiles of the sequence spread over the planned splits.
__device__ __forceinline__ int mla_split_tokens(const MlaMK& p, int seq) {
    if (!p.pos_dev) return p.split_tokens;
    const int tiles = (seq + kMTile - 1) / kMTile;
    return (tiles + p.splits - 1) / p.splits * kMTile;
}

template <bool SRC_BF16, int KR>
__global__ void __launch_bounds__(kMWaves * 64) mla_tile_kernel(const MlaMK p) {
    constexpr int KL = kMfmaLora;
    constexpr int W = KL + KR;            // latent width (elements)
    constexpr int RB = W * 2;             // row bytes
    constexpr int NK = W / 32;            // QK k-steps
    constexpr int NB = W / 64;            // 128-byte column blocks of a row
    constexpr int BB = kMTile * 128;      // block bytes
    constexpr int TB = NB * BB;           // tile bytes
    constexpr int NLD = 4 * NB;           // 1 KiB wave loads per tile, all by the PV waves
    constexpr int LDW = NLD / 4;          // loads per PV wave
    constexpr int PR = kMTile * 2 + 16;   // bytes per head row of P (k-slot order, padded)
    using MT = PvType<SRC_BF16>;          // MFMA operands in the cache type
    typedef typename MT::vec V;
    typedef typename MT::elem E;

    __shared__ __attribute__((aligned(1024))) char lds_b0[TB];
    __shared__ __attribute__((aligned(1024))) char lds_b1[TB];
    __shared__ __attribute__((aligned(1024))) char lds_b2[TB];
    __shared__ __attribute__((aligned(16))) float lds_s0[2 * kMHeads * kScoreStride];  // k halves 0, 1
    __shared__ __attribute__((aligned(16))) float lds_s1[2 * kMHeads * kScoreStride];
    __shared__ __attribute__((aligned(16))) char lds_p[2 * kMHeads * PR];  // P hi rows, then lo rows
    __shared__ float lds_corr[kMHeads];  // accumulator rescale factor of the tile
    __shared__ float lds_l[kMHeads];
    __shared__ int lds_qexp[kMHeads];

    // Launch slot b runs on XCD b % 8; consecutive logical indices (the head groups
    // of one split, then the next split) are kept on one XCD so its L2 serves the
    // repeated reads of a split's latent rows.
    const int b = blockIdx.x;
    const int idx = (b & 7) * p.per_xcd + (b >> 3);
    if (idx >= p.groups * p.splits) return;
    const int hg = idx % p.groups;
    const int split = idx / p.groups;
    const int seq = device_seq(p.pos_dev, p.seq_len);
    const int split_tokens = mla_split_tokens(p, seq);
    const int nsplit = (seq + split_tokens - 1) / split_tokens;
    if (split >= nsplit) return;
    const int t_begin = split * split_tokens;
    const int t_end = min(seq, t_begin + split_tokens);
    const int ntiles = (t_end - t_begin + kMTile - 1) / kMTile;  // >= 1
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6) & (kMWaves - 1);  // wave-uniform (SGPR)
    const bool qk_wave = wave < 4;   // waves 0-3: QK; waves 4-7: softmax, PV and the tile copies
    const int pw = wave & 3;         // index inside the role
    const int q4 = lane >> 4;
    const int l16 = lane & 15;

    // Tile copy (PV waves).  Block g of the LDS tile (4 KiB) holds logical chunks
    // 8g..8g+7 of all 32 rows, 128 bytes per row; load (g, j), j < 4, covers rows
    // 8j..8j+7 of block g, lane L the row 8j + L/8, slot L%8, which holds chunk
    // 8g + ((L%8) ^ f(row)).  Rows past the sequence end are outside the buffer range
    // and read as zeros.
    const int drow = lane >> 3;
    int dma_voff[2];  // per parity of j: f(8j + L/8) = rev3(4 (j & 1) + L/16)
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
        const int x = 4 * jp + (lane >> 4);
        const int f = ((x & 1) << 2) | (x & 2) | (x >> 2);
        dma_voff[jp] = drow * RB + 16 * ((lane & 7) ^ f);
    }
    auto page_of = [&](int t0) { return __builtin_amdgcn_readfirstlane(p.page_table[t0 >> kPageShift]); };
    typedef U32x4 TileRegs[LDW];
    auto load_tile = [&](int t0, int phys, TileRegs& r) __attribute__((always_inline)) {
        const char* base = p.pool + (static_cast<long long>(phys) * kPageTokens + (t0 & (kPageTokens - 1))) * RB;
        const int bytes = min(kMTile, t_end - t0) * RB;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, bytes, kBufferFlags);
#pragma unroll
        for (int i = 0; i < LDW; ++i) {
            const int n = pw + 4 * i;  // wave-uniform
            const int g = n >> 2, j = n & 3;
            r[i] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, dma_voff[j & 1], 8 * j * RB + 128 * g, 0));
        }
    };
    auto store_tile = [&](const TileRegs& r, char* dst) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < LDW; ++i) {
            const int n = pw + 4 * i;
            const int g = n >> 2, j = n & 3;
            *reinterpret_cast<U32x4*>(dst + BB * g + 1024 * j + 16 * lane) = r[i];
        }
    };
    TileRegs tr0, tr1;  // tiles in flight (PV waves)

    // ---- B operands of QK: lane (q4, l16) of QK wave (kh, ph) = (w / 2, w % 2) holds, for
    // k-step kk of its half and head tile ht, dims 32kk + 8q4 .. +8 of head 16ht + l16,
    // split into hi + lo parts of the cache type
    // (fp16: after the per-head power-of-two scaling).  While the PV waves wait for the
    // first two tiles, the QK waves read q~ of the workgroup's 32 heads once, coalesced,
    // convert it to hi + lo and stage it in tile buffers 1 (hi) and 2 (lo), free until
    // tiles 1 and 2 are stored; then every QK wave reads its operands.  (With all eight
    // waves staging q~ after the PV waves' tile loads, the conversion waited for those
    // loads: 24.2-24.3 vs 23.8-23.9 us per call at C5.)
    // staged rows of one part: W * 2 bytes, 16-byte chunk c of row r at chunk c ^ (r & 7)
    // (W / 8 is a multiple of 8), so the 16 rows of one operand read use distinct banks
    constexpr int QS = W * 2;
    static_assert(kMHeads * QS == TB, "one part of q~ fills one tile buffer");
    if (!qk_wave) {
        load_tile(t_begin, page_of(t_begin), tr0);
    } else {
        // eight threads per head, thread `part` takes float4 columns part, part + 8, ...
        constexpr int NQ = W / 32;
        const int hl = tid >> 3;
        const int part = tid & 7;
        const int head = min(hg * kMHeads + hl, p.heads - 1);  // padding heads are never stored
        float4 v[NQ];
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int d = 4 * (part + 8 * i);
            v[i] = d < KL ? *reinterpret_cast<const float4*>(p.q_tilde + static_cast<size_t>(head) * KL + d)
                          : *reinterpret_cast<const float4*>(p.q_rope + static_cast<size_t>(head) * KR + (d - KL));
        }
        int qexp = 0;
        if (!SRC_BF16) {
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < NQ; ++i)
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
            amax = fmaxf(amax, dpp_xor1(amax));
            amax = fmaxf(amax, dpp_xor2(amax));
            amax = fmaxf(amax, dpp_half_mirror(amax));  // the 8 lanes of the head
            if (amax > 16384.f && amax <= 3.0e38f) qexp = static_cast<int>(ceilf(log2f(amax / 16384.f)));
        }
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const float x[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
            E hi[4], lo[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float y = SRC_BF16 ? x[c] : ldexpf(x[c], -qexp);
                hi[c] = static_cast<E>(y);
                lo[c] = static_cast<E>(y - static_cast<float>(hi[c]));
            }
            const int col = part + 8 * i;  // 8-byte column: chunk col / 2, half col % 2
            const int off = hl * QS + 16 * ((col >> 1) ^ (hl & 7)) + 8 * (col & 1);
            *reinterpret_cast<uint2*>(lds_b1 + off) = __builtin_bit_cast(uint2, hi);
            *reinterpret_cast<uint2*>(lds_b2 + off) = __builtin_bit_cast(uint2, lo);
        }
        if (part == 0) lds_qexp[hl] = qexp;
    }
    if (!qk_wave) {
        // tile 1 is requested only once tile 0 has landed, so tile 0 and q~ -- all that
        // the first scores need -- do not share the CU's load path with it (C5 23.4 vs
        // 23.0 us per call; q~ loaded by each QK wave straight into its operands instead
        // of staged, twice the bytes: 25.7)
        store_tile(tr0, lds_b0);
        if (ntiles > 1) load_tile(t_begin + kMTile, page_of(t_begin + kMTile), tr1);
    }
    lds_barrier();  // q~ staged, tile 0 in LDS

    // ================================================================ QK waves
    if (qk_wave) {
        constexpr int NKH = NK / 2;   // k-steps of a half
        static_assert(NK % 2 == 0, "k halves");
        const int kh = wave >> 1;     // k half: k-steps NKH kh .. NKH kh + NKH - 1
        const int ph = wave & 1;      // position half of the tile
        V qhi[2][NKH], qlo[2][NKH];   // both head tiles
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
            const int hr = 16 * ht + l16;
#pragma unroll
            for (int kk = 0; kk < NKH; ++kk) {
                const int c = (4 * (NKH * kh + kk) + q4) ^ (hr & 7);
                qhi[ht][kk] = *reinterpret_cast<const V*>(lds_b1 + hr * QS + 16 * c);
                qlo[ht][kk] = *reinterpret_cast<const V*>(lds_b2 + hr * QS + 16 * c);
            }
        }
        // A operand of k-step kg: row 16ph + l16, logical chunk 4kg + q4 = block kg/2, slot
        // 4 (kg & 1) + q4, stored at slot (4 (kg & 1) + q4) ^ f = 4 ((kg & 1) ^ (f >> 2)) +
        // (q4 ^ (f & 3)); f depends on l16 only (16ph is a multiple of 16).
        const int rq = 16 * ph + l16;
        const int fq = row_swizzle(rq);
        const int qk_off = rq * 128 + 16 * (q4 ^ (fq & 3));
        const int qk_flip = fq >> 2;
        // raw scores of the tile in `tile` into `sbuf` (the softmax scales and masks)
        auto qk = [&](const char* tile, float* sbuf) __attribute__((always_inline)) {
            f32x4_t sc[2], sl[2];  // hi / lo chains x head tile
#pragma unroll
            for (int e = 0; e < 2; ++e) sc[e] = sl[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            U32x4 ra[NKH];
            auto load = [&](int kk) __attribute__((always_inline)) {
                const int kg = NKH * kh + kk;
                ra[kk] = *reinterpret_cast<const U32x4*>(tile + BB * (kg >> 1) + qk_off + 64 * ((kg & 1) ^ qk_flip));
            };
#pragma unroll
            for (int kk = 0; kk < kQkAhead; ++kk) load(kk);
#pragma unroll
            for (int kk = 0; kk < NKH; ++kk) {
                if (kk + kQkAhead < NKH) load(kk + kQkAhead);
                const V av = __builtin_bit_cast(V, ra[kk]);
                sc[0] = MT::mma(av, qhi[0][kk], sc[0]);
                sc[1] = MT::mma(av, qhi[1][kk], sc[1]);
                sl[0] = MT::mma(av, qlo[0][kk], sl[0]);
                sl[1] = MT::mma(av, qlo[1][kk], sl[1]);
            }
            // lane holds positions 16ph + 4q4 + r of heads 16ht + l16, k half kh
            float* sb = sbuf + kh * kMHeads * kScoreStride;
#pragma unroll
            for (int ht = 0; ht < 2; ++ht)
                *reinterpret_cast<f32x4_t*>(sb + (16 * ht + l16) * kScoreStride + 16 * ph + 4 * q4) = sc[ht] + sl[ht];
        };
        qk(lds_b0, lds_s0);
        lds_barrier();  // q~ read by every QK wave: buffer 1 may be refilled
        lds_barrier();  // scores of tile 0 published, tile 1 in LDS
        // step t: QK of tile t+1 while the PV waves run the softmax of tile t
        for (int t = 0;; t += 6) {
#define QR_QK_STEP(T, NXT, SN)                                   \
            if ((T) + 1 < ntiles) qk(NXT, SN);                   \
            lds_barrier();                                       \
            lds_barrier();                                       \
            if ((T) + 1 >= ntiles) break;
            QR_QK_STEP(t, lds_b1, lds_s1)
            QR_QK_STEP(t + 1, lds_b2, lds_s0)
            QR_QK_STEP(t + 2, lds_b0, lds_s1)
            QR_QK_STEP(t + 3, lds_b1, lds_s0)
            QR_QK_STEP(t + 4, lds_b2, lds_s1)
            QR_QK_STEP(t + 5, lds_b0, lds_s0)
#undef QR_QK_STEP
        }
        if (nsplit == 1) lds_barrier();  // l published
        return;
    }

    // ================================================================ PV waves
    // softmax: PV wave pw owns heads 8pw..8pw+7; lane (lane / 8, i8) holds positions
    // 4 i8 .. 4 i8 + 3 of head hs
    const int hs = 8 * pw + (lane >> 3);
    const int i8 = lane & 7;
    const float sscale = p.qscale * ldexpf(1.f, lds_qexp[hs]);
    float m_s = -INFINITY, l_s = 0.f;  // running max and sum of head hs
    // k-slot of position 4 i8 in the P^T operand order (slots 8q + i: positions 4q + i
    // for i < 4, 16 + 4q + i - 4 otherwise); positions 4 i8 + 1..3 follow it
    const int pslot = i8 < 4 ? 8 * i8 : 8 * (i8 - 4) + 4;
    // PV: half h of the A operand of dim tile dt reads row 16h + 4q4 + l16/4, dims
    // 128pw + 16dt + 4(l16 & 3) .. +4: logical chunk 16pw + 2dt + ((l16 & 3) >> 1) =
    // block 2pw + dt/4, slot 2 (dt & 3) + ((l16 & 3) >> 1), byte 8 (l16 & 1).  f of that
    // row depends on 4q4 + l16/4 only.
    const int rp = 4 * q4 + (l16 >> 2);
    const int fp = row_swizzle(rp);
    const int a4 = l16 & 3;
    const int pv_off = 2 * BB * pw + rp * 128 + 16 * ((a4 >> 1) ^ (fp & 1)) + 8 * (a4 & 1);
    int pv_dt[4];  // slot pair of dt & 3: 2 ((dt & 3) ^ (f >> 1)) chunks
#pragma unroll
    for (int x = 0; x < 4; ++x) pv_dt[x] = 32 * (x ^ (fp >> 1));

    lds_barrier();  // q~ read by every QK wave: buffer 1 may be refilled
    if (ntiles > 1) store_tile(tr1, lds_b1);
    int phys_next = ntiles > 2 ? page_of(t_begin + 2 * kMTile) : 0;
    lds_barrier();  // scores of tile 0 published, tile 1 in LDS

    f32x4_t acc[2][8];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[nt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // Step t: tile t in `cur` with its raw scores in `s_cur`; tile t+2 is loaded now
    // and stored into `dst` (the buffer of tile t-1) after the barrier that publishes P.
    auto step = [&](int t, const char* cur, char* dst, const float* s_cur) __attribute__((always_inline)) {
        const int t0 = t_begin + t * kMTile;
        const bool copy = t + 2 < ntiles;
        if (copy) load_tile(t0 + 2 * kMTile, phys_next, tr0);
        if (t + 3 < ntiles) phys_next = page_of(t0 + 3 * kMTile);

        // ---- softmax of tile t for head hs (only the last tile can be partial)
        {
            const float4 r0 = *reinterpret_cast<const float4*>(s_cur + hs * kScoreStride + 4 * i8);
            const float4 r1 = *reinterpret_cast<const float4*>(s_cur + (kMHeads + hs) * kScoreStride + 4 * i8);
            float v[4] = {(r0.x + r1.x) * sscale, (r0.y + r1.y) * sscale, (r0.z + r1.z) * sscale, (r0.w + r1.w) * sscale};
            if (t0 + kMTile > t_end) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (t0 + 4 * i8 + i >= t_end) v[i] = -INFINITY;
            }
            float tmax = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
            tmax = fmaxf(tmax, dpp_xor1(tmax));
            tmax = fmaxf(tmax, dpp_xor2(tmax));
            tmax = fmaxf(tmax, dpp_half_mirror(tmax));  // the same in the 8 lanes of the head
            // Lazy rescale: the reference m moves only when the tile max exceeds it by
            // more than 2^8, so P = 2^(s - m) <= 256 and the accumulators are rescaled
            // in few tiles.
            const bool grow = tmax > m_s + kRescaleSlack;
            const float corr = grow && m_s != -INFINITY ? fast_exp2(m_s - tmax) : 1.f;
            if (grow) m_s = tmax;
            const float mref = m_s == -INFINITY ? 0.f : m_s;  // masked-only so far: weights 0, not NaN
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = fast_exp2(v[i] - mref);
            l_s = l_s * corr + group_sum((e[0] + e[1]) + (e[2] + e[3]), 8);
            typedef E E4 __attribute__((ext_vector_type(4)));
            E4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                hi[i] = static_cast<E>(e[i]);
                lo[i] = static_cast<E>(e[i] - static_cast<float>(hi[i]));
            }
            *reinterpret_cast<E4*>(lds_p + hs * PR + 2 * pslot) = hi;
            *reinterpret_cast<E4*>(lds_p + (kMHeads + hs) * PR + 2 * pslot) = lo;
            if (i8 == 0) lds_corr[hs] = corr;
        }
        lds_barrier();  // P and the rescale factors of tile t are published

        // ---- PV of tile t over this wave's 128 dims, P^T of heads 16nt + l16 from LDS
        V pb[2], pl[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            pb[nt] = *reinterpret_cast<const V*>(lds_p + (16 * nt + l16) * PR + 16 * q4);
            pl[nt] = *reinterpret_cast<const V*>(lds_p + (kMHeads + 16 * nt + l16) * PR + 16 * q4);
            const float corr = lds_corr[16 * nt + l16];
            if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) acc[nt][dt] *= corr;
            }
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const char* a0 = cur + pv_off + BB * (dt >> 2) + pv_dt[dt & 3];
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
            const u32x2_t lw = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_ptr)(a0)));
            const u32x2_t hw = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_ptr)(a0 + 16 * 128)));
            const V av = __builtin_bit_cast(V, u32x4_t{lw.x, lw.y, hw.x, hw.y});
            acc[0][dt] = MT::mma(av, pb[0], acc[0][dt]);
            acc[1][dt] = MT::mma(av, pb[1], acc[1][dt]);
            acc[0][dt] = MT::mma(av, pl[0], acc[0][dt]);
            acc[1][dt] = MT::mma(av, pl[1], acc[1][dt]);
        }
        if (copy) store_tile(tr0, dst);
        lds_barrier();  // scores of tile t+1 and tile t+2 published; P, tile t free
    };
    for (int t = 0;; t += 6) {
        step(t, lds_b0, lds_b2, lds_s0);
        if (t + 1 >= ntiles) break;
        step(t + 1, lds_b1, lds_b0, lds_s1);
        if (t + 2 >= ntiles) break;
        step(t + 2, lds_b2, lds_b1, lds_s0);
        if (t + 3 >= ntiles) break;
        step(t + 3, lds_b0, lds_b2, lds_s1);
        if (t + 4 >= ntiles) break;
        step(t + 4, lds_b1, lds_b0, lds_s0);
        if (t + 5 >= ntiles) break;
        step(t + 5, lds_b2, lds_b1, lds_s1);
        if (t + 6 >= ntiles) break;
    }

    if (nsplit == 1) {
        // l of heads 16nt + l16, from the lanes that own them
        if (i8 == 0) lds_l[hs] = l_s;
        lds_barrier();  // l published
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int head = hg * kMHeads + 16 * nt + l16;
            if (head >= p.heads) continue;
            float* out = p.u + static_cast<size_t>(head) * KL + 128 * pw + 4 * q4;
            const float inv = 1.f / lds_l[16 * nt + l16];
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                *reinterpret_cast<float4*>(out + 16 * dt) =
                    make_float4(acc[nt][dt][0] * inv, acc[nt][dt][1] * inv, acc[nt][dt][2] * inv, acc[nt][dt][3] * inv);
        }
        return;
    }
    // Split partial: the unnormalised accumulators, stored as fp16 acc / 2^e with e per
    // (head, split, this wave's 128 dims) such that the block's largest |acc| lands in
    // [2^14, 2^15): no overflow and full fp16 precision whatever the latent's range.  The
    // wave assembles its 32 head segments (256 bytes each) in its own part of a tile
    // buffer no step uses any more (the buffer after the last tile's), so the epilogue
    // needs no workgroup barrier: every wave store then writes four whole segments.
    // Two tile buffers are free once the last step begins (the buffers of the two tiles
    // after the last): waves 0-1 stage in one, waves 2-3 in the other.
    // (m, l) of each head come from the softmax lanes that own them.
    {
        const int head = hg * kMHeads + hs;
        if (i8 == 0 && head < p.heads)
            p.part_ml[static_cast<size_t>(head) * p.splits + split] = make_float2(m_s, l_s);
    }
    constexpr int SRW = 256 + 16;  // staged segment pitch (bytes)
    static_assert(2 * kMHeads * SRW <= TB, "two waves' staged segments fit in one tile buffer");
    const int fb = (ntiles + (pw >> 1)) % 3;  // tile t's buffer is t % 3
    char* stage = (fb == 0 ? lds_b0 : fb == 1 ? lds_b1 : lds_b2) + (pw & 1) * kMHeads * SRW;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float amax = 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) amax = fmaxf(amax, fabsf(acc[nt][dt][r]));
        amax = max_xor32(max_xor16(amax));
        // e = floor(log2(amax)) - 14 for finite non-zero amax (subnormals included),
        // at least -128 (values below 2^-114 then still land above fp16's subnormals)
        const int e = amax > 0.f && amax <= 3.4e38f ? max(ilogbf(amax) - 14, -128) : 0;
        const int hl = 16 * nt + l16;
        const int head = hg * kMHeads + hl;
        if (q4 == 0 && head < p.heads)
            p.part_e[(static_cast<size_t>(head) * p.splits + split) * 4 + pw] = static_cast<signed char>(e);
        char* row = stage + hl * SRW;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            typedef float f32x2_t __attribute__((ext_vector_type(2)));
            typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
            const f16x2_t lo = __builtin_convertvector(f32x2_t{ldexpf(acc[nt][dt][0], -e), ldexpf(acc[nt][dt][1], -e)}, f16x2_t);
            const f16x2_t hi = __builtin_convertvector(f32x2_t{ldexpf(acc[nt][dt][2], -e), ldexpf(acc[nt][dt][3], -e)}, f16x2_t);
            *reinterpret_cast<uint2*>(row + 2 * (16 * dt + 4 * q4)) =
                make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // store i: segments of heads 4i .. 4i + 3, lane j the 16 bytes at 16 (j % 16) of head
    // 4i + j / 16, written through to device scope (sc1)
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < kMHeads / 4; ++i) {
        const int hl = 4 * i + (lane >> 4);
        const int head = hg * kMHeads + hl;
        const U32x4 v = *reinterpret_cast<const U32x4*>(stage + hl * SRW + 16 * (lane & 15));
        if (head < p.heads) {
            char* seg = static_cast<char*>(p.part_u) + ((static_cast<size_t>(head) * p.splits + split) * KL + 128 * pw) * 2;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(seg, 0, 256, kBufferFlags);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, v), rs, 16 * (lane & 15), 0, kCacheSc1);
        }
    }
}

// Split merge for the MFMA path: one workgroup per (head, 64-dim block); thread (grp, c8)
// owns 8 dims (one 16-byte load of fp16 partials per split) and splits grp, grp + 32, ...,
// all loads of a batch issued at once (in range: a repeated split weighs zero); split s
// weighs 2^(m_s - M), its stored values 2^(e of their 128-dim block), its sum l_s
// 2^(m_s - M) goes to the denominator.  The 32 split groups are merged
// through LDS.  (Against one workgroup per 128-dim block with 8-byte loads: C5 24.4 vs
// 25.1 us per call.)
__global__ void __launch_bounds__(256) mla_combine_wide_kernel(const MlaMK p) {
    constexpr int KL = kMfmaLora;
    const int h = blockIdx.x;
    const int blk = blockIdx.y;             // 64-dim block
    const int c8 = threadIdx.x & 7;         // 8-dim column inside the block
    const int grp = threadIdx.x >> 3;       // 32 split groups
    const size_t base = static_cast<size_t>(h) * p.splits;
    const int d = blk * 64 + c8 * 8;
    const _Float16* part = static_cast<const _Float16*>(p.part_u);
    const int seq = device_seq(p.pos_dev, p.seq_len);
    const int split_tokens = mla_split_tokens(p, seq);
    const int nsplit = (seq + split_tokens - 1) / split_tokens;
    if (nsplit == 1) return;  // the tile kernel wrote u
    float m = -INFINITY, l = 0.f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    constexpr int kB = 4;
    const int eb = blk >> 1;  // 128-dim block of the exponent
    for (int s0 = grp; s0 < nsplit; s0 += 32 * kB) {
        uint4 a[kB];
        float2 ml[kB];
        int ex[kB];
#pragma unroll
        for (int i = 0; i < kB; ++i) {
            const int s = min(s0 + 32 * i, nsplit - 1);
            a[i] = *reinterpret_cast<const uint4*>(part + (base + s) * KL + d);
            ml[i] = p.part_ml[base + s];
            ex[i] = p.part_e[(base + s) * 4 + eb];
        }
        float mb = m;
#pragma unroll
        for (int i = 0; i < kB; ++i) {
            if (s0 + 32 * i >= nsplit) ml[i] = make_float2(-INFINITY, 0.f);
            mb = fmaxf(mb, ml[i].x);
        }
        const float cm = m == -INFINITY ? 0.f : fast_exp2(m - mb);
        l *= cm;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] *= cm;
#pragma unroll
        for (int i = 0; i < kB; ++i) {
            const float w = ml[i].x == -INFINITY ? 0.f : fast_exp2(ml[i].x - mb);
            const float wv = ldexpf(w, ex[i]);  // weight of the stored values
            typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
            const h8_t v = __builtin_bit_cast(h8_t, a[i]);
            l = fmaf(ml[i].y, w, l);
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = fmaf(static_cast<float>(v[k]), wv, o[k]);
        }
        m = mb;
    }
    __shared__ float rm[256], rl[256];
    __shared__ float ro[8][257];
    rm[threadIdx.x] = m;
    rl[threadIdx.x] = l;
#pragma unroll
    for (int k = 0; k < 8; ++k) ro[k][threadIdx.x] = o[k];
    __syncthreads();
    if (threadIdx.x < 64) {  // dim k of column cc
        const int cc = threadIdx.x & 7, k = threadIdx.x >> 3;
        float M = -INFINITY;
        for (int g = 0; g < 32; ++g) M = fmaxf(M, rm[g * 8 + cc]);
        float L = 0.f, t = 0.f;
        for (int g = 0; g < 32; ++g) {
            const int r = g * 8 + cc;
            const float c = rm[r] == -INFINITY ? 0.f : fast_exp2(rm[r] - M);
            L = fmaf(rl[r], c, L);
            t = fmaf(ro[k][r], c, t);
        }
        p.u[static_cast<size_t>(h) * KL + blk * 64 + cc * 8 + k] = t / L;
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

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

}  // namespace

MlaPlan plan_mla(const MlaArgs& a) {
    MlaPlan pl{};
    size_t q_copy = 0;
    if (mfma_eligible(a)) {
        // about one workgroup per CU: (32-head group) x split, splits of whole 64-position tiles
        const int groups = (a.heads + kMHeads - 1) / kMHeads;
        const int tiles = (a.seq_len + kMTile - 1) / kMTile;
        int want = std::max(1, cus() / groups);
        want = std::min(want, tiles);
        const int tiles_per_split = (tiles + want - 1) / want;
        pl.split_tokens = tiles_per_split * kMTile;
        // room for 16-byte aligned copies of q~ / q_rope when the caller's are not
        q_copy = align256(static_cast<size_t>(a.heads) * a.kv_lora * 4) + align256(static_cast<size_t>(a.heads) * a.rope * 4);
    } else {
        pl.split_tokens = kGenericSplit;
    }
    pl.splits = (a.seq_len + pl.split_tokens - 1) / pl.split_tokens;
    const size_t slots = static_cast<size_t>(a.heads) * pl.splits;
    const size_t part_elem = mfma_eligible(a) ? 2 : 4;   // fp16 partials on the MFMA path
    const size_t ml_bytes = 8;                          // (m, l)
    const size_t e_bytes = mfma_eligible(a) ? align256(slots * 4) : 0;  // exponents of the fp16 partials
    pl.workspace_bytes = (pl.splits > 1 ? align256(slots * a.kv_lora * part_elem) + align256(slots * ml_bytes) + e_bytes : 0) + q_copy;
    return pl;
}

namespace {
template <bool SRC_BF16, int KR>
hipError_t launch_tile(const MlaMK& k, hipStream_t stream) {
    hipLaunchKernelGGL((mla_tile_kernel<SRC_BF16, KR>), dim3(8 * k.per_xcd), dim3(kMWaves * 64), 0, stream, k);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_mla(const MlaArgs& a, const MlaPlan& pl, void* workspace, hipStream_t stream) {
    if (pl.splits > 4096) return hipErrorInvalidValue;
    const size_t slots = static_cast<size_t>(a.heads) * pl.splits;
    char* ws = static_cast<char*>(workspace);
    if (mfma_eligible(a)) {
        MlaMK k{};
        k.pool = static_cast<const char*>(a.pool);
        k.page_table = a.page_table;
        k.heads = a.heads;
        k.seq_len = a.seq_len;
        k.pos_dev = a.pos_dev;
        k.split_tokens = pl.split_tokens;
        k.splits = pl.splits;
        k.groups = (a.heads + kMHeads - 1) / kMHeads;
        k.per_xcd = (k.groups * pl.splits + 7) / 8;
        k.u = a.u;
        const size_t part_bytes = pl.splits > 1 ? align256(slots * a.kv_lora * 2) + align256(slots * 8) + align256(slots * 4) : 0;
        k.part_u = ws;
        k.part_ml = reinterpret_cast<float2*>(ws + align256(slots * a.kv_lora * 2));
        k.part_e = reinterpret_cast<signed char*>(ws + align256(slots * a.kv_lora * 2) + align256(slots * 8));
        // the kernel reads q~ / q_rope as float4
        k.q_tilde = a.q_tilde;
        k.q_rope = a.q_rope;
        const bool misaligned = (reinterpret_cast<uintptr_t>(a.q_tilde) | reinterpret_cast<uintptr_t>(a.q_rope)) & 15;
        if (misaligned) {
            float* qt = reinterpret_cast<float*>(ws + part_bytes);
            float* qr = reinterpret_cast<float*>(ws + part_bytes + align256(static_cast<size_t>(a.heads) * a.kv_lora * 4));
            hipError_t e = hipMemcpyAsync(qt, a.q_tilde, static_cast<size_t>(a.heads) * a.kv_lora * 4, hipMemcpyDeviceToDevice, stream);
            if (e == hipSuccess && a.rope)
                e = hipMemcpyAsync(qr, a.q_rope, static_cast<size_t>(a.heads) * a.rope * 4, hipMemcpyDeviceToDevice, stream);
            if (e != hipSuccess) return e;
            k.q_tilde = qt;
            k.q_rope = a.rope ? qr : nullptr;
        }
        k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
        hipError_t e;
        const bool bf = a.dtype == QR_DTYPE_BF16;
        if (a.rope) e = bf ? launch_tile<true, 64>(k, stream) : launch_tile<false, 64>(k, stream);
        else e = bf ? launch_tile<true, 0>(k, stream) : launch_tile<false, 0>(k, stream);
        if (e != hipSuccess || pl.splits == 1) return e;
        hipLaunchKernelGGL(mla_combine_wide_kernel, dim3(a.heads, kMfmaLora / 64), dim3(256), 0, stream, k);
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
    k.pos_dev = a.pos_dev;
    k.split_tokens = pl.split_tokens;
    k.splits = pl.splits;
    k.q_tilde = a.q_tilde;
    k.q_rope = a.q_rope;
    k.u = a.u;
    k.part_u = reinterpret_cast<float*>(ws);
    k.part_ml = reinterpret_cast<float2*>(ws + align256(slots * a.kv_lora * 4));
    k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
    hipLaunchKernelGGL(mla_split_generic_kernel, dim3(pl.splits, a.heads), dim3(kThreads), 0, stream, k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.splits == 1) return e;
    hipLaunchKernelGGL(mla_combine_kernel, dim3(a.heads), dim3(kThreads), 0, stream, k);
    return hipGetLastError();
}

}  // namespace qr
