// qr_chunk.hip -- causal multi-query attention over the paged cache on MFMA tiles
// (chunked prefill and speculative verify), gfx950.
//
// Semantics: query i of the chunk sits at position pos0+i and attends positions
// 0..pos0+i, which is what nq sequential PagedKvCache.Attention calls with
// interleaved appends compute (StreamingEngine.cs:831-836, SpeculativeRunner.cs:85-93).
//
// A row is one (query, query head) pair; the G = heads/kv_heads heads of one kv
// head and a block of consecutive queries form the rows of a workgroup, so every
// K/V tile staged in LDS serves them all.  Workgroup = 4 row groups of NT x 16 rows; at
// NT >= 2 one wave per row group scores every position of a tile; at NT = 1 (a few
// queries, e.g. speculative verify) two waves per row group take one half of the tile's
// positions each, so that every SIMD runs two waves, and the halves merge once at the end.
// Waves never exchange data inside a tile.
//   QK: S^T[pos][row] = K[pos][dims] . Q^T[dims][row]     (M positions, N rows)
//   PV: O^T[dim][row] += V^T[dim][pos] . P^T[pos][row]     (M dims,      N rows)
// Tiles of 64 positions -- two steps of the MFMA operand page layout (qr_kernels.hpp) --
// are copied into LDS by buffer-load DMA as they lie in the page, NSTAGE-buffered, so
// every MFMA operand is a contiguous 1 KiB of LDS that a wave reads conflict-free, 16
// bytes per lane, and every DMA wave load covers whole 128-byte lines.  QK row m of M
// tile mt is position 32(mt/2) + 8(m/4) + 4(mt%2) + m%4 (the page layout's K operand
// order), so after QK lane quarter q holds the scores of positions 32ks + 8q .. +7, its
// PV k-slots of step ks.
// Operands stay in the cache's 16-bit type (no conversion); q enters as hi + lo parts
// when its own type is not the cache's (fp32 queries keep ~22 or ~16 bits), P is
// rounded to the cache type; accumulation and softmax are fp32.  Row sums come from
// the MFMA too (a ones operand), consistent with the rounded P of the numerator.
// The causal mask is applied only on tiles that reach past the block's first query.
#include "qr_chunk.hpp"
#include "qr_mfma.hpp"

#include <algorithm>

namespace qr {
namespace {

constexpr int kTile = 64;  // positions per tile
#ifndef QR_CHUNK_MAX_NT
#define QR_CHUNK_MAX_NT 2
#endif

// Elements 32kk + 8q4 + i (kk < NK, i < 8) of the q row starting at element `row`, as fp32.
// The dtype branch sits outside the loads, so all of them are issued before the first is
// used (one wait) -- a per-element switch made every load wait for all loads in flight.
// Element loads: the caller's q needs only element alignment.
template <int NK>
__device__ __forceinline__ void load_q_slices(const void* q, int dtype, size_t row, int q4, float (&x)[NK][8]) {
    if (dtype == QR_DTYPE_F32) {
        const float* f = static_cast<const float*>(q) + row;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[kk][i] = f[32 * kk + 8 * q4 + i];
    } else {
        const uint16_t* h = static_cast<const uint16_t*>(q) + row;
        uint16_t u[NK][8];
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int i = 0; i < 8; ++i) u[kk][i] = h[32 * kk + 8 * q4 + i];
        const bool bf = dtype == QR_DTYPE_BF16;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[kk][i] = bf ? bf16_bits_to_f32(u[kk][i]) : f16_bits_to_f32(u[kk][i]);
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
    const int* pos0_dev;     // device position of query 0 (clamped to [0, pos0]) when set
    int nq;
    int q_dtype;
    const void* q;           // [nq][heads][D]
    float* out;              // [nq][heads][D]
    float* part_acc;         // [nq*heads][splits][D]
    float2* part_ml;         // [nq*heads][splits]
    float qscale;            // scale * log2(e)
    int queries_per_block;
    int split_tokens;        // multiple of kTile
    int splits;
    int qblocks;
    int units;               // splits x qblocks x kv_heads
    int per_xcd;             // launch slots per XCD: ceil(units / 8)
    int kv_once;             // one query block: each K/V line is read once per call
};

// Position of query 0: the argument, or the device-side one bounded by it (a scalar load:
// no kernel here writes it).
__device__ __forceinline__ int chunk_pos0(const ChunkK& p) {
    if (!p.pos0_dev) return p.pos0;
    const int v = reinterpret_cast<const __attribute__((address_space(4))) int*>(
        reinterpret_cast<uintptr_t>(p.pos0_dev))[0];
    return __builtin_amdgcn_readfirstlane(min(max(v, 0), p.pos0));
}

// Keys per split: the plan's; with a device position (the plan was made for the bound)
// the keys of the last query spread over the planned splits, whole tiles per split.
__device__ __forceinline__ int chunk_split_tokens(const ChunkK& p, int pos0) {
    if (!p.pos0_dev) return p.split_tokens;
    const int tiles = (pos0 + p.nq + kTile - 1) / kTile;
    return (tiles + p.splits - 1) / p.splits * kTile;
}

// Row maxima of the scores in v_max3_f32 / v_max_f32.  The scores come straight from the
// MFMAs, so the quieting of signalling NaNs that fmaxf implies (one extra v_max per
// operand, half the VALU of the max) is not needed: a NaN score still reaches its row's
// output through P.
__device__ __forceinline__ float max3f(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max2f(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// max over the four lane quarters of a row (lanes l ^ 16, l ^ 32)
__device__ __forceinline__ float max_quarters(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// BF16: cache element type; NT: 16-row N tiles per wave; NSTAGE: LDS tile buffers;
// QSPLIT: q is not exact in the cache type and enters as hi + lo parts.
template <bool BF16, int D, int NT, int NSTAGE, bool QSPLIT>
// Workgroups per CU: two at NT <= 2 with two LDS stages (64 KiB); one with three stages
// (96 KiB of LDS) or NT = 4 (registers).  NT = 1 runs eight waves per workgroup.
__global__ void __launch_bounds__(NT == 1 ? 512 : 256, NT <= 2 && NSTAGE <= 2 ? 2 : 1) chunk_tile_kernel(const ChunkK p) {
    using T = typename std::conditional<BF16, __bf16, _Float16>::type;
    typedef T vec8 __attribute__((ext_vector_type(8)));
    constexpr int NK = D / 32;               // QK k-steps
    constexpr int NDT = D / 16;              // PV dim tiles
    constexpr int RB = D * 2;                // K row bytes
    constexpr int KB = kTile * RB;           // K tile bytes
    constexpr int VB = D * kTile * 2;        // V^T tile bytes (D rows of 128 bytes)
    constexpr bool PS = NT == 1;             // position halves: two waves per row group
    constexpr int WAVES = PS ? 8 : 4;
    constexpr int NMT = PS ? 2 : 4;          // QK M tiles (16 positions) per wave and tile
    constexpr int NKS = PS ? 1 : 2;          // PV k-steps (32 positions) per wave and tile
    constexpr int KI = KB / 1024 / WAVES;    // K DMA instructions per wave and tile
    constexpr int VI = VB / 1024 / WAVES;    // V DMA instructions per wave and tile
    constexpr int PER_TILE = KI + VI;        // vector-memory ops per wave and tile
    static_assert(KI >= 1 && VI >= 1, "tile must split over the waves");

    __shared__ __attribute__((aligned(1024))) char lds[NSTAGE][KB + VB];

    // Launch slot b runs on XCD b % 8 (round-robin dispatch); XCD x takes the contiguous
    // logical units [x per_xcd, (x + 1) per_xcd), ordered split fastest, then query
    // block, then kv head, so the query blocks of one kv head share one XCD and its L2
    // keeps that kv head's K/V (4 MB at 8192 positions, head_dim 128) instead of every
    // L2 cycling through all kv heads.  The first half of a kv head's run takes its query
    // blocks from the last (most keys under the causal mask) down, the second half from
    // the first up: with two workgroups per CU resident at once, launch slots b and
    // b + 256 run on one CU (the XCD's k-th and (k + 32)-th workgroups; measured with a
    // probe of the hardware CU ids, the same on every launch), so the pair sums to about
    // the same keys (2048 queries after 6144 positions: 255 us per call against 263 with
    // all blocks descending).
    const int bslot = blockIdx.x;
    const int unit = (bslot & 7) * p.per_xcd + (bslot >> 3);
    if (unit >= p.units) return;
    const int split = unit % p.splits;
    const int uq = (unit / p.splits) % p.qblocks;
    const int hq = (p.qblocks + 1) >> 1;
    const int qblk = uq < hq ? p.qblocks - 1 - uq : uq - hq;
    const int kvh = unit / (p.splits * p.qblocks);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & (WAVES - 1);
    const int rw = PS ? (wave & 3) : wave;  // row group
    const int ph = PS ? (wave >> 2) : 0;    // position half (NT = 1): the tile's step ph
    const int q4 = lane >> 4;
    const int col = lane & 15;

    // rows of this lane, one per N tile: (query, head) = (rho >> log2 G, rho & (G - 1))
    const int q_first = qblk * p.queries_per_block;
    int row_q[NT], row_h[NT];
    bool row_on[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int rho = rw * 16 * NT + j * 16 + col;
        row_q[j] = q_first + (rho >> p.group_shift);
        row_h[j] = kvh * p.group + (rho & (p.group - 1));
        row_on[j] = row_q[j] < p.nq && (rho >> p.group_shift) < p.queries_per_block;
    }
    const int q_last = min(p.nq, q_first + p.queries_per_block) - 1;
    const int pos0 = chunk_pos0(p);
    const int split_tokens = chunk_split_tokens(p, pos0);
    const int t_begin = split * split_tokens;
    const int t_end = min(t_begin + split_tokens, pos0 + q_last + 1);  // causal bound of the block
    const int ntiles = t_end > t_begin ? (t_end - t_begin + kTile - 1) / kTile : 0;
    const int unmasked_end = pos0 + q_first + 1;  // positions below it are seen by every row

    // ---- DMA of tile `it` into stage it % NSTAGE: the tile's two steps of K, then of V,
    // contiguous in the page, copied as they lie (1 KiB per wave load).  Positions past
    // the end are masked out of the scores (K) or cleared after they land (V, last tile
    // only), so a zero weight never meets a stale row.
    const long long kblk = static_cast<long long>(kvh) * kPageTokens * D;
    const uint32_t lane16 = static_cast<uint32_t>(16 * lane);
    // Page-table entry of tile `it`: a scalar load through the constant address space (no
    // kernel writes the table while this one runs), fetched one tile before its DMA is
    // issued.  As a vector load it needed a vmcnt(0) before its readfirstlane, which
    // drained the tile DMA still in flight on every iteration.
    auto page_entry = [&](int it) {
        return reinterpret_cast<const __attribute__((address_space(4))) int*>(
            reinterpret_cast<uintptr_t>(p.page_table))[(t_begin + it * kTile) >> kPageShift];
    };
    auto dma = [&](int it, int phys_entry) {
        const int t0 = t_begin + it * kTile;
        const long long phys = phys_entry;
        const int slot0 = t0 & (kPageTokens - 1);
        char* dst = lds[it % NSTAGE];
        const char* kbase = p.pool + (phys * p.page_elems + kblk + static_cast<long long>(slot0) * D) * 2;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kbase), 0, KB, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(kbase + p.plane_elems * 2), 0, VB, kBufferFlags);
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int n = wave + WAVES * i;
            if (p.kv_once) buffer_load_lds16<kCacheNt>(rk, dst + 1024 * n, lane16, 1024 * n);
            else buffer_load_lds16(rk, dst + 1024 * n, lane16, 1024 * n);
        }
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int n = wave + WAVES * i;
            if (p.kv_once) buffer_load_lds16<kCacheNt>(rv, dst + KB + 1024 * n, lane16, 1024 * n);
            else buffer_load_lds16(rv, dst + KB + 1024 * n, lane16, 1024 * n);
        }
    };

    // ---- q rows as B operands (dims 32kk + 8q4 .. +8), scaled per row by a power of two
    // so that fp16 cannot overflow; log2-unit score scale per row
    vec8 qhi[NT][NK], qlo[NT][NK];
    float sscale[NT];
    if (ntiles > 0) dma(0, page_entry(0));
    if (NSTAGE > 2 && ntiles > 1) dma(1, page_entry(1));
    int phys_pf = NSTAGE - 1 < ntiles ? page_entry(NSTAGE - 1) : 0;  // the next DMA's page
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const size_t qrow = (static_cast<size_t>(row_on[j] ? row_q[j] : 0) * p.heads + row_h[j]) * D;
        float x[NK][8];
        load_q_slices<NK>(p.q, p.q_dtype, qrow, q4, x);
        float amax = 0.f;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[kk][i]));
        amax = max_xor16(amax);
        amax = max_xor32(amax);
        int qexp = 0;
        if (!BF16 && amax > 16384.f && amax <= 3.0e38f) qexp = static_cast<int>(ceilf(log2f(amax / 16384.f)));
        const float down = ldexpf(1.f, -qexp);
        sscale[j] = p.qscale * ldexpf(1.f, qexp);
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float v = x[kk][i] * down;
                const T hi = static_cast<T>(v);
                qhi[j][kk][i] = hi;
                if (QSPLIT) qlo[j][kk][i] = static_cast<T>(v - static_cast<float>(hi));
            }
    }
    vec8 ones;
#pragma unroll
    for (int i = 0; i < 8; ++i) ones[i] = static_cast<T>(1.f);

    f32x4_t acc[NT][NDT], accl[NT];
    float m[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        m[j] = -INFINITY;
        accl[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NDT; ++t) acc[j][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // QK row m of M tile mt is position 32(mt/2) + 8(m/4) + 4(mt%2) + m%4, so lane quarter
    // q4 ends with positions 32ks + 8q4 .. +7: its PV k-slots of step ks in order.  In LDS
    // a step is SB bytes: K operand (mt % 2, kk) at 1024 ((mt % 2) NK + kk), V operand dt
    // at 1024 dt, lane L's 16 bytes at 16 L.
    constexpr int SB = 64 * D;

    for (int it = 0; it < ntiles; ++it) {
        const int t0 = t_begin + it * kTile;
        // tile `it` landed (the tiles after it stay in flight); the stage refilled next
        // was consumed in the previous iteration
        if (NSTAGE > 2 && it + 1 < ntiles) wait_vmcnt<PER_TILE>();
        else wait_dma();
        lds_barrier();
        if (it + NSTAGE - 1 < ntiles) {
            dma(it + NSTAGE - 1, phys_pf);
            if (it + NSTAGE < ntiles) phys_pf = page_entry(it + NSTAGE);
        }
        const char* kt = lds[it % NSTAGE];
        const char* vt = kt + KB;
        const int nvalid = min(kTile, t_end - t0);
        if (nvalid < kTile) {
            // the last tile: clear V past the end.  16-byte chunk c of the V tile (step
            // c / (NDT 64), dim tile, lane L = c % 64) holds positions 32 step + 8 (L / 16)
            // .. + 7 of one dim.
            for (int c = threadIdx.x; c < 2 * NDT * 64; c += 64 * WAVES) {
                const int pb = 32 * (c / (NDT * 64)) + 8 * ((c & 63) >> 4);
                if (pb + 8 <= nvalid) continue;
                uint32_t* w = reinterpret_cast<uint32_t*>(const_cast<char*>(vt) + 16 * c);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (pb + i >= nvalid) w[i >> 1] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
            }
            lds_barrier();
        }

        // ---- QK (M tiles mt0 .. mt0 + NMT - 1 of the tile)
        const int mt0 = PS ? 2 * ph : 0;
        f32x4_t sc[NT][NMT];
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int lm = 0; lm < NMT; ++lm) sc[j][lm] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        // The K operands of M tile mt+1 are read before the MFMAs of M tile mt (scheduling
        // barriers keep the compiler from sinking each read next to its first use, where
        // every MFMA pair waited out an LDS round trip).
        {
            vec8 ka[2][NK];
            auto kread = [&](int mt, vec8 (&dst)[NK]) __attribute__((always_inline)) {
                const char* op = kt + SB * (mt >> 1) + 1024 * NK * (mt & 1) + 16 * lane;
#pragma unroll
                for (int kk = 0; kk < NK; ++kk) dst[kk] = *reinterpret_cast<const vec8*>(op + 1024 * kk);
            };
            kread(mt0, ka[0]);
#pragma unroll
            for (int lm = 0; lm < NMT; ++lm) {
                if (lm + 1 < NMT) kread(mt0 + lm + 1, ka[(lm + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int kk = 0; kk < NK; ++kk)
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        sc[j][lm] = mfma16(ka[lm & 1][kk], qhi[j][kk], sc[j][lm]);
                        if (QSPLIT) sc[j][lm] = mfma16(ka[lm & 1][kk], qlo[j][kk], sc[j][lm]);
                    }
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // ---- causal mask and sequence end, only on tiles that reach past the block's
        // first query or the end (wave-uniform, one or two tiles per workgroup)
        if (t0 + kTile > unmasked_end || t0 + kTile > t_end) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int lim = min(t_end - 1, pos0 + row_q[j]);  // last position row j sees
#pragma unroll
                for (int lm = 0; lm < NMT; ++lm)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int mt = mt0 + lm;
                        const int tok = t0 + 32 * (mt >> 1) + 8 * q4 + 4 * (mt & 1) + r;
                        sc[j][lm][r] = tok <= lim ? sc[j][lm][r] : -INFINITY;
                    }
            }
        }

        // ---- online softmax per row: lazy rescale (m moves when the tile max exceeds it
        // by more than 2^8, so P <= 256), one wave-uniform check for all rows of the lane
        float ts[NT];
        bool grow[NT];
        bool any_rescale = false;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            // the lane's 16 scores: five v_max3 over 15 of them, two more over those five
            // and the last, one v_max (8 scores at NT = 1: three v_max3, one v_max); then
            // the other lane quarters
            float tmax;
            if constexpr (NMT == 4) {
                const float a0 = max3f(sc[j][0][0], sc[j][0][1], sc[j][0][2]);
                const float a1 = max3f(sc[j][0][3], sc[j][1][0], sc[j][1][1]);
                const float a2 = max3f(sc[j][1][2], sc[j][1][3], sc[j][2][0]);
                const float a3 = max3f(sc[j][2][1], sc[j][2][2], sc[j][2][3]);
                const float a4 = max3f(sc[j][3][0], sc[j][3][1], sc[j][3][2]);
                tmax = max_quarters(max2f(max3f(a0, a1, a2), max3f(a3, a4, sc[j][3][3])));
            } else {
                const float a0 = max3f(sc[j][0][0], sc[j][0][1], sc[j][0][2]);
                const float a1 = max3f(sc[j][0][3], sc[j][1][0], sc[j][1][1]);
                tmax = max_quarters(max3f(a0, a1, max2f(sc[j][1][2], sc[j][1][3])));
            }
            ts[j] = tmax * sscale[j];
            grow[j] = ts[j] > m[j] + 8.f;
            any_rescale |= grow[j] && m[j] != -INFINITY;
        }
        if (__builtin_amdgcn_ballot_w64(any_rescale)) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const float corr = grow[j] && m[j] != -INFINITY ? fast_exp2(m[j] - ts[j]) : 1.f;
                accl[j] *= corr;
#pragma unroll
                for (int t = 0; t < NDT; ++t) acc[j][t] *= corr;
            }
        }
        vec8 pb[NT][NKS];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            if (grow[j]) m[j] = ts[j];
            const float mneg = m[j] == -INFINITY ? 0.f : -m[j];
#pragma unroll
            for (int lm = 0; lm < NMT; ++lm)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    pb[j][lm >> 1][4 * (lm & 1) + r] = static_cast<T>(fast_exp2(fmaf(sc[j][lm][r], sscale[j], mneg)));
        }

        // ---- PV (and the row sums: a ones operand turns the MFMA into sum over positions).
        // Every V^T operand of a k-slot half is read before its MFMAs (a scheduling barrier
        // keeps the reads ahead), so the later reads land while the first MFMAs run.
#pragma unroll
        for (int kq = 0; kq < NKS; ++kq) {
            const int ks = PS ? ph : kq;
            vec8 va[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                va[dt] = *reinterpret_cast<const vec8*>(vt + SB * ks + 1024 * dt + 16 * lane);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NT; ++j) accl[j] = mfma16(ones, pb[j][kq], accl[j]);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[j][dt] = mfma16(va[dt], pb[j][kq], acc[j][dt]);
        }
    }

    if constexpr (PS) {
        // The position halves of each row group merge: waves 4-7 hand (m, l, o) to waves
        // 0-3 through LDS stages 0 and 1 (free once every wave is past the last tile), lane
        // for lane in the accumulators' own layout.  (The tile buffers stay the kernel's
        // only LDS object: with a second one the compiler waited for every tile copy in
        // flight before each tile's first operand read.)
        static_assert(NSTAGE >= 2 && 4 * NDT * 64 * 16 <= KB + VB, "the handed-over rows fit stage 0");
        f32x4_t* xo = reinterpret_cast<f32x4_t*>(lds[0]) + (rw * NDT) * 64 + lane;
        float* xm = reinterpret_cast<float*>(lds[1]) + rw * 64 + lane;  // [4][64], then l
        float* xl = xm + 4 * 64;
        lds_barrier();
        if (ph == 1) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) xo[dt * 64] = acc[0][dt];
            *xm = m[0];
            *xl = accl[0][0];
        }
        lds_barrier();
        if (ph == 1) return;
        const float m1 = *xm;
        const float M = fmaxf(m[0], m1);
        const float c0 = m[0] == -INFINITY ? 0.f : fast_exp2(m[0] - M);
        const float c1 = m1 == -INFINITY ? 0.f : fast_exp2(m1 - M);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[0][dt] = acc[0][dt] * c0 + xo[dt * 64] * c1;
        accl[0][0] = accl[0][0] * c0 + *xl * c1;
        m[0] = M;
    }

#pragma unroll
    for (int j = 0; j < NT; ++j) {
        if (!row_on[j]) continue;
        const float l = accl[j][0];
        const size_t r = static_cast<size_t>(row_q[j]) * p.heads + row_h[j];
        if (p.splits == 1) {
            float* o = p.out + r * D;
            const float inv = 1.f / l;
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
            if (q4 == 0) p.part_ml[slot] = make_float2(m[j], l);
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

template <bool BF, int D, int NT, int NSTAGE>
hipError_t launch_q(const ChunkK& k, bool qsplit, dim3 grid, hipStream_t s) {
    if constexpr (NT == 4 && D == 128) {  // hi + lo queries there would spill: the plan never asks
        if (qsplit) return hipErrorInvalidValue;
    } else {
        if (qsplit) {
            hipLaunchKernelGGL((chunk_tile_kernel<BF, D, NT, NSTAGE, true>), grid, dim3(NT == 1 ? 512 : 256), 0, s, k);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((chunk_tile_kernel<BF, D, NT, NSTAGE, false>), grid, dim3(NT == 1 ? 512 : 256), 0, s, k);
    return hipGetLastError();
}

// NT 4 and 2 (prefill-sized query blocks) are MFMA-bound and double buffer; NT 1 (a
// few queries, e.g. speculative verify) streams the cache and keeps three tiles in LDS.
template <bool BF, int D>
hipError_t launch_nt(const ChunkK& k, int nt, bool qsplit, dim3 grid, hipStream_t s) {
    switch (nt) {
        case 1: return launch_q<BF, D, 1, 3>(k, qsplit, grid, s);
        case 2: return launch_q<BF, D, 2, 2>(k, qsplit, grid, s);
        default: return launch_q<BF, D, 4, 2>(k, qsplit, grid, s);
    }
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
    // (hi + lo queries at head_dim 128 need the registers of two N tiles)
    int nt = QR_CHUNK_MAX_NT;
    while (nt > 1 && (64 * nt) / g > std::max(1, a.nq)) nt >>= 1;
    pl.nt = nt;
    pl.queries_per_block = std::max(1, 64 * nt / g);
    const int qblocks = (a.nq + pl.queries_per_block - 1) / pl.queries_per_block;
    const int units = qblocks * a.geom.kv_heads;
    // split the keys when there are too few (query block, kv head) units to fill the GPU
    int splits = 1;
    if (units < cu_total()) splits = std::min((cu_total() + units - 1) / units, (total + kTile - 1) / kTile);
    int split_tokens = ((total + splits - 1) / splits + kTile - 1) / kTile * kTile;
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
    k.pos0_dev = a.pos0_dev;
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
    k.qblocks = pl.qblocks;
    k.units = pl.splits * pl.qblocks * a.geom.kv_heads;
    k.per_xcd = (k.units + 7) / 8;
    // With one query block per kv head every K/V line is read once per call and the loads
    // are marked non-temporal (C4 verify: 101.7-102.2 vs 104.1-104.2 us in one A/B run, no
    // difference in another); query blocks that share a kv head re-read its tiles through
    // L2 and keep the default policy (C3 232.8 with nt vs 230.5 us).
    k.kv_once = pl.qblocks == 1;
    const dim3 grid(8 * k.per_xcd);
    const bool bf = a.kv_dtype == QR_DTYPE_BF16;
    const bool qsplit = a.q_dtype != a.kv_dtype;  // q not exact in the cache's 16-bit type
    hipError_t e;
    if (a.geom.head_dim == 128)
        e = bf ? launch_nt<true, 128>(k, pl.nt, qsplit, grid, stream) : launch_nt<false, 128>(k, pl.nt, qsplit, grid, stream);
    else
        e = bf ? launch_nt<true, 64>(k, pl.nt, qsplit, grid, stream) : launch_nt<false, 64>(k, pl.nt, qsplit, grid, stream);
    if (e != hipSuccess) return e;
    if (after_split && (e = hipEventRecord(after_split, stream)) != hipSuccess) return e;
    if (pl.splits == 1) return hipSuccess;
    if (a.geom.head_dim == 128) hipLaunchKernelGGL((chunk_combine_kernel<128>), dim3(rows), dim3(64), 0, stream, k);
    else hipLaunchKernelGGL((chunk_combine_kernel<64>), dim3(rows), dim3(64), 0, stream, k);
    return hipGetLastError();
}

}  // namespace qr
