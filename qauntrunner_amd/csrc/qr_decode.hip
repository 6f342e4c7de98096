// qr_decode.hip -- split-K (flash-decoding) GQA decode attention for gfx950.
//
// Replaces the two-pass, fully materialised PagedKvCache.Attention
// (PagedKvCache.cs:83-136) with decode_stream_kernel (decode_mfma_kernel for
// 16-bit caches) + decode_combine_kernel.
//
// Grid: (split, unit, entry).  A unit is one kv head with up to GMAX of its
// query heads (or one query head when kv_heads does not divide heads).  A
// split is a run of whole pages of one entry; every K/V row of the split is
// read from HBM exactly once and shared by all query heads of the unit.
//
// Lane layout (wave64): a token row of head_dim elements is spread over
// LPT = head_dim/8 consecutive lanes, 8 elements per lane, taken as 16-byte
// chunks c = sub + LPT*j (sub = lane % LPT).  One load instruction of a wave
// reads LPT*16 contiguous bytes from each of 64/LPT consecutive rows, and the
// rows of one (page, kv head) are contiguous in the pool, so every wave load
// is a single contiguous run.  Dot products finish with DPP butterflies
// inside the LPT lanes of a token.
//
// Streaming: the workgroup walks its split in steps of U*256/LPT consecutive
// positions (U = 2 rows per token group for fp32, 4 for 16-bit, so a step is
// 32 KB of K+V at head_dim >= 32).  The K/V chunks of the next kPrefetch steps
// are already in flight in registers while a step is computed, so HBM sees
// a steady queue without any LDS staging of the stream.
//
// Softmax: online, in log2 units (q is pre-multiplied by scale*log2(e) and
// exponentials are v_exp_f32).  Each token group keeps its own running max
// and rescales its accumulator only when that max grows, which becomes rare
// after the first steps; no lane exchange sits inside the stream.  Token
// groups, waves, then splits are merged with the log-sum-exp rule.
// decode_combine_kernel then merges the splits of every (entry, head); an
// entry covered by a single split is written directly by the split kernel.
#include "qr_kernels.hpp"
#include "qr_mfma.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

namespace qr {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
// Register buffers of the step pipeline: one step in flight beyond the one computed.
// Measured at the 8B 32K fp32 shape: 2 buffers 52.0-52.3 us per call, 3 buffers
// 53.0-53.4, 4-6 buffers slower still (the loads queue deeper in the memory system
// without moving more bytes).
constexpr int kStreamBuffers = 2;
constexpr int kPrefetch = kStreamBuffers - 1;
constexpr int kMaxSplits = 256;     // splits per entry (grid x dimension of a launch)
constexpr int kMaxGroup = 8;        // GMAX upper bound

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
    int per_head;        // 1: one query head per unit (kv_heads does not divide heads)
    int units;
    const float* q;
    float* out;
    float* part_acc;     // [nb][heads][split_stride][head_dim]
    float2* part_ml;     // [nb][heads][split_stride] (max in log2 units, sum)
    int split_stride;    // splits of the longest entry
    float qscale;        // scale * log2(e)
    int split_tokens;
    int seq_len[kMaxDecodeBatch];
    int pt_off[kMaxDecodeBatch];
    const int* pos_dev;  // device positions (seq = pos + 1, clamped to [1, seq_len]) when set
    // In-kernel split merge (null: decode_combine_kernel merges): one arrival counter per
    // (entry, unit), zero between calls; the last workgroup of a unit to arrive merges it.
    unsigned* counters;
    // XCD-local slots: a 1-D grid where (entry, unit) pair p runs on launch slots b with
    // b % 8 == p % 8, i.e. on one XCD, so its partials stay in that XCD's L2.
    int xmap;
};

// Split, unit and entry of this workgroup.  Launch slot b runs on XCD b % 8 (the
// dispatcher's round robin over the 8 XCDs); with xmap set the slots of XCD x take the
// pairs x, x + 8, ... with their splits consecutive.  Correctness does not depend on where
// a slot runs: the merge protocol below is coherent across XCDs.
__device__ __forceinline__ void slot_coords(const DecodeK& p, int& split, int& unit, int& b) {
    if (p.xmap) {
        const int bid = blockIdx.x;
        const int k = bid >> 3;
        const int j = k / p.split_stride;
        split = k - j * p.split_stride;
        const int pair = (bid & 7) + 8 * j;
        unit = pair % p.units;
        b = pair / p.units;
    } else {
        split = blockIdx.x;
        unit = blockIdx.y;
        b = blockIdx.z;
    }
}

// Values of a lane pair (lanes l and l ^ off) in every lane of the pair: lo = the lower
// lane's, hi = the upper's.  off 16 and 32 take one v_permlane16/32_swap (no LDS).
__device__ __forceinline__ void lane_pair(float x, int off, float& lo, float& hi) {
    if (off == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else if (off == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else {
        const float o = __shfl_xor(x, off);
        const bool upper = (threadIdx.x & off) != 0;
        lo = upper ? o : x;
        hi = upper ? x : o;
    }
}

// Positions attended by entry b: seq_len[b], or a device position + 1 bounded by it.
// Workgroup-uniform: the position is a scalar load (no kernel here writes positions).
__device__ __forceinline__ int entry_seq(const DecodeK& p, int b) {
    if (!p.pos_dev) return p.seq_len[b];
    const int pos = reinterpret_cast<const __attribute__((address_space(4))) int*>(
        reinterpret_cast<uintptr_t>(p.pos_dev))[b];
    return __builtin_amdgcn_readfirstlane(min(max(pos + 1, 1), p.seq_len[b]));
}

// Positions per split of an entry attending `seq` positions: the plan's; with device
// positions (the plan was made for the bound) the entry's pages spread over the planned
// splits instead, so a short sequence still spreads over the GPU.  Never more than the
// plan's (the partials buffer holds split_stride splits).
__device__ __forceinline__ int entry_split_tokens(const DecodeK& p, int seq) {
    if (!p.pos_dev) return p.split_tokens;
    const int pages = (seq + kPageTokens - 1) >> kPageShift;
    return ((pages + p.split_stride - 1) / p.split_stride) << kPageShift;
}

__device__ __forceinline__ float exp2_or_zero(float x_minus_m, float m) {
    return m == -INFINITY ? 0.f : fast_exp2(x_minus_m);
}

// ---- in-kernel split merge (DecodeK::counters set)
//
// Every split workgroup stores its partial (unnormalised o, then max and sum) with
// write-through device-scope stores, waits until they are complete, and adds itself to its
// unit's arrival counter.  The workgroup that arrives last knows every other partial of the
// unit is in memory: it invalidates the caches that may hold an older copy (device-scope
// acquire), merges the unit's splits, writes the output and resets the counter for the
// next call.  No workgroup waits for another, so any grid size and any placement is safe;
// XCD-local slots only make the partials' round trip shorter.

// A partial value, written through to device scope.
__device__ __forceinline__ void store_partial(float* dst, float v) {
    __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LSE merge of the nsplit partials of heads h0..h0+G-1 of entry b by one workgroup.  T
// threads share a float4 column (T = 1, 2 or 4: lanes l, l ^ 32 and l ^ 16 of one wave),
// each merging every T-th split online with all its loads of a batch issued at once (always
// in range: no branch around them); the T parts are merged through lane swaps.
__device__ __forceinline__ void merge_unit(const DecodeK& p, int b, int h0, int G, int nsplit) {
    const int D = p.head_dim;
    const int d4n = D >> 2;
    const int ncol = G * d4n;
    const size_t row0 = static_cast<size_t>(b) * p.heads + h0;
    const float4* acc4 = reinterpret_cast<const float4*>(p.part_acc);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int T = ncol > 128 ? 1 : ncol > 64 ? 2 : 4;
    const int part = T == 1 ? 0 : T == 2 ? lane >> 5 : lane >> 4;
    const int cpw = 64 / T;  // columns per wave
    constexpr int kB = 16;
    for (int c0 = 0; c0 < ncol; c0 += kWaves * cpw) {
        const int c = c0 + wave * cpw + (lane & (cpw - 1));
        const bool active = c < ncol;
        const int cc = active ? c : 0;
        const int g = cc / d4n;
        const int d4 = cc - g * d4n;
        const size_t base = (row0 + g) * p.split_stride;
        float m = -INFINITY, l = 0.f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = part; s0 < nsplit; s0 += T * kB) {
            float4 a[kB];
            float2 ml[kB];
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int sp = min(s0 + i * T, nsplit - 1);
                a[i] = acc4[(base + sp) * d4n + d4];
                ml[i] = p.part_ml[base + sp];
            }
            float mb = m;
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                if (s0 + i * T >= nsplit) ml[i] = make_float2(-INFINITY, 0.f);  // a repeated split
                mb = fmaxf(mb, ml[i].x);
            }
            const float cm = exp2_or_zero(m - mb, m);
            l *= cm;
            o.x *= cm; o.y *= cm; o.z *= cm; o.w *= cm;
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const float w = exp2_or_zero(ml[i].x - mb, ml[i].x);
                l = fmaf(ml[i].y, w, l);
                o.x = fmaf(a[i].x, w, o.x);
                o.y = fmaf(a[i].y, w, o.y);
                o.z = fmaf(a[i].z, w, o.z);
                o.w = fmaf(a[i].w, w, o.w);
            }
            m = mb;
        }
        // every lane takes part in the swaps (inactive columns carry m = -inf, l = 0)
        for (int off = T == 4 ? 16 : 32; T > 1 && off <= 32; off <<= 1) {
            float mlo, mhi, llo, lhi, xlo, xhi;
            lane_pair(m, off, mlo, mhi);
            lane_pair(l, off, llo, lhi);
            const float M = fmaxf(mlo, mhi);
            const float clo = exp2_or_zero(mlo - M, mlo), chi = exp2_or_zero(mhi - M, mhi);
            l = llo * clo + lhi * chi;
            lane_pair(o.x, off, xlo, xhi);
            o.x = xlo * clo + xhi * chi;
            lane_pair(o.y, off, xlo, xhi);
            o.y = xlo * clo + xhi * chi;
            lane_pair(o.z, off, xlo, xhi);
            o.z = xlo * clo + xhi * chi;
            lane_pair(o.w, off, xlo, xhi);
            o.w = xlo * clo + xhi * chi;
            m = M;
        }
        if (active && part == 0)
            *reinterpret_cast<float4*>(p.out + (row0 + g) * D + d4 * 4) = make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
    }
}

// Called by every thread of a split workgroup after its partial stores.
__device__ __forceinline__ void arrive_and_merge(const DecodeK& p, int b, int unit, int h0, int G, int nsplit) {
    // the write-through partial stores are complete before the count moves
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ unsigned s_ticket;
    unsigned* ctr = p.counters + static_cast<size_t>(b) * p.units + unit;
    if (threadIdx.x == 0) s_ticket = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_ticket != static_cast<unsigned>(nsplit - 1)) return;
    if (threadIdx.x == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // device-scope acquire: the partial loads below miss the vector L1 and any L2 line that
    // may hold an older copy
    asm volatile("buffer_inv sc1" ::: "memory");
    merge_unit(p, b, h0, G, nsplit);
}

// DT: head_dim fixed at compile time (0: read from the arguments).
template <typename KT, int GMAX, int DPL, int U, int DT>
__global__ void __launch_bounds__(kThreads) decode_stream_kernel(const DecodeK p) {
    using C = Chunk<KT>;
    constexpr int EPC = C::kElems;  // elements per 16-byte chunk
    constexpr int NC = DPL / EPC;   // chunks per lane per row
    constexpr int ESZ = 16 / EPC;   // bytes per element
    constexpr int UMAX = U;         // rows per token group per step

    int split, unit, b;
    slot_coords(p, split, unit, b);
    const int seq = entry_seq(p, b);
    const int split_tokens = entry_split_tokens(p, seq);
    const int nsplit = (seq + split_tokens - 1) / split_tokens;
    if (split >= nsplit) return;
    const int t_begin = split * split_tokens;
    const int t_end = min(seq, t_begin + split_tokens);

    const int D = DT ? DT : p.head_dim;
    const int lsh = DT ? __builtin_ctz(DT / DPL) : p.lpt_shift;
    const int LPT = 1 << lsh;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane & (LPT - 1);
    const int tpw = 64 >> lsh;
    const int ntg = kWaves * tpw;
    const int tg = wave * tpw + (lane >> lsh);
    const int step_tokens = U * ntg;

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

    float q[GMAX][DPL];  // filled once the first K/V step is in flight
    const int* pt = p.page_table + p.pt_off[b];
    const long long head_off = static_cast<long long>(kvh) * kPageTokens * D;
    // row u of a lane's token group in a step: row_in_step + u * ntg
    const int row_in_step = tg;
    const int nsteps = (t_end - t_begin + step_tokens - 1) / step_tokens;

    // Addresses are a wave-uniform 64-bit base (the step's first row in the (page, kv
    // head) block, in SGPRs) plus a loop-invariant 32-bit lane offset, so the loads take
    // the scalar-base form and no per-lane address is recomputed per step.  (With
    // per-lane 64-bit addresses the compiler rebuilt them every step in registers that
    // the previous step's loads were still writing, and waited for every load in
    // flight -- the whole prefetch -- once per loop iteration.)
    const uint32_t lane_off = static_cast<uint32_t>((row_in_step * D + sub * EPC) * ESZ);
    // Head sizes that are a multiple of 8 but not a power of two (80, 96, ...) round the
    // lanes per row up to a power of two: a chunk past the row end gets an offset beyond
    // the buffer range, which loads zeros without touching memory, and a zero q slice.
    constexpr uint32_t kOutOfRange = 0xF0000000u;
    bool chunk_on[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) chunk_on[j] = DT != 0 || (sub + LPT * j) * EPC < D;

    U32x4 kbuf[kPrefetch + 1][UMAX][NC];
    U32x4 vbuf[kPrefetch + 1][UMAX][NC];
    // Splits start at different steps and wrap around: in lockstep, every workgroup
    // would read the same offset of its page at the same moment (measured: 1.5-3 us per
    // 32K-token call).  The units of one split stay together (rotating them apart too
    // cost 5% at batch 16).
    const int rot = (split * 7) % nsteps;
    auto step_t0 = [&](int st) { return t_begin + (st + rot < nsteps ? st + rot : st + rot - nsteps) * step_tokens; };
    // Page-table entry of the step starting at row t0: a scalar load through the constant
    // address space (the table is not written while the kernel runs, so it stays a scalar
    // load whatever else the kernel stores).
    auto phys_of = [&](int t0_in) -> long long {
        return reinterpret_cast<const __attribute__((address_space(4))) int*>(
            reinterpret_cast<uintptr_t>(pt))[__builtin_amdgcn_readfirstlane(t0_in) >> kPageShift];
    };
    // t0: first row of the step (wave-uniform: a step never crosses a page); phys: its page
    // live = false: a step past the end, issued only to keep the load count of every
    // iteration the same; its buffer resource has no records, so the loads return zeros
    // without touching memory (re-reading a step with non-temporal loads would go to HBM)
    auto issue_at = [&](int t0_in, long long phys, U32x4 (&kb)[UMAX][NC], U32x4 (&vb)[UMAX][NC], bool live) {
        const int t0 = __builtin_amdgcn_readfirstlane(t0_in);
        const char* kbase = p.pool + (phys * p.page_elems + head_off +
                                      static_cast<long long>(t0 & (kPageTokens - 1)) * D) * ESZ;
        // one buffer resource over the step's K rows and V rows (both planes of the page):
        // the byte offsets of the step stay far below 2^32.  The loads are marked
        // non-temporal (nt): every K/V line is read once per call, and a wave instruction
        // covers whole 128-byte lines, so nothing is lost by not keeping them (C2 fp32 B1:
        // 47.1-47.5 vs 51.4-52.2 us per call).
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(kbase), 0, live ? 0x7FFFFFFF : 0, kBufferFlags);
        const uint32_t vplane = static_cast<uint32_t>(p.plane_elems * ESZ);
#pragma unroll
        for (int u = 0; u < UMAX; ++u) {
            const uint32_t off = lane_off + static_cast<uint32_t>(u * ntg * D * ESZ);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const uint32_t o = chunk_on[j] ? off + LPT * j * 16 : kOutOfRange;
                kb[u][j] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, kCacheNt));
            }
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const uint32_t o = chunk_on[j] ? off + LPT * j * 16 : kOutOfRange;
                vb[u][j] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, vplane, kCacheNt));
            }
        }
    };

    float m[GMAX], l[GMAX], acc[GMAX][DPL];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;
    }

    auto compute = [&](int t_step, const U32x4 (&kb)[UMAX][NC], const U32x4 (&vb)[UMAX][NC]) {
        const int t0 = t_step + row_in_step;
        float s[UMAX][GMAX];
#pragma unroll
        for (int u = 0; u < UMAX; ++u) {
            float k[DPL];
#pragma unroll
            for (int j = 0; j < NC; ++j) C::widen(kb[u][j], &k[j * EPC]);
            const bool valid = t0 + u * ntg < t_end;
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < DPL; ++e) d = fmaf(q[g][e], k[e], d);
                d = group_sum(d, LPT);
                s[u][g] = valid ? d : -INFINITY;
            }
        }
        // running max of this token group (equal in its LPT lanes); the accumulator
        // is rescaled only in lanes whose max grows
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            float smax = s[0][g];
#pragma unroll
            for (int u = 1; u < UMAX; ++u) smax = fmaxf(smax, s[u][g]);
            if (smax > m[g]) {
                const float corr = exp2_or_zero(m[g] - smax, m[g]);
                l[g] *= corr;
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[g][e] *= corr;
                m[g] = smax;
            }
        }
        // a token group that has seen only masked rows still has m = -inf: weigh them 0, not NaN
        float mref[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) mref[g] = m[g] == -INFINITY ? 0.f : m[g];
#pragma unroll
        for (int u = 0; u < UMAX; ++u) {
            float v[DPL];
#pragma unroll
            for (int j = 0; j < NC; ++j) C::widen(vb[u][j], &v[j * EPC]);
            // rows past the end may hold stale data: a zero weight must not meet a NaN
            const bool valid = t0 + u * ntg < t_end;
#pragma unroll
            for (int e = 0; e < DPL; ++e) v[e] = valid ? v[e] : 0.f;
#pragma unroll
            for (int g = 0; g < GMAX; ++g) {
                const float pr = fast_exp2(s[u][g] - mref[g]);  // masked rows: exp2(-inf) = 0
                l[g] += pr;
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(pr, v[e], acc[g][e]);
            }
        }
    };

    // ---- query slice of this lane, pre-scaled into log2 units (loaded after the
    // first K/V step is in flight, so the two latencies overlap)
    auto load_q = [&]() {
        const float* qb = p.q + static_cast<size_t>(b) * p.heads * D;
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
#pragma unroll
            for (int j = 0; j < NC; ++j)
#pragma unroll
                for (int e = 0; e < EPC; ++e) {
                    const int dim = (sub + LPT * j) * EPC + e;
                    const int h = min(h0 + g, p.heads - 1);  // rows past the unit's heads are read, then zeroed
                    q[g][j * EPC + e] = chunk_on[j] ? qb[static_cast<size_t>(h) * D + dim] * ((g < G) ? p.qscale : 0.f) : 0.f;
                }
    };

    // ---- software-pipelined stream.  Every step issues the same number of loads (past
    // the end with an empty buffer range: no memory access), so the compiler's load
    // counting stays exact and each step waits only for its own loads.
    issue_at(step_t0(0), phys_of(step_t0(0)), kbuf[0], vbuf[0], true);
    load_q();
#pragma unroll
    for (int i = 1; i < kPrefetch; ++i) {
        const int t0 = step_t0(min(i, nsteps - 1));
        issue_at(t0, phys_of(t0), kbuf[i], vbuf[i], i < nsteps);
    }
    // Unrolled by the buffer count so every buffer index is a constant: step s0 + k is
    // computed from buffer k while step nxt(s0 + k) = s0 + k + kPrefetch is loaded into the
    // buffer computed last (past the end, an empty load of the step being computed).  The
    // page-table entry of each issued step is loaded one issue ahead, so its latency never
    // holds the loads back.  Exits only through the goto: the back-edge is steady state.
    auto nxt = [&](int i) { return i + kPrefetch < nsteps ? i + kPrefetch : i; };
    long long ph_next = phys_of(step_t0(nxt(0)));
    for (int s0 = 0;; s0 += kStreamBuffers) {
#pragma unroll
        for (int k = 0; k < kStreamBuffers; ++k) {
            const long long ph = ph_next;
            ph_next = phys_of(step_t0(nxt(s0 + k + 1)));
            issue_at(step_t0(nxt(s0 + k)), ph, kbuf[(k + kPrefetch) % kStreamBuffers],
                     vbuf[(k + kPrefetch) % kStreamBuffers], s0 + k + kPrefetch < nsteps);
            // the loads leave before any use of the step being computed, so that waiting
            // for that step never holds back the next one
            __builtin_amdgcn_sched_barrier(0);
            compute(step_t0(s0 + k), kbuf[k], vbuf[k]);
            if (s0 + k + 1 >= nsteps) goto streamed;
        }
    }
streamed:

    // ---- merge the token groups of the wave (lanes with equal `sub`), lane pairs l and
    // l ^ off exchanged through permlane swaps where off is 16 or 32
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            float mlo, mhi, llo, lhi;
            lane_pair(m[g], off, mlo, mhi);
            lane_pair(l[g], off, llo, lhi);
            const float M = fmaxf(mlo, mhi);
            const float clo = exp2_or_zero(mlo - M, mlo);
            const float chi = exp2_or_zero(mhi - M, mhi);
            l[g] = llo * clo + lhi * chi;
#pragma unroll
            for (int e = 0; e < DPL; ++e) {
                float alo, ahi;
                lane_pair(acc[g][e], off, alo, ahi);
                acc[g][e] = alo * clo + ahi * chi;
            }
            m[g] = M;
        }
    }

    // ---- merge the waves through LDS
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

    const size_t row_base = static_cast<size_t>(b) * p.heads;
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
        if (nsplit == 1) {
            p.out[(row_base + h) * D + d] = o / L;
        } else if (p.counters) {
            const size_t slot = (row_base + h) * p.split_stride + split;
            store_partial(&p.part_acc[slot * D + d], o);
            if (d == 0) {
                store_partial(&p.part_ml[slot].x, M);
                store_partial(&p.part_ml[slot].y, L);
            }
        } else {
            const size_t slot = (row_base + h) * p.split_stride + split;
            p.part_acc[slot * D + d] = o;
            if (d == 0) p.part_ml[slot] = make_float2(M, L);
        }
    }
    if (p.counters && nsplit > 1) arrive_and_merge(p, b, unit, h0, G, nsplit);
}

// ---------------------------------------------------------------------------
// MFMA decode for 16-bit caches with head_dim 64 or 128 (pages in the MFMA operand layout).
//
// Workgroup = 4 waves, one unit (a kv head and up to 16 of its query heads), one
// split.  The split is walked in 32-position steps; wave w takes steps w, w+4, ...
// with its own online softmax, and the four waves are merged through LDS at the end.
//   QK  S^T[pos][head] = K[pos][dims] . q^T[dims][head]: A = 16 K rows, one 1 KiB
//       operand block of the page (16 bytes per lane), B = q held in registers.
//   PV  O^T[dim][head] += V^T[dim][pos] . P^T[pos][head]: A = 8 consecutive positions
//       of each of 16 dims, one 1 KiB operand block of the V plane.
// Each wave load reads whole 128-byte lines and is marked non-temporal (with the
// earlier token-major K and dims-major V each load read half lines, the other halves
// by the next k-step or another wave's step, and nt loads then lost the lines between
// the two; C2 fp16 B1 / C4 decode / fp16 B16 measured 32.6 / 98.4 / 360 us then).
// v_mfma_f32_16x16x32_{f16,bf16} lane layout (checked on gfx950):
//   A[m = lane%16][k = 8*(lane/16)+i], B[k = 8*(lane/16)+i][n = lane%16],
//   D[m = 4*(lane/16)+r][n = lane%16].
// QK M tile mt takes row m as position 8(m/4) + 4mt + m%4, so after QK lane quarter
// q holds the scores of positions 8q..8q+7 of the step: exactly its PV k-slots.
// Precision: q and P are split into hi + lo parts of the cache's 16-bit type and
// every product is two MFMAs with fp32 accumulation, so q and P keep about 22
// (fp16) or 16 (bf16) significant bits while K and V enter exactly.  q is
// pre-multiplied per head by the power of two that brings its largest element to at
// most 2^14 (exact), so fp16 never overflows; the scores are scaled back.
constexpr int kMfmaGroup = 16;  // query heads per unit on the MFMA path

#ifndef QR_MFMA_DECODE_WG_PER_CU
#define QR_MFMA_DECODE_WG_PER_CU 2
#endif
constexpr int kMfmaWgPerCu = QR_MFMA_DECODE_WG_PER_CU;  // resident workgroups per CU the registers allow

template <bool BF16, int D>
__global__ void __launch_bounds__(kThreads, kMfmaWgPerCu) decode_mfma_kernel(const DecodeK p) {
    using T = typename std::conditional<BF16, __bf16, _Float16>::type;
    typedef T vec8 __attribute__((ext_vector_type(8)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int NK = D / 32;   // QK k-steps
    constexpr int NDT = D / 16;  // PV dim tiles
    constexpr int kStep = 32;    // positions per step

    int split, unit, b;
    slot_coords(p, split, unit, b);
    const int seq = entry_seq(p, b);
    const int split_tokens = entry_split_tokens(p, seq);
    const int t_begin = split * split_tokens;
    if (t_begin >= seq) return;
    const int t_end = min(seq, t_begin + split_tokens);
    const int lane = threadIdx.x & 63;
    // wave-uniform (SGPR): step positions, and so the page-table entry of a step, are
    // scalar; a vector load there would make every step wait for all loads in flight
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & (kWaves - 1);
    const int q4 = lane >> 4;
    const int n = lane & 15;

    int kvh, h0, G;
    if (p.per_head) {
        h0 = unit;
        kvh = static_cast<int>(static_cast<long long>(unit) * p.kv_heads / p.heads);
        G = 1;
    } else {
        const int c = unit % p.head_chunks;
        kvh = unit / p.head_chunks;
        h0 = kvh * p.group + c * kMfmaGroup;
        G = min(kMfmaGroup, p.group - c * kMfmaGroup);
    }
    const int* pt = p.page_table + p.pt_off[b];
    const long long kblk = static_cast<long long>(kvh) * kPageTokens * D;
    const int total_steps = (t_end - t_begin + kStep - 1) / kStep;
    const int nst = total_steps > wave ? (total_steps - wave + kWaves - 1) / kWaves : 0;
    // splits start at different steps and wrap around (see decode_stream_kernel)
    const int rot = (split * 7) % total_steps;
    auto step_t0 = [&](int st) { return t_begin + (st + rot < total_steps ? st + rot : st + rot - total_steps) * kStep; };

    U32x4 kb[2][2][NK];
    U32x4 vb[2][NDT];
    // Page-table entry of step st: a scalar load through the constant address space (the
    // table is not written while the kernel runs).
    auto phys_of = [&](int st) -> long long {
        return reinterpret_cast<const __attribute__((address_space(4))) int*>(
            reinterpret_cast<uintptr_t>(pt))[__builtin_amdgcn_readfirstlane(step_t0(st)) >> kPageShift];
    };
    // Loads of step st into buffer buf: buffer loads from a wave-uniform base (the step's
    // K and V operand blocks, in SGPRs) plus the loop-invariant lane offset, so no
    // per-step vector address is built (a per-step address in registers that the
    // previous step's loads were still writing made the compiler drain every load in
    // flight at the loop head).  A step is 32 x D contiguous elements of each plane.
    const uint32_t lane16 = static_cast<uint32_t>(16 * lane);
    // live = false: a step past the end (see decode_stream_kernel): no records, no access
    auto issue_at = [&](int st, long long phys, int buf, bool live) {
        const int t0 = __builtin_amdgcn_readfirstlane(step_t0(st));  // a step never crosses a page
        const int slot0 = t0 & (kPageTokens - 1);
        const char* kp = p.pool + (phys * p.page_elems + kblk + static_cast<long long>(slot0) * D) * 2;
        const int range = live ? 0x7FFFFFFF : 0;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kp), 0, range, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char*>(kp + p.plane_elems * 2), 0, range, kBufferFlags);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int kk = 0; kk < NK; ++kk)
                kb[buf][mt][kk] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    rk, lane16, 1024 * (mt * NK + kk), kCacheNt));
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            vb[buf][dt] = __builtin_bit_cast(U32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, lane16, 1024 * dt, kCacheNt));
    };
    if (nst > 0) issue_at(wave, phys_of(wave), 0, true);

    // ---- q of head h0 + n (zero for padding columns), log2 units, split into hi + lo
    const float* qb = p.q + static_cast<size_t>(b) * p.heads * D;
    const int hq = min(h0 + n, p.heads - 1);
    const float qs = n < G ? p.qscale : 0.f;
    float qf[NK][8];
    float amax = 0.f;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // scalar loads: the caller's q needs only 4-byte alignment
            qf[kk][i] = qb[static_cast<size_t>(hq) * D + 32 * kk + 8 * q4 + i] * qs;
            amax = fmaxf(amax, fabsf(qf[kk][i]));
        }
    amax = max_xor16(amax);
    amax = max_xor32(amax);
    int qexp = 0;
    if (!BF16 && amax > 16384.f && amax <= 3.0e38f) qexp = static_cast<int>(ceilf(log2f(amax / 16384.f)));
    const float down = ldexpf(1.f, -qexp);
    const float sscale = ldexpf(1.f, qexp);
    vec8 qhi[NK], qlo[NK];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = qf[kk][i] * down;
            const T hi = static_cast<T>(x);
            qhi[kk][i] = hi;
            qlo[kk][i] = static_cast<T>(x - static_cast<float>(hi));
        }

    f32x4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    auto compute = [&](int st, int buf) {
        const int t0 = step_t0(st);
        f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) {
                const vec8 a = __builtin_bit_cast(vec8, kb[buf][mt][kk]);
                sc[mt] = mfma16(a, qhi[kk], sc[mt]);
                sc[mt] = mfma16(a, qlo[kk], sc[mt]);
            }
        // scores of positions t0 + 8q4 + i, i = 4mt + r
        float s[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s[i] = t0 + 8 * q4 + i < t_end ? sc[i >> 2][i & 3] * sscale : -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = max_xor16(tmax);
        tmax = max_xor32(tmax);
        // lazy rescale: m moves only when the step max exceeds it by more than 2^8,
        // so P = 2^(s - m) <= 256; the whole wave skips the rescale when no lane needs it
        const bool grow = tmax > m + 8.f;
        const bool rescale = grow && m != -INFINITY;
        if (__builtin_amdgcn_ballot_w64(rescale)) {
            const float corr = rescale ? fast_exp2(m - tmax) : 1.f;
            l *= corr;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] *= corr;
        }
        if (grow) m = tmax;
        const float mref = m == -INFINITY ? 0.f : m;
        vec8 phi, plo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float e = fast_exp2(s[i] - mref);  // masked positions: 2^-inf = 0
            l += e;
            const T hi = static_cast<T>(e);
            phi[i] = hi;
            plo[i] = static_cast<T>(e - static_cast<float>(hi));
        }
        // a partial last step: positions past the end hold stale rows; zero their V
        // elements so that a zero weight cannot meet a NaN
        if (t0 + kStep > t_end) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                uint32_t w[4] = {vb[buf][dt].x, vb[buf][dt].y, vb[buf][dt].z, vb[buf][dt].w};
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (t0 + 8 * q4 + i >= t_end) w[i >> 1] &= (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
                vb[buf][dt] = U32x4{w[0], w[1], w[2], w[3]};
            }
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const vec8 a = __builtin_bit_cast(vec8, vb[buf][dt]);
            acc[dt] = mfma16(a, phi, acc[dt]);
            acc[dt] = mfma16(a, plo, acc[dt]);
        }
    };

    // ---- pipeline over this wave's steps with two register buffers (one step in flight
    // ahead of the one computed); every iteration issues the same loads (past the end
    // empty ones) so the compiler's load counting stays exact.  The
    // loads of the next step leave before any MFMA of the current one (scheduling barrier)
    // and the page-table entry of each issued step is loaded one issue ahead.
    auto gstep = [&](int i) { return wave + kWaves * min(i, nst - 1); };
    if (nst > 0) {
        long long ph_next = phys_of(gstep(1));
        for (int i = 0;; i += 2) {
            long long ph = ph_next;
            ph_next = phys_of(gstep(i + 2));
            issue_at(gstep(i + 1), ph, 1, i + 1 < nst);
            __builtin_amdgcn_sched_barrier(0);
            compute(gstep(i), 0);
            if (i + 1 >= nst) break;
            ph = ph_next;
            ph_next = phys_of(gstep(i + 3));
            issue_at(gstep(i + 2), ph, 0, i + 2 < nst);
            __builtin_amdgcn_sched_barrier(0);
            compute(gstep(i + 1), 1);
            if (i + 2 >= nst) break;
        }
    }

    // ---- merge the four waves through LDS (l is summed over the lane quarters first)
    l = sum_xor16(l);
    l = sum_xor32(l);
    __shared__ float sm_acc[kWaves][kMfmaGroup][D];
    __shared__ float sm_m[kWaves][kMfmaGroup];
    __shared__ float sm_l[kWaves][kMfmaGroup];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
        *reinterpret_cast<float4*>(&sm_acc[wave][n][16 * dt + 4 * q4]) = make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
    if (q4 == 0) {
        sm_m[wave][n] = m;
        sm_l[wave][n] = l;
    }
    __syncthreads();
    const int nsplit = (seq + split_tokens - 1) / split_tokens;
    const size_t row_base = static_cast<size_t>(b) * p.heads;
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
        if (nsplit == 1) {
            p.out[(row_base + h) * D + d] = o / L;
        } else if (p.counters) {
            const size_t slot = (row_base + h) * p.split_stride + split;
            store_partial(&p.part_acc[slot * D + d], o);
            if (d == 0) {
                store_partial(&p.part_ml[slot].x, M);
                store_partial(&p.part_ml[slot].y, L);
            }
        } else {
            const size_t slot = (row_base + h) * p.split_stride + split;
            p.part_acc[slot * D + d] = o;
            if (d == 0) p.part_ml[slot] = make_float2(M, L);
        }
    }
    if (p.counters && nsplit > 1) arrive_and_merge(p, b, unit, h0, G, nsplit);
}

// Log-sum-exp merge of the split partials: one workgroup per (head, entry).
// Thread t owns float4 column t % (head_dim/4) and every (256*4/head_dim)-th
// split; it loads up to 8 of its partials at once (one memory round trip for
// up to 64 splits at head_dim 128), merges them online, and the threads of a
// column are then merged through LDS.
__global__ void __launch_bounds__(kThreads) decode_combine_kernel(const DecodeK p) {
    const int h = blockIdx.x;
    const int b = blockIdx.y;
    const int seq = entry_seq(p, b);
    const int split_tokens = entry_split_tokens(p, seq);
    const int nsplit = (seq + split_tokens - 1) / split_tokens;
    if (nsplit <= 1) return;
    const int D = p.head_dim;
    const size_t base = (static_cast<size_t>(b) * p.heads + h) * p.split_stride;
    const int d4n = D >> 2;
    const int groups = kThreads / d4n;
    const int d4 = threadIdx.x % d4n;
    const int grp = threadIdx.x / d4n;
    const float4* acc4 = reinterpret_cast<const float4*>(p.part_acc);
    constexpr int kBatch = 8;

    float m = -INFINITY, l = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = grp; s0 < nsplit; s0 += groups * kBatch) {
        float4 a[kBatch];
        float2 ml[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int s = s0 + i * groups;
            const bool in = s < nsplit;
            a[i] = in ? acc4[(base + s) * d4n + d4] : make_float4(0.f, 0.f, 0.f, 0.f);
            ml[i] = in ? p.part_ml[base + s] : make_float2(-INFINITY, 0.f);
        }
        float mb = m;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) mb = fmaxf(mb, ml[i].x);
        const float cm = exp2_or_zero(m - mb, m);
        l *= cm;
        o.x *= cm; o.y *= cm; o.z *= cm; o.w *= cm;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const float c = exp2_or_zero(ml[i].x - mb, ml[i].x);
            l = fmaf(ml[i].y, c, l);
            o.x = fmaf(a[i].x, c, o.x);
            o.y = fmaf(a[i].y, c, o.y);
            o.z = fmaf(a[i].z, c, o.z);
            o.w = fmaf(a[i].w, c, o.w);
        }
        m = mb;
    }

    __shared__ float red_m[kThreads];
    __shared__ float red_l[kThreads];
    __shared__ float4 red_o[kThreads];
    red_m[threadIdx.x] = m;
    red_l[threadIdx.x] = l;
    red_o[threadIdx.x] = o;
    __syncthreads();
    if (threadIdx.x < d4n) {
        float M = -INFINITY;
        for (int gi = 0; gi < groups; ++gi) M = fmaxf(M, red_m[gi * d4n + threadIdx.x]);
        float L = 0.f;
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int gi = 0; gi < groups; ++gi) {
            const int k = gi * d4n + threadIdx.x;
            const float c = exp2_or_zero(red_m[k] - M, red_m[k]);
            L = fmaf(red_l[k], c, L);
            t.x = fmaf(red_o[k].x, c, t.x);
            t.y = fmaf(red_o[k].y, c, t.y);
            t.z = fmaf(red_o[k].z, c, t.z);
            t.w = fmaf(red_o[k].w, c, t.w);
        }
        float* out = p.out + (static_cast<size_t>(b) * p.heads + h) * D + threadIdx.x * 4;
        out[0] = t.x / L;
        out[1] = t.y / L;
        out[2] = t.z / L;
        out[3] = t.w / L;
    }
}

// ---- any head size the vector kernels do not take (not a multiple of 8, or outside
// 16..256): scalar split kernel.  One workgroup per (split, head, entry): the query row in
// LDS, one position per thread for the scores (staged in LDS), the split's max and sum by
// block reductions, then one dim per thread for the weighted sum of the V rows.  Partials
// as the other decode kernels' ([nb][heads][split_stride][head_dim] unnormalised, (max,
// sum) in log2 units), merged by decode_generic_combine_kernel.  Correct rather than
// fast: no model uses such head sizes, the reference accepts them (PagedKvCache.cs:29-37,
// SimdMath.cs:36-52 with its scalar tail).
constexpr int kGenericMaxSplitTokens = 16 * kPageTokens;  // the plan's longest split

__device__ __forceinline__ float load_cache(const char* pool, int dtype, long long i) {
    switch (dtype) {
        case QR_DTYPE_F32: return reinterpret_cast<const float*>(pool)[i];
        case QR_DTYPE_F16: return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(pool)[i]);
        default: return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(pool)[i]);
    }
}

__device__ __forceinline__ float block_max(float x, float* red) {
    x = fmaxf(x, dpp_xor1(x));
    x = fmaxf(x, dpp_xor2(x));
    x = fmaxf(x, dpp_half_mirror(x));
    x = fmaxf(x, dpp_mirror(x));
    x = max_xor32(max_xor16(x));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float block_sum(float x, float* red) {
    x = group_sum(x, 16);
    x = sum_xor32(sum_xor16(x));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ void __launch_bounds__(kThreads) decode_generic_kernel(const DecodeK p, int dtype) {
    static_assert(kThreads == 4 * 64, "block reductions over four waves");
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int seq = entry_seq(p, b);
    const int st = entry_split_tokens(p, seq);
    const int nsplit = (seq + st - 1) / st;
    if (split >= nsplit) return;
    const int t0 = split * st;
    const int t1 = min(seq, t0 + st);
    const int D = p.head_dim;
    const int kvh = static_cast<int>(static_cast<long long>(h) * p.kv_heads / p.heads);
    __shared__ float qs[kGenericMaxDim];
    __shared__ float sc[kGenericMaxSplitTokens];
    __shared__ float red[kWaves];
    const size_t row = static_cast<size_t>(b) * p.heads + h;
    for (int d = threadIdx.x; d < D; d += kThreads) qs[d] = p.q[row * D + d];
    __syncthreads();
    const int* pt = p.page_table + p.pt_off[b];
    const long long head_off = static_cast<long long>(kvh) * kPageTokens * D;
    float mx = -INFINITY;
    for (int t = t0 + threadIdx.x; t < t1; t += kThreads) {
        const long long k0 = pt[t >> kPageShift] * p.page_elems + head_off + static_cast<long long>(t & (kPageTokens - 1)) * D;
        float s = 0.f;
        for (int d = 0; d < D; ++d) s = fmaf(qs[d], load_cache(p.pool, dtype, k0 + d), s);
        s *= p.qscale;
        sc[t - t0] = s;
        mx = fmaxf(mx, s);
    }
    const float M = block_max(mx, red);
    float l = 0.f;
    for (int t = t0 + threadIdx.x; t < t1; t += kThreads) {
        const float e = fast_exp2(sc[t - t0] - M);
        sc[t - t0] = e;
        l += e;
    }
    const float L = block_sum(l, red);  // its barriers also publish the weights
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float acc = 0.f;
        for (int t = t0; t < t1; ++t) {
            const long long v0 = pt[t >> kPageShift] * p.page_elems + p.plane_elems + head_off +
                                 static_cast<long long>(t & (kPageTokens - 1)) * D;
            acc = fmaf(sc[t - t0], load_cache(p.pool, dtype, v0 + d), acc);
        }
        if (nsplit == 1) p.out[row * D + d] = acc / L;
        else p.part_acc[(row * p.split_stride + split) * D + d] = acc;
    }
    if (nsplit > 1 && threadIdx.x == 0) p.part_ml[row * p.split_stride + split] = make_float2(M, L);
}

// Merge of the generic kernel's splits: one workgroup per (head, entry).
__global__ void __launch_bounds__(kThreads) decode_generic_combine_kernel(const DecodeK p) {
    const int h = blockIdx.x, b = blockIdx.y;
    const int seq = entry_seq(p, b);
    const int st = entry_split_tokens(p, seq);
    const int nsplit = (seq + st - 1) / st;
    if (nsplit == 1) return;  // the split kernel wrote the output
    const int D = p.head_dim;
    const size_t row = static_cast<size_t>(b) * p.heads + h;
    const size_t base = row * p.split_stride;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p.part_ml[base + s].x);
    float L = 0.f;
    for (int s = 0; s < nsplit; ++s) L = fmaf(p.part_ml[base + s].y, fast_exp2(p.part_ml[base + s].x - M), L);
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float o = 0.f;
        for (int s = 0; s < nsplit; ++s)
            o = fmaf(p.part_acc[(base + s) * D + d], fast_exp2(p.part_ml[base + s].x - M), o);
        p.out[row * D + d] = o / L;
    }
}

int pick_gmax(int group) {
    if (group <= 1) return 1;
    if (group <= 2) return 2;
    if (group <= 4) return 4;
    return kMaxGroup;
}

int log2_exact(int v) {
    int s = 0;
    while ((1 << s) < v) ++s;
    return s;
}

constexpr int kDimsPerLane = 8;


template <typename KT, int GMAX, int U, int DT>
const void* kernel_ptr() {
    return reinterpret_cast<const void*>(&decode_stream_kernel<KT, GMAX, kDimsPerLane, U, DT>);
}

template <typename KT, int U, int DT>
const void* by_gmax(int gmax) {
    return gmax == 1 ? kernel_ptr<KT, 1, U, DT>() : gmax == 2 ? kernel_ptr<KT, 2, U, DT>()
         : gmax == 4 ? kernel_ptr<KT, 4, U, DT>() : kernel_ptr<KT, 8, U, DT>();
}

// A step is 32 KB of K+V: 2 fp32 or 4 16-bit rows per token group.  At head_dim
// 16 a step of 4 16-bit rows would cross a page, so it takes 2.  head_dim 64
// and 128 get instances with the dimension fixed at compile time.
template <typename KT, int U>
const void* by_dim(int gmax, int head_dim) {
    return head_dim == 128 ? by_gmax<KT, U, 128>(gmax) : head_dim == 64 ? by_gmax<KT, U, 64>(gmax)
         : by_gmax<KT, U, 0>(gmax);
}

// 16-bit caches reach this path only with head_dim 16, 32 or 256 (64 and 128 run
// on MFMA tiles).
const void* select_kernel(int dtype, int gmax, int head_dim) {
    const bool narrow = head_dim == 16;
    switch (dtype) {
        case QR_DTYPE_F32: return by_dim<float, 2>(gmax, head_dim);
        case QR_DTYPE_F16: return narrow ? by_gmax<F16Tag, 2, 0>(gmax) : by_gmax<F16Tag, 4, 0>(gmax);
        default: return narrow ? by_gmax<BF16Tag, 2, 0>(gmax) : by_gmax<BF16Tag, 4, 0>(gmax);
    }
}

// Resident workgroups per CU of a kernel instance (queried once per instance).
int blocks_per_cu(const void* fn) {
    static std::mutex mu;
    static const void* keys[64];
    static int vals[64];
    static int n = 0;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n; ++i)
        if (keys[i] == fn) return vals[i];
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kThreads, 0) != hipSuccess || blocks < 1) {
        (void)hipGetLastError();
        blocks = 1;
    }
    if (n < 64) {
        keys[n] = fn;
        vals[n] = blocks;
        ++n;
    }
    return blocks;
}

int cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            cus = prop.multiProcessorCount;
        if (cus <= 0) cus = 256;
    }
    return cus;
}

// The MFMA operand page layout marks the caches whose decode runs on MFMA tiles.
bool uses_mfma(const DecodeArgs& a) { return a.geom.mfma_layout != 0; }

int units_of(const DecodeArgs& a, int* gmax) {
    const int kvh = a.geom.kv_heads;
    if (a.heads % kvh == 0) {
        const int group = a.heads / kvh;
        *gmax = uses_mfma(a) ? kMfmaGroup : pick_gmax(group);
        return kvh * ((group + *gmax - 1) / *gmax);
    }
    *gmax = 1;
    return a.heads;
}

}  // namespace

// Scratch of qr_kv_attention_dev_noalloc (arrival counters, then split partials): a fixed
// array in device memory, so the call allocates nothing.  Each GPU holds its own copy until the process ends; in host
// code the array's name is not a device address, so its address is taken once per
// device with hipGetSymbolAddress and only that address is used.
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

int decode_scratch_address(int device, void** ptr) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) {
        set_error("device %d outside [0, %d)", device, kMaxDevices);
        return QR_ERR_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        int cur = -1;
        QR_HIP(hipGetDevice(&cur));
        if (cur != device) {
            set_error("scratch address requested for device %d while device %d is current", device, cur);
            return QR_ERR_INVALID_ARGUMENT;
        }
        void* a = nullptr;
        QR_HIP(hipGetSymbolAddress(&a, HIP_SYMBOL(scratch)));
        if (!a) {
            set_error("hipGetSymbolAddress returned a null scratch address on device %d", device);
            return QR_ERR_HIP;
        }
        // the arrival counters at the front start at zero (set up once per device, before any call)
        QR_HIP(hipMemset(a, 0, kDecodeCounterBytes));
        addr[device] = a;
    }
    *ptr = addr[device];
    return QR_OK;
}

DecodePlan plan_decode(const DecodeArgs& a) {
    DecodePlan pl{};
    int gmax = 1;
    pl.units = units_of(a, &gmax);
    const bool per_head = a.heads % a.geom.kv_heads != 0;
    const int group = per_head ? 1 : a.heads / a.geom.kv_heads;
    int max_pages = 1;
    long long work = 0;  // (unit, page) items of the launch
    for (int i = 0; i < a.nb; ++i) {
        const int pages = (a.seq_len[i] + kPageTokens - 1) / kPageTokens;
        max_pages = std::max(max_pages, pages);
        work += static_cast<long long>(pages) * pl.units;
    }
    // about one workgroup per CU, whole pages per split, at most 16 pages per split
    // (measured on MI355X: fewer, longer splits beat more resident workgroups -- also on
    // the MFMA path, whose registers allow two workgroups per CU: planning for two
    // per CU cost 2 us at the 8B 32K fp16 shape and at the 70B 128K decode)
    (void)blocks_per_cu;
    const int slots = cu_count();
    long long pps = std::max<long long>(1, work / slots);
    pps = std::min<long long>(pps, 16);
    pps = std::max<long long>(pps, (max_pages + kMaxSplits - 1) / kMaxSplits);
    pps = std::min<long long>(pps, max_pages);
    pl.split_tokens = static_cast<int>(pps) * kPageTokens;
    pl.max_splits = (max_pages + static_cast<int>(pps) - 1) / static_cast<int>(pps);
    pl.workspace_bytes = pl.max_splits > 1
        ? static_cast<size_t>(a.nb) * a.heads * pl.max_splits * (static_cast<size_t>(a.geom.head_dim) * 4 + 8)
        : 0;
    // In-kernel merge when the whole grid runs in one pass (every split workgroup resident at
    // once, so the merge sits on the call's critical path) and a unit's partials are small
    // (at most 1024 outputs per split); otherwise the combine kernel spreads the merge over
    // the GPU.  Measured on MI355X, per call: 8B 32K decode fp32 50.8 vs 51.9 us, fp16 32.1
    // vs 32.8 us, 70B 128K fp16 97.8 vs 98.0 us; at batch 16 (four passes) the combine
    // kernel is faster.
    const int pairs = pl.units * a.nb;
    const int unit_heads = per_head ? 1 : std::min(gmax, group);
    pl.fused = !decode_generic(a.geom.head_dim) && pl.max_splits > 1 &&
               static_cast<long long>(pl.max_splits) * pairs <= cu_count() &&
               unit_heads * a.geom.head_dim <= 1024 && pairs <= kDecodeCounters;
    // XCD-local slots need whole XCD rounds of pairs with equal head counts
    pl.xmap = pl.fused && pairs % 8 == 0 && (per_head || group % gmax == 0 || group < gmax);
    return pl;
}

hipError_t launch_decode(const DecodeArgs& a, const DecodePlan& pl, void* workspace, hipStream_t stream,
                         hipEvent_t after_split) {
    DecodeK k{};
    int gmax = 1;
    k.units = units_of(a, &gmax);
    k.pool = static_cast<const char*>(a.pool);
    k.page_table = a.page_table;
    k.page_elems = a.geom.page_elems();
    k.plane_elems = a.geom.plane_elems();
    k.head_dim = a.geom.head_dim;
    k.lpt_shift = log2_exact(a.geom.head_dim / kDimsPerLane);
    k.kv_heads = a.geom.kv_heads;
    k.heads = a.heads;
    if (a.heads % a.geom.kv_heads == 0) {
        k.group = a.heads / a.geom.kv_heads;
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
    k.split_stride = pl.max_splits;
    k.qscale = static_cast<float>(static_cast<double>(a.scale) * 1.4426950408889634);
    k.split_tokens = pl.split_tokens;
    for (int i = 0; i < a.nb; ++i) {
        k.seq_len[i] = a.seq_len[i];
        k.pt_off[i] = a.pt_off[i];
    }
    k.pos_dev = a.pos_dev;
    const bool fused = pl.fused && a.counters;
    k.counters = fused ? a.counters : nullptr;
    k.xmap = fused && pl.xmap;
    if (pl.max_splits > kMaxSplits) return hipErrorInvalidValue;
    if (decode_generic(a.geom.head_dim)) {
        if (a.geom.head_dim > kGenericMaxDim || pl.split_tokens > kGenericMaxSplitTokens) return hipErrorInvalidValue;
        hipLaunchKernelGGL(decode_generic_kernel, dim3(pl.max_splits, a.heads, a.nb), dim3(kThreads), 0, stream, k, a.dtype);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (after_split && (e = hipEventRecord(after_split, stream)) != hipSuccess) return e;
        if (pl.max_splits == 1) return hipSuccess;
        hipLaunchKernelGGL(decode_generic_combine_kernel, dim3(a.heads, a.nb), dim3(kThreads), 0, stream, k);
        return hipGetLastError();
    }
    const void* fn;
    if (uses_mfma(a)) {
        const bool bf = a.dtype == QR_DTYPE_BF16;
        fn = a.geom.head_dim == 128
            ? (bf ? reinterpret_cast<const void*>(&decode_mfma_kernel<true, 128>) : reinterpret_cast<const void*>(&decode_mfma_kernel<false, 128>))
            : (bf ? reinterpret_cast<const void*>(&decode_mfma_kernel<true, 64>) : reinterpret_cast<const void*>(&decode_mfma_kernel<false, 64>));
    } else {
        fn = select_kernel(a.dtype, gmax, a.geom.head_dim);
    }
    void* args[] = {&k};
    const dim3 grid = k.xmap ? dim3(pl.max_splits * k.units * a.nb) : dim3(pl.max_splits, k.units, a.nb);
    hipError_t e = hipLaunchKernel(fn, grid, dim3(kThreads), args, 0, stream);
    if (e != hipSuccess) return e;
    if (after_split && (e = hipEventRecord(after_split, stream)) != hipSuccess) return e;
    if (pl.max_splits == 1 || fused) return hipSuccess;
    hipLaunchKernelGGL(decode_combine_kernel, dim3(a.heads, a.nb), dim3(kThreads), 0, stream, k);
    return hipGetLastError();
}

}  // namespace qr
