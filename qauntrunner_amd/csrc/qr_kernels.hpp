// qr_kernels.hpp -- launch interfaces shared by the translation units of libqr_attn.
#pragma once

#include "qr_common.hpp"

namespace qr {

// ------------------------------------------------------------------ paging
// Page layout in the HBM pool (elements of the cache dtype):
//   page = planes x kv_heads x kPageTokens x head_dim
// plane 0 holds K, plane 1 holds V (GQA cache); the MLA cache has one plane with
// kv_heads = 1 and head_dim = latent width.  Inside a plane each kv head owns a
// contiguous block of kPageTokens x head_dim elements: [token][dim] (one contiguous
// stream of 256 rows), or, when mfma_layout is set (16-bit caches with head_dim 64 or
// 128), the MFMA operand layout below.
//
// MFMA operand layout: the block is 8 steps of 32 tokens, step s holding tokens
// 32s..32s+31 in 32 x head_dim contiguous elements, cut into 1 KiB operand blocks of
// 64 x 8 elements; element e of lane L sits at 512 b + 8 L + e.  Lane L = 16 q + n is
// the lane that holds those 8 elements as an operand of v_mfma_f32_16x16x32_{f16,bf16}
// (A[m = n][k = 8 q + e]):
//   K (plane 0): block b = mt * head_dim/32 + kk holds token 8 (n / 4) + 4 mt + n % 4
//                of the step, dims 32 kk + 8 q + e (the QK A operand of M tile mt,
//                k-step kk);
//   V (plane 1): block b = dt holds dim 16 dt + n, tokens 8 q + e of the step (the PV
//                A operand of dim tile dt).
// So every operand the decode and chunk kernels feed to an MFMA is one contiguous
// 1 KiB (whole 128-byte lines per wave load, which the loads can mark non-temporal),
// and 8 consecutive dims of a K row or 8 aligned consecutive tokens of one V dim are one
// contiguous 16-byte run for the appends.
struct PageGeom {
    int planes;
    int kv_heads;
    int head_dim;
    int mfma_layout = 0;
    __host__ __device__ long long plane_elems() const { return (long long)kv_heads * kPageTokens * head_dim; }
    __host__ __device__ long long page_elems() const { return plane_elems() * planes; }
    // element offset of (plane, kv head, slot, dim) inside page `phys`
    __host__ __device__ long long offset(long long phys, int plane, int kvh, int slot, int d) const {
        const long long blk = phys * page_elems() + plane * plane_elems() + (long long)kvh * kPageTokens * head_dim;
        if (!mfma_layout) return blk + (long long)slot * head_dim + d;
        const int r = slot & 31;  // token within its step
        int b, lane;
        if (plane == 0) {
            b = ((r >> 2) & 1) * (head_dim >> 5) + (d >> 5);
            lane = 16 * ((d >> 3) & 3) + (((r >> 3) << 2) | (r & 3));
        } else {
            b = d >> 4;
            lane = 16 * (r >> 3) + (d & 15);
        }
        const int e = plane == 0 ? (d & 7) : (r & 7);
        return blk + (long long)(slot >> 5) * 32 * head_dim + 512 * b + 8 * lane + e;
    }
};
// 16-bit GQA caches with head_dim 64 or 128 use the MFMA operand layout (their decode
// and chunk kernels run on MFMA tiles).
inline bool kv_mfma_layout(int dtype, int head_dim) {
    return dtype != QR_DTYPE_F32 && (head_dim == 64 || head_dim == 128);
}

// Writes rows pos0..pos0+n-1 of `planes` source arrays into their pages.
// src[p] is [n][src_stride] of src_dtype; only the first row_len[p] elements of
// each row are written (row_len <= kv_heads*head_dim).
struct AppendArgs {
    void* pool;
    const int* page_table;  // device, entries of this (sequence, layer)
    PageGeom geom;
    int dtype;              // cache dtype
    const void* src[2];
    int row_len[2];
    int src_stride;
    int src_dtype;
    int pos0;
    int n;
    // Device-side position (appends and RoPE appends): when set, pos0 is *pos_dev, read by the
    // kernel, and the n rows are written only if the page of the last is held (*held_dev
    // pages) and positions pos0 .. pos0 + n - 1 lie in [0, max_seq).
    const int* pos_dev;
    const int* held_dev;
    int max_seq;
};
hipError_t launch_append(const AppendArgs& a, hipStream_t stream);

// Device-side page claim for n appended positions from *pos_dev on: pages
// held..((pos + n - 1) >> 8) of one (sequence, layer) get the next indices of the pool's
// device counter and their page-table entries; SeqLen's device copy grows to pos + n.
// state: [0] pages handed out, [1] error bits (1: pool full, 2: positions outside
// [0, max_seq)), then `held` and `seq_len` entries at the given indices.
struct PageClaimArgs {
    int* page_table;   // entries of this (sequence, layer)
    int* state;
    int held_index;    // index of this (sequence, layer)'s held count in state
    int seq_index;     // index of the sequence's SeqLen in state
    int capacity;      // pages in the pool
    int max_seq;
    const int* pos_dev;  // first position of the rows
    int n;               // rows: positions pos .. pos + n - 1
};
hipError_t launch_page_claim(const PageClaimArgs& a, hipStream_t stream);

// Gathers rows back out in the cache dtype ([n][kv_heads*head_dim] per plane),
// or decoded to fp32 when to_f32 is set.
struct GatherArgs {
    const void* pool;
    const int* page_table;
    PageGeom geom;
    int dtype;
    void* dst[2];
    int pos0;
    int n;
    int to_f32;
};
hipError_t launch_gather(const GatherArgs& a, hipStream_t stream);

// Fused RoPE + append (StreamingEngine.cs:245-248): rows pos0..pos0+n-1 of fp32 K are
// rotated (rotate-half, TransformerOps.cs:56-88) and, with V, converted to the cache
// dtype and scattered into their pages; q rows of the same positions ([n][q_width],
// q_width a multiple of head_dim) are rotated in place.  freq[i] = theta^(-2i/D) is
// computed on the host with the same libm powf as the reference's MathF.Pow path.
constexpr int kMaxRopeHalf = 256;  // head_dim <= 512
struct RopeAppendArgs {
    AppendArgs app;         // src[0] = K, src[1] = V, fp32, row length kv_dim
    float* q;               // may be null
    int q_width;
    float freq[kMaxRopeHalf];
};
hipError_t launch_rope_append(const RopeAppendArgs& a, hipStream_t stream);
// One workgroup of kRopeThreads threads per position, each thread taking up to
// kRopeMaxItems items of 8 dims (K heads plus q heads); wider rows use a row kernel that
// cannot read the position on the device, so device-position RoPE appends need
// rope_items_per_thread(...) <= kRopeMaxItems.
constexpr int kRopeThreads = 256;
constexpr int kRopeMaxItems = 8;
// Head sizes the item kernels do not take run on a generic per-pair kernel (any position,
// device-side too).
inline bool rope_generic(int head_dim) { return head_dim % 8 != 0 || head_dim > 256; }
inline int rope_items_per_thread(int heads, int head_dim) {
    return (heads * (head_dim / 8) + kRopeThreads - 1) / kRopeThreads;
}

// Widens 16-bit rows to fp32 (exact) -- used for 16-bit query inputs.
hipError_t launch_widen(const void* src, int src_dtype, float* dst, long long n, hipStream_t stream);

// out[i] = *pos0_dev + i for i < n (device positions of the queries of a chunk).
hipError_t launch_positions(int* out, const int* pos0_dev, int n, hipStream_t stream);

// ------------------------------------------------------------------ GQA decode
constexpr int kMaxDecodeBatch = 64;  // decode entries per launch (descriptor passed by value)
// Head sizes: the vector and MFMA decode kernels take multiples of 8 from 16 to 256; any
// other size up to kGenericMaxDim runs on the scalar generic kernel.
constexpr int kGenericMaxDim = 512;
inline bool decode_generic(int head_dim) { return head_dim % 8 != 0 || head_dim < 16 || head_dim > 256; }

struct DecodeArgs {
    const void* pool;
    const int* page_table;  // device page table (all sequences and layers)
    PageGeom geom;          // planes = 2
    int dtype;              // cache dtype
    int heads;
    const float* q;         // [nb][heads*head_dim]
    float* out;             // [nb][heads*head_dim]
    float scale;
    int nb;
    int seq_len[kMaxDecodeBatch];  // positions attended per entry (pos + 1)
    int pt_off[kMaxDecodeBatch];   // offset of the entry's page-table row
    // Device-side positions: when set, entry b attends positions 0..pos_dev[b] (read by
    // the kernels, clamped to [0, seq_len[b] - 1]); seq_len[b] then only bounds the plan.
    const int* pos_dev;
    // kDecodeCounters arrival counters in device memory, zero before the first call (each
    // call leaves the ones it used at zero), for plans that merge splits inside the split
    // kernel; null: the combine kernel merges.  Calls that share counters must not overlap.
    unsigned* counters;
};

// Split-K plan for one launch.
struct DecodePlan {
    int split_tokens;  // tokens per workgroup
    int max_splits;    // splits of the longest entry
    int units;         // workgroups per (entry, split): kv heads x head chunks, or heads
    size_t workspace_bytes;  // split partials
    int fused;         // splits merged inside the split kernel (needs DecodeArgs::counters)
    int xmap;          // XCD-local launch slots (with fused)
};
// Arrival counters of the in-kernel split merge: one per (entry, unit) of a launch.
constexpr int kDecodeCounters = 16384;
DecodePlan plan_decode(const DecodeArgs& a);
// workspace: at least plan.workspace_bytes of device memory (split partials).
// after_split: when not null, recorded on `stream` between the split kernel
// and the combine kernel (benchmark instrumentation).
hipError_t launch_decode(const DecodeArgs& a, const DecodePlan& plan, void* workspace, hipStream_t stream,
                         hipEvent_t after_split = nullptr);

// Scratch of the no-allocation decode entry point: a device array of this many bytes (per
// GPU, for the life of the process), the arrival counters (kDecodeCounterBytes, zero at
// load) followed by the split partials.
constexpr size_t kDecodeScratchBytes = size_t(8) << 20;
constexpr size_t kDecodeCounterBytes = kDecodeCounters * sizeof(unsigned);
// Device address of that array on `device`, which must be the current device; taken
// once per device with hipGetSymbolAddress (thread-safe).
int decode_scratch_address(int device, void** ptr);

}  // namespace qr
