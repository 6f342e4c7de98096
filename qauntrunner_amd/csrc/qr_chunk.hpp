// qr_chunk.hpp -- launch interface of the MFMA causal multi-query (chunk) kernel.
#pragma once

#include "qr_kernels.hpp"

namespace qr {

struct ChunkArgs {
    const void* pool;
    const int* page_table;  // device, entries of this (sequence, layer)
    PageGeom geom;          // planes = 2
    int kv_dtype;           // F16 or BF16
    int heads;
    int pos0;               // position of query 0
    // Device-side position of query 0: when set the kernels read it, clamped to [0, pos0];
    // pos0 is then the largest position query 0 may take, which the plan is made for.
    const int* pos0_dev;
    int nq;
    const void* q;          // device [nq][heads][head_dim] in q_dtype
    int q_dtype;
    float* out;             // device [nq][heads][head_dim]
    float scale;
};

struct ChunkPlan {
    int nt;                 // 16-row N tiles per wave
    int queries_per_block;
    int qblocks;
    int splits;
    int split_tokens;
    size_t workspace_bytes;
};

// 16-bit cache, head_dim 64 or 128, power-of-two group heads/kv_heads <= 64.
bool chunk_mfma_eligible(int kv_dtype, int head_dim, int heads, int kv_heads);
ChunkPlan plan_chunk(const ChunkArgs& a);
// after_split: when not null, recorded on `stream` right after the main kernel.
hipError_t launch_chunk(const ChunkArgs& a, const ChunkPlan& plan, void* workspace, hipStream_t stream,
                        hipEvent_t after_split = nullptr);

}  // namespace qr
