// qr_mla.hpp -- launch interface of the MLA absorbed-attention kernels.
#pragma once

#include "qr_kernels.hpp"

namespace qr {

constexpr int kMlaMaxHeads = 256;
constexpr int kMlaMaxLora = 1024;
constexpr int kMlaMaxRope = 256;

struct MlaArgs {
    const void* pool;        // latent pages: [page][256][kv_lora + rope]
    const int* page_table;   // entries of this layer
    int dtype;
    int kv_lora;
    int rope;
    int heads;
    int seq_len;             // pos + 1 (the bound, when pos_dev is set)
    const int* pos_dev;      // device position read by the kernels (clamped to [0, seq_len - 1]), or null
    const float* q_tilde;    // [heads][kv_lora]
    const float* q_rope;     // [heads][rope]
    float* u;                // [heads][kv_lora]
    float scale;
};

struct MlaPlan {
    int split_tokens;
    int splits;
    size_t workspace_bytes;
};

MlaPlan plan_mla(const MlaArgs& a);
hipError_t launch_mla(const MlaArgs& a, const MlaPlan& plan, void* workspace, hipStream_t stream);

}  // namespace qr
