// qr_proj.hpp -- launch interface of the MLA q-absorb and W_UV projection kernels
// (StreamingEngine.cs:517-529 and :569-576).
#pragma once

#include "qr_dequant.hpp"
#include "qr_store.hpp"

namespace qr {

// kvb rows: [heads * (nope + vdim)][row_bytes] in format fmt; row h*(nope+vdim)+j is
// W_UK,h[j] for j < nope and W_UV,h[j-nope] after it (each row kv_lora weights).
struct MlaProjArgs {
    const uint8_t* w;
    int fmt;
    long long row_bytes;
    int heads, nope, rope, vdim, kv_lora;
    int nq;             // query rows
    const float* in;    // absorb: q [nq][heads][nope+rope];  W_UV: u [nq][heads][kv_lora]
    float* out;         // absorb: q_tilde [nq][heads][kv_lora];  W_UV: [nq][heads][vdim]
    float* q_rope;      // absorb only, may be null: receives q[.][h][nope:] as [nq][heads][rope]
};

constexpr int kMlaProjMaxNope = 256;  // query nope values the absorb kernel keeps in registers

// Shape rules both kernels assume (checked by the entry points): a decoded format,
// kv_lora a multiple of 8 and of the format's block, w 16-byte aligned, in/out
// 8-byte aligned.
bool mla_proj_shape_ok(int fmt, int kv_lora);
hipError_t launch_mla_absorb(const MlaProjArgs& a, hipStream_t stream);
hipError_t launch_mla_wuv(const MlaProjArgs& a, hipStream_t stream);

// Validates a projection call and fills `a` (except in/out/q_rope/nq); returns a
// QR_* status with the message set.
int mla_proj_prepare(MlaProjArgs& a, const void* kvb_dev, int fmt, int heads, int nope, int rope, int vdim,
                     int kv_lora);

}  // namespace qr

// One weight tensor resident in HBM: rows x cols weights of one QuantFormat, rows
// packed back to back (ModelStore tensor view: Fmt, Ptr, RowBytes; ModelStore.cs).
struct qr_weight {
    int device = 0;
    int format = 0;
    long long rows = 0;
    int cols = 0;
    long long row_bytes = 0;
    void* dev = nullptr;
    qr::DevBuf stage;       // x / y of the host-pointer calls
    hipStream_t stream = nullptr;
};
