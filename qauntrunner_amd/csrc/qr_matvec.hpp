// qr_matvec.hpp -- launch interface of the fused dequant + dot MatVec
// (DotKernels.MatVec / MatVecParallel, DotKernels.cs:599-633).
#pragma once

#include "qr_dequant.hpp"

namespace qr {

struct MatVecArgs {
    const uint8_t* w;    // [rows][row_bytes] in format fmt
    int fmt;
    long long rows;
    int cols;
    long long row_bytes;
    int nq;              // input vectors
    const float* x;      // [nq][cols]
    float* y;            // [nq][rows]
};

// A decoded format whose rows of `cols` weights the kernel takes: whole blocks, and
// cols a multiple of 8 for F32/F16/BF16 (the lane sums then need no tail).
bool matvec_shape_ok(int fmt, int cols);
hipError_t launch_matvec(const MatVecArgs& a, hipStream_t stream);
// n <= kMatVecGroupMax MatVecs that read the same x (same format, cols and nq): one launch
// when the format streams rows in the single-wave form (F32/F16/BF16), else one per matrix;
// every y equals launch_matvec's.
constexpr int kMatVecGroupMax = 4;
hipError_t launch_matvec_group(const MatVecArgs* a, int n, hipStream_t stream);

}  // namespace qr
