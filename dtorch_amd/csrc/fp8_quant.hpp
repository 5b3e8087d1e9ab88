// Batched per-head absmax e4m3fn quantization (fp8_quant.hip), shared with the fused fp8 attention.
#pragma once

#include "dtattn_common.hpp"

namespace dtattn {

constexpr int kQuantMaxTensors = 3;

// Up to three tensors of one element type quantized together (q, k, v of one attention call): grid
// (max slices, max B*H, tensor).  Workgroups past a tensor's own extents exit at once.
struct QuantTensor {
    const void* x;
    uint8_t* x8;     // codes [B, H, S, D] contiguous; NULL: only the scales (the attention kernel
                     // quantizes this tensor itself)
    float* descale;  // [B*H] amax / 448
    float* inv;      // [B*H] 448 / amax, the factor applied before rounding; may be NULL
    float* part;     // [B*H, nslice] slice maxima (workspace)
    int64_t xs_b, xs_h, xs_s;
    int32_t H, S, nslice;
};
struct QuantParams {
    QuantTensor t[kQuantMaxTensors];
    int32_t B, D;
};

// Slices of 64 rows per head (the first launch's workgroups along x).
int32_t quant_slices(int64_t S);
// Quantizes p.t[0 .. n-1] (dtype BF16, FP16 or FP32) in two launches on `stream`.
int fp8_quantize_batch(QuantParams& p, int n, int32_t dtype, hipStream_t stream);

}  // namespace dtattn
