// Launch parameters shared by the bf16/fp16 and fp32 prefill kernels (prefill_fwd.hip,
// prefill_f32.hip): pointers, [B, H, S] element strides, sizes and the softmax constants, filled once
// by dtattn_prefill_fwd.
#pragma once

#include "dtattn_common.hpp"

namespace dtattn {

struct PrefillParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int64_t qs_b, qs_h, qs_s;
    int64_t ks_b, ks_h, ks_s;
    int64_t vs_b, vs_h, vs_s;
    int64_t os_b, os_h, os_s;
    int64_t lses_b, lses_h;
    int32_t B, Hq, Hkv, Sq, Sk, group;
    int32_t n_qblocks;
    int32_t delta;  // key j visible to query i iff j <= i + delta (causal only)
    float c;        // softmax scale * log2(e)
    int32_t xcd_map;  // 1: group the workgroups of each (batch, kv head) slice on one XCD
    // additive fp32 attention mask (MASKED kernels): element (b, h, i, j) at
    // mask + b*ms_b + h*ms_h + i*ms_l + j (key stride 1, strides multiples of 4, 16-byte aligned base);
    // it enters the raw scores as m / scale, so -inf and the dtype-minimum fills both hide a key
    const float* mask;
    int64_t ms_b, ms_h, ms_l;
    float inv_scale;
    // Head dims below the kernel's D (PAD kernels): Q/K rows hold qk_ch valid 16-byte chunks and V/O rows
    // v_ch; the chunks past them load as zeros (adding nothing to the scores, giving O columns that are
    // never stored).
    int32_t qk_ch, v_ch;
    // Key blocks (wide kernel): workgroup (x, y) takes keys [y kblock, (y + 1) kblock) and writes its
    // partial O and LSE at o + y os_split, lse + y lses_split; nsplit = 1 is the unsplit launch.
    int32_t nsplit, kblock;
    int64_t os_split, lses_split;
    // q's words pass through (w & q_and) ^ q_xor at load: negation or zeroing for scales <= 0
    uint32_t q_and, q_xor;
};

// Lazy rescaling: the running max only moves (and O, l are only rescaled) when some row's max grew
// by more than 2^8; otherwise P is taken against the stale max (values up to 2^8, exact in the
// normalisation, which uses the same max for O and l).
constexpr float kRescaleThreshold = 8.0f;

template <bool CAUSAL>
__device__ __forceinline__ BlockCoord block_coord(const PrefillParams& p) {
    return block_coord<CAUSAL>(p.B, p.Hq, p.Hkv, p.group, p.n_qblocks, p.xcd_map);
}

}  // namespace dtattn
