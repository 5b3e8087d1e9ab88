// Per-head absmax quantization to OCP fp8 e4m3fn (pre-pass of the fp8 prefill).
//
// Supersedes the quantization inside the reference's SageAttention branch
// (dtorch/external/sage_attn/sage_attn_adapter.cc:28-158).  For each (b, h):
//   amax = max|x|, inv = 448 / amax, code = e4m3fn_rne(float(x * inv)) saturated to +-448,
//   descale = amax / 448 (amax == 0: inv = descale = 1).
// Two launches for up to three tensors (q, k, v of one call), no atomics and no zero-initialised memory:
//   1. fp8_absmax_partial_kernel: one workgroup per (tensor, b, h, slice of 64 rows) writes the slice's
//      max|x|.
//   2. fp8_quantize_kernel: each workgroup reduces its head's slice maxima, then converts its slice
//      with v_cvt_pk_fp8_f32 (round to nearest even) and writes 16 codes per thread per step; for a
//      tensor without a code buffer (the fused attention quantizes Q itself) it writes the scales only.
// HBM-bound: a thread puts all loads of a batch in flight before the first use (a slice of 64 rows
// at D = 128 is one batch per thread), and the second pass reads x again, mostly from L2 / MALL.
#include <string.h>

#include "dtattn_common.hpp"
#include "fp8_quant.hpp"

namespace dtattn {

constexpr int kQuantRowsPerSlice = 64;
constexpr int kQuantBatch = 4;  // 16-byte chunks (pass 1) or 16-element groups (pass 2) per thread per batch

template <typename T>
__global__ void __launch_bounds__(256) fp8_absmax_partial_kernel(const QuantParams qp) {
    __shared__ float wmax[4];
    const QuantTensor& p = qp.t[blockIdx.z];
    const int slice = blockIdx.x;
    const int bh = blockIdx.y;
    if (slice >= p.nslice || bh >= qp.B * p.H) return;  // workgroup-uniform
    const int b = bh / p.H, h = bh % p.H;
    const T* xp = reinterpret_cast<const T*>(p.x) + b * p.xs_b + h * p.xs_h;
    const int cpr = qp.D / 8;
    const int r0 = slice * kQuantRowsPerSlice;
    const int total = (min(p.S, r0 + kQuantRowsPerSlice) - r0) * cpr;
    float m = 0.f;
    for (int base = 0; base < total; base += 256 * kQuantBatch) {
        Chunk<T> raw[kQuantBatch] = {};
#pragma unroll
        for (int k = 0; k < kQuantBatch; ++k) {
            const int idx = base + k * 256 + (int)threadIdx.x;
            if (idx < total) raw[k] = load_chunk<T, false>(xp + (int64_t)(r0 + idx / cpr) * p.xs_s + (idx % cpr) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);  // the batch's loads are all in flight before the first use
#pragma unroll
        for (int k = 0; k < kQuantBatch; ++k) {
            float v[8];
            unpack_chunk<T>(raw[k], v);  // chunks past the slice are zeros
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
        }
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0)
        p.part[(int64_t)bh * p.nslice + slice] = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}


template <typename T>
__global__ void __launch_bounds__(256) fp8_quantize_kernel(const QuantParams qp) {
    __shared__ float s_inv;
    const QuantTensor& p = qp.t[blockIdx.z];
    const int slice = blockIdx.x;
    const int bh = blockIdx.y;
    if (slice >= p.nslice || bh >= qp.B * p.H) return;  // workgroup-uniform
    if (p.x8 == nullptr && slice != 0) return;          // scales only: one workgroup per head
    const int b = bh / p.H, h = bh % p.H;
    if (threadIdx.x < 64) {
        float m = 0.f;
        for (int i = threadIdx.x; i < p.nslice; i += 64) m = fmaxf(m, p.part[(int64_t)bh * p.nslice + i]);
        m = wave_max(m);
        if (threadIdx.x == 0) {
            s_inv = quant_inv(m);
            if (slice == 0) {
                p.descale[bh] = quant_descale(m);
                if (p.inv != nullptr) p.inv[bh] = quant_inv(m);
            }
        }
    }
    if (p.x8 == nullptr) return;  // (uniform) no barrier follows on this path
    const T* xp = reinterpret_cast<const T*>(p.x) + b * p.xs_b + h * p.xs_h;
    uint8_t* yp = p.x8 + ((int64_t)bh * p.S) * qp.D;
    const int cpr = qp.D / 16;  // 16 codes per thread per group
    const int r0 = slice * kQuantRowsPerSlice;
    const int total = (min(p.S, r0 + kQuantRowsPerSlice) - r0) * cpr;
    bool first = true;
    for (int base = 0; base < total; base += 256 * kQuantBatch) {
        Chunk<T> raw[kQuantBatch][2] = {};
#pragma unroll
        for (int k = 0; k < kQuantBatch; ++k) {  // x is read for the last time: non-temporal
            const int idx = base + k * 256 + (int)threadIdx.x;
            if (idx < total) {
                const T* src = xp + (int64_t)(r0 + idx / cpr) * p.xs_s + (idx % cpr) * 16;
                raw[k][0] = load_chunk<T, true>(src);
                raw[k][1] = load_chunk<T, true>(src + 8);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (first) {  // the head's scale (the loads above do not depend on it)
            __syncthreads();
            first = false;
        }
        const float inv = s_inv;
#pragma unroll
        for (int k = 0; k < kQuantBatch; ++k) {
            const int idx = base + k * 256 + (int)threadIdx.x;
            if (idx >= total) continue;
            float v[16];
            unpack_chunk<T>(raw[k][0], v);
            unpack_chunk<T>(raw[k][1], v + 8);
            uint32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = quant4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3], inv);
            st16(yp + (int64_t)(r0 + idx / cpr) * qp.D + (idx % cpr) * 16, u32x4{w[0], w[1], w[2], w[3]});
        }
    }
    if (first) __syncthreads();  // every thread reaches the workgroup barrier exactly once
}

template <typename T>
static int launch_quant(const QuantParams& p, int n, hipStream_t stream) {
    int32_t ms = 0, mbh = 0;
    for (int i = 0; i < n; ++i) {
        ms = max(ms, p.t[i].nslice);
        mbh = max(mbh, p.B * p.t[i].H);
    }
    if (ms == 0 || mbh == 0) return DTATTN_OK;
    dim3 grid((unsigned)ms, (unsigned)mbh, (unsigned)n);
    hipLaunchKernelGGL((fp8_absmax_partial_kernel<T>), grid, dim3(256), 0, stream, p);
    int st = check_launch("fp8_absmax_partial_kernel");
    if (st != DTATTN_OK) return st;
    hipLaunchKernelGGL((fp8_quantize_kernel<T>), grid, dim3(256), 0, stream, p);
    return check_launch("fp8_quantize_kernel");
}

// Quantization of up to three same-typed tensors in two launches (used by the fused fp8 attention).
int fp8_quantize_batch(QuantParams& p, int n, int32_t dtype, hipStream_t stream) {
    if (n < 1 || n > kQuantMaxTensors) return fail(DTATTN_ERR_INVALID_ARGUMENT, "quantize: %d tensors", n);
    if (dtype == DTATTN_BF16) return launch_quant<bf16_t>(p, n, stream);
    if (dtype == DTATTN_FP16) return launch_quant<f16_t>(p, n, stream);
    if (dtype == DTATTN_FP32) return launch_quant<float>(p, n, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "quantize: dtype %d not supported", dtype);
}

int32_t quant_slices(int64_t S) { return (int32_t)((S + kQuantRowsPerSlice - 1) / kQuantRowsPerSlice); }

}  // namespace dtattn

using namespace dtattn;

extern "C" size_t dtattn_fp8_quantize_workspace_size(int64_t B, int64_t H, int64_t S, int64_t D) {
    (void)D;
    if (B <= 0 || H <= 0 || S <= 0) return 0;
    const int64_t nslice = (S + kQuantRowsPerSlice - 1) / kQuantRowsPerSlice;
    return (((size_t)B * H * nslice * sizeof(float)) + 255) & ~(size_t)255;
}

extern "C" int dtattn_fp8_quantize_per_head(const void* x, int32_t x_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                            const int64_t x_stride[3], void* x8, float* descale, void* workspace,
                                            size_t workspace_bytes, void* stream_) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (B < 0 || H < 0 || S < 0 || D <= 0) return fail(DTATTN_ERR_INVALID_ARGUMENT, "quantize: bad sizes");
    if (D % 16 != 0) return fail(DTATTN_ERR_UNSUPPORTED, "quantize: D=%lld must be a multiple of 16", (long long)D);
    if (B == 0 || H == 0 || S == 0) return DTATTN_OK;
    if (x == nullptr || x8 == nullptr || descale == nullptr || x_stride == nullptr)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "quantize: null pointer");
    if (B * H > 65535 || S > 0x3fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "quantize: sizes too large");
    const int esz = x_dtype == DTATTN_FP32 ? 4 : 2;
    for (int j = 0; j < 3; ++j)
        if ((x_stride[j] * esz) % 16 != 0)
            return fail(DTATTN_ERR_UNSUPPORTED, "quantize: strides must be multiples of 16 bytes");
    const size_t need = dtattn_fp8_quantize_workspace_size(B, H, S, D);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(DTATTN_ERR_WORKSPACE, "quantize: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    QuantParams p;
    memset(&p, 0, sizeof(p));
    QuantTensor& t = p.t[0];
    t.x = x;
    t.x8 = reinterpret_cast<uint8_t*>(x8);
    t.descale = descale;
    t.inv = nullptr;
    t.part = reinterpret_cast<float*>(workspace);
    t.xs_b = x_stride[0], t.xs_h = x_stride[1], t.xs_s = x_stride[2];
    t.H = (int32_t)H, t.S = (int32_t)S;
    t.nslice = quant_slices(S);
    p.B = (int32_t)B, p.D = (int32_t)D;
    return fp8_quantize_batch(p, 1, x_dtype, stream);
}
