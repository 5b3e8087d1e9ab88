// LSE merge of n partial attention blocks (the combine step of blockwise ring attention).
//
// No counterpart in the reference: its ring context parallelism all-gathers K/V and runs one SDPA
// (python/dtorch/nn/scaled_dot_product_attention_with_cp.py:87-101).  Closed form, per query row:
//   m = max_b LSE_b,  LSE = m + log sum_b exp(LSE_b - m),  O = sum_b exp(LSE_b - LSE) O_b.
// HBM-bound: each thread merges one 16-byte output chunk (8 elements), or two for n = 2 and n = 4; per chunk
// it reads the n LSE values of its row (shared by the D/8 threads of the row through L1) and n input chunks,
// and writes one chunk.  A workgroup covers 256 (or 512) consecutive chunks of one (batch, head) slab, so
// the only divisions are per workgroup and scalar; a thread's row and chunk come from shifts.
#include "dtattn_common.hpp"

namespace dtattn {

struct MergeParams {
    const void* o_blocks[DTATTN_MAX_MERGE_BLOCKS];
    const float* lse_blocks[DTATTN_MAX_MERGE_BLOCKS];
    void* o;
    float* lse;
    int64_t bo_b, bo_h, bo_s;
    int64_t bl_b, bl_h;
    int64_t o_b, o_h, o_s;
    int64_t l_b, l_h;
    int64_t slabs;  // B * H
    int32_t H, S, n;
    int32_t wg_per_slab;  // ceil(S * D / 8 / (256 * chunks per thread))
    int32_t cpr;          // 16-byte chunks per row (D / 8); read by the generic (D = 0) instantiation
};

// Block outputs are read exactly once: non-temporal loads (load_chunk<TI, true>).  The merged output is
// written through to memory (cache policy sc0 sc1, vector stores): at 4 blocks of [1, 32, 4096, 128] bf16
// from HBM that measured 33.7 -> 31.3 us per launch against non-temporal stores, and 34.4 with plain ones.
// The compiler has no intrinsic for this policy on a 16-byte global store and does not see into the asm,
// so the asm pays the hazard it would otherwise insert: a VALU write to the data VGPRs of a store wider
// than 8 bytes needs two wait states after it on gfx950 (s_nop 1).  Nothing after the store waits on it.
__device__ __forceinline__ void st16_wt(void* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}

template <typename TO>
__device__ __forceinline__ void store8(TO* p, const float* in) {
    if constexpr (sizeof(TO) == 4) {
        st16_wt(p, __builtin_bit_cast(u32x4, f32x4{in[0], in[1], in[2], in[3]}));
        st16_wt(p + 4, __builtin_bit_cast(u32x4, f32x4{in[4], in[5], in[6], in[7]}));
    } else {
        st16_wt(p, pack8<TO>(in));
    }
}

// Chunks per thread: two for n = 2 and n = 4 (every load of both in one round trip: 33.7 -> 30.3 us at
// 4 blocks of [1, 32, 4096, 128] bf16, with half the workgroups), one for the generic n.
template <int NB>
constexpr int merge_cpt() {
    return NB > 0 ? 2 : 1;
}

// D = 0: any head dim that is a multiple of 8, with the row split computed at run time.
template <typename TI, typename TO, int D, int NB>
__global__ void __launch_bounds__(256) lse_merge_kernel(const MergeParams p) {
    constexpr int CPT = merge_cpt<NB>();
    const int64_t bh = blockIdx.x / p.wg_per_slab;  // wave-uniform
    const int idx0 = (int)(blockIdx.x - bh * p.wg_per_slab) * (256 * CPT) + (int)threadIdx.x;
    const int cpr = D > 0 ? D / 8 : p.cpr;  // chunks per row (a power of two when D > 0)
    int s[CPT], c[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        s[k] = (idx0 + k * 256) / cpr;
        c[k] = idx0 + k * 256 - s[k] * cpr;
    }
    if (s[0] >= p.S) return;
    const int h = (int)(bh % p.H);
    const int64_t b = bh / p.H;
    const int n = NB > 0 ? NB : p.n;
    const int64_t lse_b = b * p.bl_b + h * p.bl_h;
    const int64_t in_b = b * p.bo_b + h * p.bo_h;
    const int64_t out_b = b * p.o_b + h * p.o_h;
    // A block with weight 0 (LSE = -inf) adds nothing, whatever its O holds (NaN included).
    auto add = [](float* acc, const Chunk<TI>& raw, float w) {
        float x[8];
        unpack_chunk<TI>(raw, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = w != 0.f ? __builtin_fmaf(w, x[e], acc[e]) : acc[e];
    };
    auto finish = [&](int k, const float* acc, float mb, float sum) {
        store8<TO>(reinterpret_cast<TO*>(p.o) + out_b + (int64_t)s[k] * p.o_s + c[k] * 8, acc);
        if (p.lse != nullptr && c[k] == 0)
            p.lse[b * p.l_b + h * p.l_h + s[k]] = sum > 0.f ? mb + __logf(sum) : kNegInf;
    };
    if constexpr (NB > 0) {
        // Every LSE and O load of the thread's chunks in one memory round trip.  A second chunk past the
        // slab's last row loads that row again (unconditional loads keep the waits counted) and stores nothing.
        const bool second = s[CPT - 1] < p.S;
        float l[CPT][NB];
        Chunk<TI> raw[CPT][NB];
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int sl = min(s[k], p.S - 1);
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                l[k][i] = p.lse_blocks[i][lse_b + sl];
                raw[k][i] = load_chunk<TI, true>(reinterpret_cast<const TI*>(p.o_blocks[i]) + in_b +
                                                 (int64_t)sl * p.bo_s + c[k] * 8);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keeps the scheduler from issuing the later loads after waits
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            if (k > 0 && !second) break;
            float m = kNegInf, sum = 0.f;
#pragma unroll
            for (int i = 0; i < NB; ++i) m = fmaxf(m, l[k][i]);
            const float mb = m == kNegInf ? 0.f : m;
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                l[k][i] = __expf(l[k][i] - mb);
                sum += l[k][i];
            }
            const float inv = sum > 0.f ? 1.f / sum : 0.f;
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < NB; ++i) add(acc, raw[k][i], l[k][i] * inv);
            finish(k, acc, mb, sum);
        }
    } else {
        // the n LSE values first, then the O chunks in batches of four loads in flight together
        const int64_t in_off = in_b + (int64_t)s[0] * p.bo_s + c[0] * 8;
        float l[DTATTN_MAX_MERGE_BLOCKS];
#pragma unroll
        for (int i = 0; i < DTATTN_MAX_MERGE_BLOCKS; ++i) l[i] = i < n ? p.lse_blocks[i][lse_b + s[0]] : kNegInf;
        __builtin_amdgcn_sched_barrier(0);
        float m = kNegInf, sum = 0.f;
#pragma unroll
        for (int i = 0; i < DTATTN_MAX_MERGE_BLOCKS; ++i) m = fmaxf(m, l[i]);
        const float mb = m == kNegInf ? 0.f : m;
#pragma unroll
        for (int i = 0; i < DTATTN_MAX_MERGE_BLOCKS; ++i) {
            l[i] = __expf(l[i] - mb);  // blocks past n have LSE -inf: weight 0
            sum += l[i];
        }
        const float inv = sum > 0.f ? 1.f / sum : 0.f;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i0 = 0; i0 < DTATTN_MAX_MERGE_BLOCKS; i0 += 4) {
            if (i0 >= n) break;
            Chunk<TI> raw[4] = {};
#pragma unroll
            for (int j = 0; j < 4; ++j)  // uniform guard: the loads of a batch issue back to back
                if (i0 + j < n) raw[j] = load_chunk<TI, true>(reinterpret_cast<const TI*>(p.o_blocks[i0 + j]) + in_off);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) add(acc, raw[j], l[i0 + j] * inv);
        }
        finish(0, acc, mb, sum);
    }
}

template <typename TI, typename TO, int D>
static int launch_merge(const MergeParams& p, hipStream_t stream) {
    MergeParams q = p;
    const int64_t per_wg = 256 * (p.n == 2 || p.n == 4 ? merge_cpt<2>() : merge_cpt<0>());
    q.wg_per_slab = (int32_t)(((int64_t)p.S * p.cpr + per_wg - 1) / per_wg);
    const int64_t blocks = p.slabs * q.wg_per_slab;
    if (blocks == 0) return DTATTN_OK;
    if (blocks > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "merge: grid too large");
    switch (p.n) {
        case 2:
            hipLaunchKernelGGL((lse_merge_kernel<TI, TO, D, 2>), dim3((unsigned)blocks), dim3(256), 0, stream, q);
            break;
        case 4:
            hipLaunchKernelGGL((lse_merge_kernel<TI, TO, D, 4>), dim3((unsigned)blocks), dim3(256), 0, stream, q);
            break;
        default:
            hipLaunchKernelGGL((lse_merge_kernel<TI, TO, D, 0>), dim3((unsigned)blocks), dim3(256), 0, stream, q);
            break;
    }
    return check_launch("lse_merge_kernel");
}

template <typename TI, typename TO>
static int dispatch_merge_d(const MergeParams& p, int D, hipStream_t stream) {
    if (D == 128) return launch_merge<TI, TO, 128>(p, stream);
    if (D == 64) return launch_merge<TI, TO, 64>(p, stream);
    if (D == 256) return launch_merge<TI, TO, 256>(p, stream);
    if (D == 512) return launch_merge<TI, TO, 512>(p, stream);
    return launch_merge<TI, TO, 0>(p, stream);
}

template <typename TI>
static int dispatch_merge_o(const MergeParams& p, int D, int o_dtype, hipStream_t stream) {
    if (o_dtype == DTATTN_BF16) return dispatch_merge_d<TI, bf16_t>(p, D, stream);
    if (o_dtype == DTATTN_FP16) return dispatch_merge_d<TI, f16_t>(p, D, stream);
    if (o_dtype == DTATTN_FP32) return dispatch_merge_d<TI, float>(p, D, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "merge: output dtype %d not supported", o_dtype);
}

}  // namespace dtattn

using namespace dtattn;

extern "C" int dtattn_lse_merge(const dtattn_merge_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "merge: args is NULL");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (a->n_blocks < 1 || a->n_blocks > DTATTN_MAX_MERGE_BLOCKS)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "merge: n_blocks=%d outside [1, %d]", a->n_blocks,
                    DTATTN_MAX_MERGE_BLOCKS);
    if (a->B < 0 || a->H < 0 || a->S < 0 || a->D <= 0) return fail(DTATTN_ERR_INVALID_ARGUMENT, "merge: bad sizes");
    if (a->D % 8 != 0 || a->D > 4096)
        return fail(DTATTN_ERR_UNSUPPORTED, "merge: head dim %lld must be a multiple of 8 up to 4096", (long long)a->D);
    if (a->B == 0 || a->H == 0 || a->S == 0) return DTATTN_OK;
    // chunk indices within one (batch, head) slab, rounded up to whole workgroups, are int32
    if (a->S * (a->D / 8) >= ((int64_t)1 << 31) - 512 || a->H > 0x7fffffff)
        return fail(DTATTN_ERR_UNSUPPORTED, "merge: sizes too large");
    if (a->o == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "merge: null output");
    const int in_esz = a->block_dtype == DTATTN_FP32 ? 4 : 2;
    const int out_esz = a->o_dtype == DTATTN_FP32 ? 4 : 2;
    for (int j = 0; j < 3; ++j) {
        if ((a->block_o_stride[j] * in_esz) % 16 != 0 || (a->o_stride[j] * out_esz) % 16 != 0)
            return fail(DTATTN_ERR_UNSUPPORTED, "merge: strides must be multiples of 16 bytes");
    }
    MergeParams p;
    for (int i = 0; i < DTATTN_MAX_MERGE_BLOCKS; ++i) {
        p.o_blocks[i] = i < a->n_blocks ? a->o_blocks[i] : nullptr;
        p.lse_blocks[i] = i < a->n_blocks ? a->lse_blocks[i] : nullptr;
        if (i < a->n_blocks && (p.o_blocks[i] == nullptr || p.lse_blocks[i] == nullptr))
            return fail(DTATTN_ERR_INVALID_ARGUMENT, "merge: block %d has a null pointer", i);
        if (i < a->n_blocks && (reinterpret_cast<uintptr_t>(p.o_blocks[i]) & 15u) != 0)
            return fail(DTATTN_ERR_UNSUPPORTED, "merge: block %d is not 16-byte aligned", i);
    }
    p.o = a->o;
    p.lse = a->lse;
    p.bo_b = a->block_o_stride[0], p.bo_h = a->block_o_stride[1], p.bo_s = a->block_o_stride[2];
    p.bl_b = a->block_lse_stride[0], p.bl_h = a->block_lse_stride[1];
    p.o_b = a->o_stride[0], p.o_h = a->o_stride[1], p.o_s = a->o_stride[2];
    p.l_b = a->lse ? a->lse_stride[0] : 0;
    p.l_h = a->lse ? a->lse_stride[1] : 0;
    p.slabs = a->B * a->H;
    p.wg_per_slab = 0;
    p.H = (int32_t)a->H;
    p.S = (int32_t)a->S;
    p.n = a->n_blocks;
    p.cpr = (int32_t)(a->D / 8);
    const int D = (int)a->D;
    if (a->block_dtype == DTATTN_BF16) return dispatch_merge_o<bf16_t>(p, D, a->o_dtype, stream);
    if (a->block_dtype == DTATTN_FP16) return dispatch_merge_o<f16_t>(p, D, a->o_dtype, stream);
    if (a->block_dtype == DTATTN_FP32) return dispatch_merge_o<float>(p, D, a->o_dtype, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "merge: block dtype %d not supported", a->block_dtype);
}
