// fp8 (OCP e4m3fn) attention forward for gfx950: Q/K/V codes with per-head descales, fp32
// accumulation on v_mfma_f32_32x32x64_f8f6f4, fp32 online softmax, bf16 output, fp32 LSE.
//
// Supersedes the quantized branch of SdpaOp::Compute, which hands q/k/v to the third-party
// SageAttention package (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:110-117,
// dtorch/external/sage_attn/sage_attn_adapter.cc:28-158).
//
// Same decomposition as the bf16 kernel (4 waves x 32 queries, 64-key tiles, S^T = K Q^T so a lane
// owns one query row), with 64-wide MFMA reduction steps:
//   S^T: A = K codes (lane: key l%32, 32 bytes of d), B = Q codes held in registers.
//   O^T: A = V^T codes from LDS, B = P^T re-quantized to e4m3 as P * 256 straight from the score
//        registers.  The reduction slots of one 32x32x64 step cover the 64 keys of the tile: lane
//        half hf holds the 4-key groups of parity hf, so V^T rows store even groups then odd groups.
//   Dequantisation: logits use scale * log2(e) * dq * dk; the output is acc * dv / (256 * l).
#include "dtattn_common.hpp"

namespace dtattn {

struct PrefillFp8Params {
    const uint8_t* q;
    const uint8_t* k;
    const uint8_t* v;
    bf16_t* o;
    float* lse;
    const float* qd;
    const float* kd;
    const float* vd;
    int64_t qs_b, qs_h, qs_s;
    int64_t ks_b, ks_h, ks_s;
    int64_t vs_b, vs_h, vs_s;
    int64_t os_b, os_h, os_s;
    int64_t lses_b, lses_h;
    int32_t B, Hq, Hkv, Sq, Sk, group;
    int32_t n_qblocks;
    int32_t delta;
    float c;
};

constexpr float kPScale = 256.f;

// 4x4 byte transpose: out[e] = (a.byte e, b.byte e, c.byte e, d.byte e).
__device__ __forceinline__ void transpose4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t* out) {
    const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
    const uint32_t t1 = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
    const uint32_t t2 = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
    const uint32_t t3 = __builtin_amdgcn_perm(d, c, 0x07030602u);  // c2 d2 c3 d3
    out[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    out[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    out[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// byte offset of 4-key group g in V^T row d (64 keys = 64 bytes): even groups first, then odd,
// with the four 16-byte chunks of the row XOR-swizzled by (d >> 1) & 3.
__device__ __forceinline__ int vt8_off(int d, int g) {
    const int pos = (g & 1) * 8 + (g >> 1);
    return 16 * ((pos >> 2) ^ ((d >> 1) & 3)) + 4 * (pos & 3);
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(256, 2) prefill_fp8_kernel(const PrefillFp8Params p) {
    constexpr int NW = 4;
    constexpr int BN = 64;
    constexpr int BM = NW * 32;
    constexpr int DCH = D / 16;          // 16-byte chunks per row
    constexpr int KSTEPS = D / 64;       // 32x32x64 steps of S^T
    constexpr int DT = D / 32;
    constexpr int KT = BN / 32;
    constexpr int KPT = (BN * DCH + 255) / 256;
    constexpr int NVB = (BN / 4) * DCH;  // 4-key x 16-d blocks
    constexpr int OSTR = D + 8;
    constexpr int KV_BYTES = 2 * BN * D;
    constexpr int O_BYTES = NW * 32 * OSTR * 2;
    constexpr int SMEM = KV_BYTES > O_BYTES ? KV_BYTES : O_BYTES;
    static_assert(NVB <= 256, "one V block per thread at most");

    __shared__ __attribute__((aligned(16))) char smem[SMEM];
    uint8_t* Ks = reinterpret_cast<uint8_t*>(smem);
    uint8_t* VTs = Ks + BN * D;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const int bh = p.B * p.Hq;
    const int bid = blockIdx.x;
    const int qb = CAUSAL ? (p.n_qblocks - 1 - bid / bh) : (bid / bh);
    const int rest = bid % bh;
    const int hq = rest % p.Hq;
    const int b = rest / p.Hq;
    const int hk = hq / p.group;

    const uint8_t* qp = p.q + b * p.qs_b + hq * p.qs_h;
    const uint8_t* kp = p.k + b * p.ks_b + hk * p.ks_h;
    const uint8_t* vp = p.v + b * p.vs_b + hk * p.vs_h;
    const float cq = p.c * p.qd[b * p.Hq + hq] * p.kd[b * p.Hkv + hk];
    const float vdesc = p.vd[b * p.Hkv + hk] * (1.f / kPScale);

    const int q0 = qb * BM;
    const int wq0 = q0 + wave * 32;

    int kend = p.Sk;
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;
        kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
    }
    const int nt = (kend + BN - 1) / BN;

    // Q codes: lane holds query l32, d = ks*64 + hf*32 .. +32.
    i32x8 qf[KSTEPS];
    {
        const int qrow = wq0 + l32;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
            if (qrow < p.Sq) {
                const uint8_t* src = qp + (int64_t)qrow * p.qs_s + ks * 64 + hf * 32;
                lo = ld16(src);
                hi = ld16(src + 16);
            }
            qf[ks] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
    }

    f32x16 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
    float mrow = kNegInf, lrow = 0.f;

    u32x4 kreg[KPT];
    u32x4 vreg[4];

    auto load_k = [&](int t) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int id = i * 256 + tid;
            const int r = id / DCH, c = id % DCH;
            const int key = t * BN + r;
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (id < BN * DCH && key < p.Sk) raw = ld16(kp + (int64_t)key * p.ks_s + c * 16);
            kreg[i] = raw;
        }
    };
    auto store_k = [&]() {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int id = i * 256 + tid;
            if (id < BN * DCH) {
                const int r = id / DCH, c = id % DCH;
                st16(Ks + r * D + 16 * (c ^ (r & (DCH - 1) & 7)), kreg[i]);
            }
        }
    };
    auto load_v = [&](int t) {
        if (tid < NVB) {
            const int g = tid / DCH, c = tid % DCH;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = t * BN + 4 * g + i;
                u32x4 raw = {0u, 0u, 0u, 0u};
                if (key < p.Sk) raw = ld16(vp + (int64_t)key * p.vs_s + c * 16);
                vreg[i] = raw;
            }
        }
    };
    auto store_v = [&]() {
        if (tid < NVB) {
            const int g = tid / DCH, c = tid % DCH;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t out[4];
                transpose4x4(vreg[0][w], vreg[1][w], vreg[2][w], vreg[3][w], out);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d = c * 16 + 4 * w + e;
                    *reinterpret_cast<uint32_t*>(VTs + d * BN + vt8_off(d, g)) = out[e];
                }
            }
        }
    };

    if (nt > 0) {
        load_k(0);
        store_k();
        load_v(0);
    }

    for (int t = 0; t < nt; ++t) {
        lds_barrier();
        if (t + 1 < nt) load_k(t + 1);

        const int kbase = t * BN;
        const bool wave_skip = CAUSAL && (kbase > wq0 + 31 + p.delta);
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > wq0 + p.delta));

        f32x16 s[KT];
        i32x8 pb;
        if (!wave_skip) {
#pragma unroll
            for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) s[kt][i] = 0.f;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    const int r = kt * 32 + l32;
                    const int c0 = ks * 4 + hf * 2;
                    const int sw = r & (DCH - 1) & 7;
                    const u32x4 lo = ld16(Ks + r * D + 16 * ((c0) ^ sw));
                    const u32x4 hi = ld16(Ks + r * D + 16 * ((c0 + 1) ^ sw));
                    const i32x8 a = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                     (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                    s[kt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, qf[ks], s[kt], 0, 0, 0, 0, 0, 0);
                }
            }
        }

        store_v();

        if (!wave_skip) {
            if (need_mask) {
                int lim = p.Sk - 1 - kbase;
                if (CAUSAL) lim = min(lim, wq0 + l32 + p.delta - kbase);
                lim -= 4 * hf;
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (kt * 32 + 8 * (i >> 2) + (i & 3) > lim) s[kt][i] = kNegInf;
            }
            float mx = kNegInf;
#pragma unroll
            for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][i]);
            mx = max_xor32(mx);
            const float mnew = fmaxf(mrow, mx * cq);
            const float mbase = (mnew == kNegInf) ? 0.f : mnew;
            const float alpha = fast_exp2(mrow - mbase);
            mrow = mnew;
            float ls = lrow * alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
            uint32_t pw[8];
#pragma unroll
            for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    float pv[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pv[e] = fast_exp2(__builtin_fmaf(s[kt][4 * w + e], cq, -mbase));
                        ls += pv[e];
                    }
                    int packed = __builtin_amdgcn_cvt_pk_fp8_f32(pv[0] * kPScale, pv[1] * kPScale, 0, false);
                    packed = __builtin_amdgcn_cvt_pk_fp8_f32(pv[2] * kPScale, pv[3] * kPScale, packed, true);
                    pw[kt * 4 + w] = (uint32_t)packed;
                }
            pb = i32x8{(int)pw[0], (int)pw[1], (int)pw[2], (int)pw[3], (int)pw[4], (int)pw[5], (int)pw[6], (int)pw[7]};
            lrow = ls;
        }

        lds_barrier();
        if (t + 1 < nt) {
            store_k();
            load_v(t + 1);
        }

        if (!wave_skip) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int d = dt * 32 + l32;
                const int sw = (d >> 1) & 3;
                const u32x4 lo = ld16(VTs + d * BN + 16 * ((2 * hf) ^ sw));
                const u32x4 hi = ld16(VTs + d * BN + 16 * ((2 * hf + 1) ^ sw));
                const i32x8 a = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                oacc[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, pb, oacc[dt], 0, 0, 0, 0, 0, 0);
            }
        }
    }

    __syncthreads();
    bf16_t* Os = reinterpret_cast<bf16_t*>(smem) + wave * 32 * OSTR;
    {
        const float l = sum_xor32(lrow);
        const float inv = l > 0.f ? vdesc / l : 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                bf16x4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = static_cast<bf16_t>(oacc[dt][4 * i4 + e] * inv);
                *reinterpret_cast<bf16x4*>(Os + l32 * OSTR + dt * 32 + 8 * i4 + 4 * hf) = o4;
            }
        if (p.lse != nullptr && hf == 0) {
            const int qrow = wq0 + l32;
            if (qrow < p.Sq) {
                const float lse = l > 0.f ? (mrow + __log2f(l)) * kLn2 : kNegInf;
                p.lse[b * p.lses_b + hq * p.lses_h + qrow] = lse;
            }
        }
    }
    __syncthreads();
    bf16_t* op = p.o + b * p.os_b + hq * p.os_h;
    constexpr int OCH = D / 8;
#pragma unroll
    for (int it = 0; it < 32 * OCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / OCH, c = id % OCH;
        const int qrow = wq0 + row;
        if (qrow < p.Sq) st16(op + (int64_t)qrow * p.os_s + c * 8, ld16(Os + row * OSTR + c * 8));
    }
}

template <int D, bool CAUSAL>
static int launch_fp8(const PrefillFp8Params& prm, hipStream_t stream) {
    PrefillFp8Params p = prm;
    p.n_qblocks = (p.Sq + 127) / 128;
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    hipLaunchKernelGGL((prefill_fp8_kernel<D, CAUSAL>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    return check_launch("prefill_fp8_kernel");
}

int prefill_fp8(const dtattn_prefill_args* a, float c, int32_t delta, hipStream_t stream) {
    PrefillFp8Params p;
    p.q = reinterpret_cast<const uint8_t*>(a->q);
    p.k = reinterpret_cast<const uint8_t*>(a->k);
    p.v = reinterpret_cast<const uint8_t*>(a->v);
    p.o = reinterpret_cast<bf16_t*>(a->o);
    p.lse = a->lse;
    p.qd = a->q_descale;
    p.kd = a->k_descale;
    p.vd = a->v_descale;
    p.qs_b = a->q_stride[0], p.qs_h = a->q_stride[1], p.qs_s = a->q_stride[2];
    p.ks_b = a->k_stride[0], p.ks_h = a->k_stride[1], p.ks_s = a->k_stride[2];
    p.vs_b = a->v_stride[0], p.vs_h = a->v_stride[1], p.vs_s = a->v_stride[2];
    p.os_b = a->o_stride[0], p.os_h = a->o_stride[1], p.os_s = a->o_stride[2];
    p.lses_b = a->lse ? a->lse_stride[0] : 0;
    p.lses_h = a->lse ? a->lse_stride[1] : 0;
    p.B = (int32_t)a->B;
    p.Hq = (int32_t)a->Hq;
    p.Hkv = (int32_t)a->Hkv;
    p.Sq = (int32_t)a->Sq;
    p.Sk = (int32_t)a->Sk;
    p.group = (int32_t)(a->Hq / a->Hkv);
    p.n_qblocks = 0;
    p.delta = delta;
    p.c = c;
    const bool causal = a->causal != 0;
    if (a->D == 128) return causal ? launch_fp8<128, true>(p, stream) : launch_fp8<128, false>(p, stream);
    if (a->D == 64) return causal ? launch_fp8<64, true>(p, stream) : launch_fp8<64, false>(p, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: head dim %lld not supported (64 or 128)", (long long)a->D);
}

}  // namespace dtattn
