// fp8 (OCP e4m3fn) attention forward for gfx950: Q/K/V codes with per-head descales, fp32
// accumulation on v_mfma_f32_32x32x64_f8f6f4, fp32 online softmax, bf16 output, fp32 LSE.
//
// Supersedes the quantized branch of SdpaOp::Compute, which hands q/k/v to the third-party
// SageAttention package (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:110-117,
// dtorch/external/sage_attn/sage_attn_adapter.cc:28-158).
//
// Same decomposition and pipeline as the bf16 kernel (4 waves x 32 queries, 64-key K and V tiles
// double-buffered in LDS by direct buffer->LDS loads, one barrier per tile, S^T = K Q^T so a lane owns
// one query row), with 64-deep MFMA reductions:
//   S^T: A = K codes, B = Q codes held in registers.  The A operand of key tile kt takes key row
//        pi_kt(R) = 32*((R/4)%2) + 16*kt + 4*(R/8) + R%4 at MFMA row R, which puts keys
//        32*hf .. 32*hf+31 of the 64-key tile in lane half hf of the score accumulators (element i of
//        tile kt is key 32*hf + 16*kt + i).
//   O^T: A = V^T codes read from the row-major V tile with ds_read_b64_tr_b8 (8 consecutive keys of
//        one d per lane and read; four reads give keys 32*hf .. +31), B = P^T re-quantized to e4m3
//        as P * 2^7 straight from the score registers, in the same key order.
//   Dequantisation: logits use scale * log2(e) * dq * dk; the output is acc * dv / l, with the row
//   sum l accumulated over the same 2^7-scaled P.
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
    int32_t xcd_map;
};

// P enters the PV MFMA as e4m3 codes of P * 2^kPScaleLog2.  With lazy rescaling P can exceed 1 by up
// to 2^kFp8RescaleThreshold before the running max moves, so 2^(7 + 1.5) = 362 stays below the e4m3
// maximum of 448.
constexpr float kPScaleLog2 = 7.f;
constexpr float kFp8RescaleThreshold = 1.5f;

// XOR swizzle of the 16-byte chunk index of fp8 tile row r (K and V).  Conflict-free for the 16-byte
// K reads of the permuted key rows (16 lanes per LDS cycle) and for the 8-byte transposed V reads
// (32 lanes per LDS cycle: 8 consecutive rows x 2 chunks).
template <int D>
__device__ __forceinline__ int fswz(int r) {
    return D >= 128 ? (2 * ((r >> 1) & 3)) ^ ((r >> 5) & 1) : (2 * ((r >> 2) & 1)) ^ ((r >> 5) & 1);
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
    typedef int i32x2 __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

    // K and V tiles, double-buffered, each [64 keys][D bytes] with chunk c of row r at c ^ fswz(r).
    __shared__ __attribute__((aligned(16))) uint8_t Ka[BN * D];
    __shared__ __attribute__((aligned(16))) uint8_t Kb[BN * D];
    __shared__ __attribute__((aligned(16))) uint8_t Va[BN * D];
    __shared__ __attribute__((aligned(16))) uint8_t Vb[BN * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const BlockCoord bc = block_coord<CAUSAL>(p.B, p.Hq, p.Hkv, p.group, p.n_qblocks, p.xcd_map);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;

    const uint8_t* qp = p.q + b * p.qs_b + hq * p.qs_h;
    const uint8_t* kp = p.k + b * p.ks_b + hk * p.ks_h;
    const uint8_t* vp = p.v + b * p.vs_b + hk * p.vs_h;
    const float cq = p.c * p.qd[b * p.Hq + hq] * p.kd[b * p.Hkv + hk];
    const float vdesc = p.vd[b * p.Hkv + hk];

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

    const int krow = (int)p.ks_s;  // row pitch in bytes (< 2^25, host-checked)
    const int vrow = (int)p.vs_s;

    // Tile t of K or V -> LDS: one wave instruction fills 1 KB (lane l -> byte 16*l), i.e. 1024/D
    // rows; lane l loads the global chunk that belongs at its slot, c = slot ^ fswz(row).  Rows past
    // Sk read zeros through the buffer resource's bound.
    auto dma = [&](uint8_t* dst, const uint8_t* base, int pitch, int64_t stride, int t) {
        constexpr int ROWS_PER_INSTR = 1024 / D;
        constexpr int INSTR = BN / ROWS_PER_INSTR / NW;  // per wave
        const int rows = min(BN, p.Sk - t * BN);
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, (uint32_t)((rows - 1) * pitch + D));
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int r0 = (wave * INSTR + i) * ROWS_PER_INSTR;
            const int r = r0 + lane / DCH;
            const int c = (lane % DCH) ^ fswz<D>(r);
            buf_ld16_lds_async(rs, dst + r0 * D, (uint32_t)(r * pitch + c * 16));
        }
    };

    // MFMA row R = l32 of key tile kt reads key row pi_kt(R).
    const int krow0 = 32 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3);
    // Transposed V reads: lane 2j+a of each 16-lane block addresses row K0 + j, bytes D0 + 8a .. +7,
    // and receives column D0 + (lane & 15) of rows K0 .. K0+7.
    const int blk = lane >> 4, bl = lane & 15;
    const int tr_row = 32 * (blk >> 1) + (bl >> 1);  // K0 = 32*hf + 8m, plus j
    const int tr_chunk = blk & 1;                    // D0 = 32*dt + 16*(blk & 1)
    const int tr_byte = 8 * (bl & 1);

    auto tile = [&](const uint8_t* Kc, const uint8_t* Vc, uint8_t* Kn, uint8_t* Vn, int t) {
        wait_vmem();
        lds_barrier();  // tile t landed everywhere; every wave finished tile t-1 (so Kn/Vn are free)
        if (t + 1 < nt) {
            dma(Kn, kp, krow, p.ks_s, t + 1);
            dma(Vn, vp, vrow, p.vs_s, t + 1);
        }
        const int kbase = t * BN;
        if (CAUSAL && kbase > wq0 + 31 + p.delta) return;  // every row of this wave precedes the tile
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > wq0 + p.delta));

        f32x16 s[KT];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[kt][i] = 0.f;
        // No wave-priority raises in this kernel: measured A/B on one MI355X, removing them made the
        // MMDiT 1x24x4608 and causal GQA 4x32x2048 fp8 launches 1.6% and 2.9% faster.
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            const int r = krow0 + 16 * kt;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                const int c0 = ks * 4 + hf * 2;
                const u32x4 lo = ld16(Kc + r * D + 16 * (c0 ^ fswz<D>(r)));
                const u32x4 hi = ld16(Kc + r * D + 16 * ((c0 + 1) ^ fswz<D>(r)));
                const i32x8 a = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                 (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                s[kt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, qf[ks], s[kt], 0, 0, 0, 0, 0, 0);
            }
        }
        if (need_mask) {
            // Element i of key tile kt is key kbase + 32*hf + 16*kt + i: visible iff 16*kt + i <= lim.
            int lim = p.Sk - 1 - kbase;
            if (CAUSAL) lim = min(lim, wq0 + l32 + p.delta - kbase);
            lim -= 32 * hf;
#pragma unroll
            for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (16 * kt + i > lim) s[kt][i] = kNegInf;
        }
        float mx = kNegInf;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][i]);
        mx = max_xor32(mx);
        const float mcand = fmaxf(mrow, mx * cq);
        if (__any(mcand - mrow > kFp8RescaleThreshold)) {  // wave-uniform
            const float alpha = fast_exp2(mrow - (mcand == kNegInf ? 0.f : mcand));
            mrow = mcand;
            lrow *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
        }
        // P * 2^7 = exp2(s * cq - m + 7), summed in fp32 and packed to e4m3 in key order
        const float mshift = ((mrow == kNegInf) ? 0.f : mrow) - kPScaleLog2;
        float ls = lrow;
        uint32_t pw[8];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                float pv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pv[e] = fast_exp2(__builtin_fmaf(s[kt][4 * w + e], cq, -mshift));
                    ls += pv[e];
                }
                int packed = __builtin_amdgcn_cvt_pk_fp8_f32(pv[0], pv[1], 0, false);
                packed = __builtin_amdgcn_cvt_pk_fp8_f32(pv[2], pv[3], packed, true);
                pw[kt * 4 + w] = (uint32_t)packed;
            }
        const i32x8 pb = {(int)pw[0], (int)pw[1], (int)pw[2], (int)pw[3],
                          (int)pw[4], (int)pw[5], (int)pw[6], (int)pw[7]};
        lrow = ls;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            i32x8 a;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int r = tr_row + 8 * m;
                const int c = 2 * dt + tr_chunk;
                const i32x2 v2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (lds_i32x2*)(Vc + r * D + 16 * (c ^ fswz<D>(r)) + tr_byte));
                a[2 * m] = v2[0];
                a[2 * m + 1] = v2[1];
            }
            oacc[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, pb, oacc[dt], 0, 0, 0, 0, 0, 0);
        }
    };

    if (nt > 0) {
        dma(Ka, kp, krow, p.ks_s, 0);
        dma(Va, vp, vrow, p.vs_s, 0);
    }
    // Q codes (and tile 0) complete here, visibly to the compiler, so that it inserts no load waits
    // inside the loop (where they would also drain the asynchronous tile loads).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    for (int t = 0; t < nt; t += 2) {  // unrolled by two so each tile names its buffers statically
        tile(Ka, Va, Kb, Vb, t);
        if (t + 1 < nt) tile(Kb, Vb, Ka, Va, t + 1);
    }

    // Epilogue: normalise, stage O (bf16) through LDS -- wave w in the 32 x D bf16 slab that is tile
    // buffer w, 16-byte chunk c of row r at c ^ (r % OCH) -- for 16-byte coalesced row stores, and
    // write the LSE.
    constexpr int OCH = D / 8;  // 16-byte chunks per bf16 output row
    static_assert(32 * D * 2 <= BN * D, "a tile buffer holds one wave's output rows");
    __syncthreads();
    bf16_t* Os = reinterpret_cast<bf16_t*>(wave == 0 ? Ka : wave == 1 ? Kb : wave == 2 ? Va : Vb);
    {
        const float l = sum_xor32(lrow);
        const float inv = l > 0.f ? vdesc / l : 0.f;
        const int row = l32;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                bf16x4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = static_cast<bf16_t>(oacc[dt][4 * i4 + e] * inv);
                const int c = dt * 4 + i4;
                *reinterpret_cast<bf16x4*>(Os + row * D + 8 * (c ^ (row % OCH)) + 4 * hf) = o4;
            }
        if (p.lse != nullptr && hf == 0) {
            const int qrow = wq0 + row;
            if (qrow < p.Sq) {
                const float lse = l > 0.f ? (mrow + __log2f(l) - kPScaleLog2) * kLn2 : kNegInf;
                p.lse[b * p.lses_b + hq * p.lses_h + qrow] = lse;
            }
        }
    }
    __syncthreads();
    bf16_t* op = p.o + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < 32 * OCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / OCH, c = id % OCH;
        const int qrow = wq0 + row;
        if (qrow < p.Sq) st16(op + (int64_t)qrow * p.os_s + c * 8, ld16(Os + row * D + 8 * (c ^ (row % OCH))));
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
    p.xcd_map = (p.B * p.Hkv) % 8 == 0 ? 1 : 0;
    const bool causal = a->causal != 0;
    if (a->D == 128) return causal ? launch_fp8<128, true>(p, stream) : launch_fp8<128, false>(p, stream);
    if (a->D == 64) return causal ? launch_fp8<64, true>(p, stream) : launch_fp8<64, false>(p, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: head dim %lld not supported (64 or 128)", (long long)a->D);
}

}  // namespace dtattn
