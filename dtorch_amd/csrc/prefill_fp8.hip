// fp8 (OCP e4m3fn) attention forward for gfx950: Q/K/V codes with per-head descales, fp32
// accumulation on v_mfma_f32_32x32x64_f8f6f4, fp32 online softmax, bf16 or fp16 output, fp32 LSE.
//
// Two entry points: dtattn_prefill_fwd with FP8 codes from the caller, and dtattn_prefill_fp8, the
// native fp8 path from bf16/fp16 inputs in three launches: per-head maxima of q, k and v; K/V codes
// plus the scales of all three; then this kernel, which rounds its own 128 Q rows to e4m3 in registers
// with the same per-head factor (so Q's codes never go through memory).  Non-causal grids whose last
// round over the GPU's workgroup slots is partly empty split that round's query blocks into key pieces,
// merged by a fourth launch (fp8_tail_merge_kernel) in either entry point.
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
#include <string.h>

#include <atomic>

#include "dtattn_common.hpp"
#include "fp8_quant.hpp"

namespace dtattn {

struct PrefillFp8Params {
    const void* q;  // codes, or bf16/fp16 rows rounded in the kernel (factor qinv)
    const uint8_t* k;
    const uint8_t* v;
    void* o;
    float* lse;
    const float* qd;
    const float* kd;
    const float* vd;
    const float* qinv;  // [B*Hq] 448 / amax of q's head, for 16-bit q
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
    uint32_t q_and, q_xor;  // applied to q's words at load (codes or 16-bit rows), as in ScalePlan
    // Tail split (non-causal only): workgroups below n_full take whole query blocks; the query blocks
    // n_full .. of the plain grid run as tail_s pieces of tail_tiles key tiles each, which store their
    // partials in tail_part for fp8_tail_merge_kernel.
    int32_t n_full, tail_s, tail_tiles;
    uint8_t* tail_part;
};

// Bytes of one tail piece's partial: its O normalised by its own row sum, in fp16 (an average of V codes,
// so within +-448), as [wave][pair of 4-value groups][lane][8] in the accumulator's register order; then
// the running max and the row sum in fp32 as [wave][lane][2].
template <int D>
constexpr int64_t fp8_tail_o_bytes() { return 4 * (D / 32) * 2 * 64 * 16; }
template <int D>
constexpr int64_t fp8_tail_part_bytes() { return fp8_tail_o_bytes<D>() + 4 * 64 * 8; }
constexpr int kFp8TailMaxPieces = 8;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two floats as fp16 (round to nearest even) in one word, and back.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}
__device__ __forceinline__ f32x2 unpack_f16x2(uint32_t w) {
    const f16x2 h = __builtin_bit_cast(f16x2, w);
    return f32x2{(float)h[0], (float)h[1]};
}

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

// Normalises one wave's 32 query rows and writes them: O^T accumulators `oacc` (lane: row l32, d rows of
// half hf), running max `mrow` (log2 units) and row sum `l`, both of the 2^kPScaleLog2-scaled P.  O is staged through the wave's slab `Os` of 32 x D 16-bit values in LDS
// (16-byte chunk c of row r at c ^ (r % (D / 8))) for 16-byte coalesced row stores.  Holds workgroup
// barriers: every wave of the workgroup calls it.
template <int D, typename TO>
__device__ __forceinline__ void fp8_write_rows(const PrefillFp8Params& p, int b, int hq, int wq0, const f32x16* oacc,
                                               float mrow, float l, float vdesc, TO* Os) {
    typedef typename Elem<TO>::vec4 O4;
    constexpr int OCH = D / 8;  // 16-byte chunks per 16-bit output row
    constexpr int DT = D / 32;
    const int lane = threadIdx.x & 63, hf = lane >> 5;
    {
        const float inv = l > 0.f ? vdesc / l : 0.f;
        const int row = lane & 31;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                O4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = Elem<TO>::from_f32(oacc[dt][4 * i4 + e] * inv);
                const int c = dt * 4 + i4;
                *reinterpret_cast<O4*>(Os + row * D + 8 * (c ^ (row % OCH)) + 4 * hf) = o4;
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
    TO* op = reinterpret_cast<TO*>(p.o) + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < 32 * OCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / OCH, c = id % OCH;
        const int qrow = wq0 + row;
        if (qrow < p.Sq)
            __builtin_nontemporal_store(ld16(Os + row * D + 8 * (c ^ (row % OCH))),
                                        reinterpret_cast<u32x4*>(op + (int64_t)qrow * p.os_s + c * 8));
    }
}

// TQ: uint8_t (Q given as codes) or bf16_t / f16_t (Q rounded here); TO: the output element type.
template <int D, bool CAUSAL, typename TQ, typename TO>
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

    // Pieces are ordered so that piece bid' of tail block tb runs on tb's XCD (n_full, the tail and the
    // grid are multiples of 8 by the host's plan): the 8 XCDs take blocks round robin.
    int bid = blockIdx.x, piece = -1;
    if (!CAUSAL && bid >= p.n_full) {
        const int j = bid - p.n_full;
        piece = (j >> 3) % p.tail_s;
        bid = p.n_full + ((j >> 3) / p.tail_s) * 8 + (j & 7);
    }
    const BlockCoord bc = block_coord_at<CAUSAL>(bid, p.B, p.Hq, p.Hkv, p.group, p.n_qblocks, p.xcd_map);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;

    const TQ* qp = reinterpret_cast<const TQ*>(p.q) + b * p.qs_b + hq * p.qs_h;
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
    int nt = (kend + BN - 1) / BN;
    int t0 = 0;
    if (!CAUSAL && piece >= 0) {  // the host's plan leaves every piece at least one tile
        t0 = piece * p.tail_tiles;
        nt = min(nt, t0 + p.tail_tiles);
    }

    // Q codes: lane holds query l32, d = ks*64 + hf*32 .. +32.
    i32x8 qf[KSTEPS];
    {
        const int qrow = wq0 + l32;
        if constexpr (sizeof(TQ) == 1) {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
                if (qrow < p.Sq) {
                    const TQ* src = qp + (int64_t)qrow * p.qs_s + ks * 64 + hf * 32;
                    lo = q_bits(ld16(src), p.q_and, p.q_xor);
                    hi = q_bits(ld16(src + 16), p.q_and, p.q_xor);
                }
                qf[ks] = i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
        } else {
            // 16-bit rows rounded to e4m3 with the head's factor, exactly as the quantizer rounds them
            const float qinv = p.qinv[b * p.Hq + hq];
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                u32x4 raw[4] = {};
                if (qrow < p.Sq) {
                    const TQ* src = qp + (int64_t)qrow * p.qs_s + ks * 64 + hf * 32;
#pragma unroll
                    for (int j = 0; j < 4; ++j) raw[j] = q_bits(ld16(src + 8 * j), p.q_and, p.q_xor);
                }
                uint32_t w[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float x[8];
                    unpack8<TQ>(raw[j], x);
                    w[2 * j] = quant4(x[0], x[1], x[2], x[3], qinv);
                    w[2 * j + 1] = quant4(x[4], x[5], x[6], x[7], qinv);
                }
                qf[ks] = i32x8{(int)w[0], (int)w[1], (int)w[2], (int)w[3], (int)w[4], (int)w[5], (int)w[6], (int)w[7]};
            }
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

    if (nt > t0) {
        dma(Ka, kp, krow, p.ks_s, t0);
        dma(Va, vp, vrow, p.vs_s, t0);
    }
    // Q codes (and tile 0) complete here, visibly to the compiler, so that it inserts no load waits
    // inside the loop (where they would also drain the asynchronous tile loads).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    for (int t = t0; t < nt; t += 2) {  // unrolled by two so each tile names its buffers statically
        tile(Ka, Va, Kb, Vb, t);
        if (t + 1 < nt) tile(Kb, Vb, Ka, Va, t + 1);
    }

    if (!CAUSAL && piece >= 0) {
        // A piece stores its O over its own row sum, running max and row sum for fp8_tail_merge_kernel.
        const float lsum = sum_xor32(lrow);
        uint8_t* mine = p.tail_part + ((int64_t)(bid - p.n_full) * p.tail_s + piece) * fp8_tail_part_bytes<D>();
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        u32x4* po = reinterpret_cast<u32x4*>(mine) + wave * DT * 2 * 64 + lane;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[e] = pack_f16x2(oacc[dt][8 * h + 2 * e] * inv, oacc[dt][8 * h + 2 * e + 1] * inv);
                po[(dt * 2 + h) * 64] = u32x4{w[0], w[1], w[2], w[3]};
            }
        reinterpret_cast<f32x2*>(mine + fp8_tail_o_bytes<D>())[wave * 64 + lane] = f32x2{mrow, lsum};
        return;
    }

    // Epilogue: wave w stages its rows in the 32 x D slab that is tile buffer w.
    static_assert(32 * D * 2 <= BN * D, "a tile buffer holds one wave's output rows");
    __syncthreads();
    TO* Os = reinterpret_cast<TO*>(wave == 0 ? Ka : wave == 1 ? Kb : wave == 2 ? Va : Vb);
    fp8_write_rows<D, TO>(p, b, hq, wq0, oacc, mrow, sum_xor32(lrow), vdesc, Os);
}

// Merges the pieces of the tail blocks: workgroup 4*t + w takes wave w's 32 rows of tail block t, reads
// the pieces' partials in piece order (so the result does not depend on the order the pieces ran in) and
// writes the rows as an unsplit workgroup would.  A separate launch: stream order makes every piece's
// stores visible to it, with no cache maintenance inside the attention kernel.
template <int D, typename TO>
__global__ void __launch_bounds__(64) fp8_tail_merge_kernel(const PrefillFp8Params p) {
    constexpr int DT = D / 32;
    constexpr int64_t PART = fp8_tail_part_bytes<D>();
    constexpr int NP = DT * 2;  // 16-byte pairs of 4-value groups per lane
    __shared__ __attribute__((aligned(16))) TO slab[32 * D];
    const int tb = blockIdx.x >> 2, wave = blockIdx.x & 3, lane = threadIdx.x;
    const BlockCoord bc = block_coord_at<false>(p.n_full + tb, p.B, p.Hq, p.Hkv, p.group, p.n_qblocks, p.xcd_map);
    const uint8_t* blk = p.tail_part + (int64_t)tb * p.tail_s * PART;
    // Loads are unconditional and batched over every piece (a branch per load would make each wait for the
    // one before; a loop over pieces would wait once per piece): pieces past tail_s re-read the last
    // piece's values and get weight 0.
    const int last = p.tail_s - 1;
    f32x2 ml[kFp8TailMaxPieces];
#pragma unroll
    for (int j = 0; j < kFp8TailMaxPieces; ++j)
        ml[j] = reinterpret_cast<const f32x2*>(blk + min(j, last) * PART + fp8_tail_o_bytes<D>())[wave * 64 + lane];
    float mtot = kNegInf;
#pragma unroll
    for (int j = 0; j < kFp8TailMaxPieces; ++j) mtot = fmaxf(mtot, ml[j][0]);
    float c[kFp8TailMaxPieces], ltot = 0.f;  // piece j's share of the row sum
#pragma unroll
    for (int j = 0; j < kFp8TailMaxPieces; ++j) {
        c[j] = j > last || ml[j][0] == kNegInf ? 0.f : fast_exp2(ml[j][0] - mtot) * ml[j][1];
        ltot += c[j];
    }
    f32x16 oacc[DT];
    constexpr int KC = NP < 4 ? NP : 4;  // pairs per batch: 8 pieces x 4 loads in flight
#pragma unroll
    for (int k0 = 0; k0 < NP; k0 += KC) {
        u32x4 o[kFp8TailMaxPieces][KC];
#pragma unroll
        for (int j = 0; j < kFp8TailMaxPieces; ++j) {
            const u32x4* po = reinterpret_cast<const u32x4*>(blk + min(j, last) * PART) + wave * NP * 64 + lane;
#pragma unroll
            for (int q = 0; q < KC; ++q) o[j][q] = po[(k0 + q) * 64];
        }
#pragma unroll
        for (int q = 0; q < KC; ++q) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kFp8TailMaxPieces; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f32x2 v = unpack_f16x2(o[j][q][e]);
                    acc[2 * e] += c[j] * v[0];
                    acc[2 * e + 1] += c[j] * v[1];
                }
            const int k = k0 + q;  // d tile k / 2, values 8 * (k % 2) .. +7
#pragma unroll
            for (int e = 0; e < 8; ++e) oacc[k / 2][8 * (k % 2) + e] = acc[e];
        }
    }
    fp8_write_rows<D, TO>(p, bc.b, bc.hq, bc.qb * 128 + wave * 32, oacc, mtot, ltot, p.vd[bc.b * p.Hkv + bc.hk], slab);
}

// The tail split of a non-causal launch.  A grid of `blocks` query blocks that is not a whole number of
// rounds over the GPU's workgroup slots leaves its last round partly empty, and the first round's
// workgroups end at different times (the oldest workgroup on a CU runs ahead).  The blocks of that
// last round therefore run as s key pieces each, which the hardware dispatches into whichever slots free
// up first: s = ceil(slots / tail) pieces (at most 8, at least 4 key tiles each); a second launch
// merges them.
struct Fp8TailPlan {
    int64_t grid;              // workgroups launched
    int32_t n_full, s, tiles;  // whole blocks; pieces per tail block; key tiles per piece
    int64_t n_tail;            // tail blocks (0: no split)
    size_t bytes;              // workspace: the pieces' partials
};

static Fp8TailPlan fp8_tail_plan(int64_t blocks, int64_t Sk, int64_t D, bool causal, int64_t slots) {
    Fp8TailPlan t;
    memset(&t, 0, sizeof(t));
    t.grid = blocks;
    t.n_full = (int32_t)(blocks < 0x7fffffff ? blocks : 0x7fffffff);
    t.s = 1;
    t.tiles = 1 << 30;
    const int64_t nt = (Sk + 63) / 64;
    if (causal || slots <= 0 || slots % 8 != 0 || blocks <= slots || blocks % 8 != 0 || blocks > 0x7fffffff) return t;
    const int64_t r = blocks % slots;
    if (r == 0 || 4 * r > 3 * slots) return t;  // no partly empty round, or one nearly full
    int64_t s = (slots + r - 1) / r;
    if (s > kFp8TailMaxPieces) s = kFp8TailMaxPieces;
    if (s > nt / 4) s = nt / 4;
    if (s < 2) return t;
    const int64_t tiles = (nt + s - 1) / s;
    s = (nt + tiles - 1) / tiles;  // every piece gets at least one tile
    if (s < 2) return t;
    t.n_full = (int32_t)(blocks - r);
    t.s = (int32_t)s;
    t.tiles = (int32_t)tiles;
    t.n_tail = r;
    t.grid = t.n_full + r * s;
    const int64_t part = D == 128 ? fp8_tail_part_bytes<128>() : fp8_tail_part_bytes<64>();
    t.bytes = (size_t)r * s * part;
    return t;
}

// Workgroup slots of the non-causal kernel on `device`: its occupancy per CU times the CUs.  The
// codes-input instantiation stands for all of them, so that the native path and the codes path split
// alike (and their results stay bit-identical); 0 when the runtime cannot say.
static int64_t fp8_slots(int64_t D, int device) {
    static std::atomic<int> per_cu[2] = {{0}, {0}};
    std::atomic<int>& c = per_cu[D == 128 ? 1 : 0];
    int n = c.load(std::memory_order_relaxed);
    if (n == 0) {
        const void* fn = D == 128 ? reinterpret_cast<const void*>(&prefill_fp8_kernel<128, false, uint8_t, bf16_t>)
                                  : reinterpret_cast<const void*>(&prefill_fp8_kernel<64, false, uint8_t, bf16_t>);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, 256, 0) != hipSuccess || n < 0) return 0;
        c.store(n, std::memory_order_relaxed);
    }
    dtattn_device_peaks pk;
    if (dtattn_get_device_peaks(device, &pk) != DTATTN_OK) return 0;
    return (int64_t)n * pk.cu_count;
}

static Fp8TailPlan fp8_plan_for(const dtattn_prefill_args* a, int device) {
    const int64_t blocks = (a->Sq + 127) / 128 * a->B * a->Hq;
    const bool causal = a->causal != 0;
    return fp8_tail_plan(blocks, a->Sk, a->D, causal, causal ? 0 : fp8_slots(a->D, device));
}

// Applies `tp` to the kernel parameters when `ws` holds its partials (256-byte aligned); without room
// the launch runs unsplit.
static void fp8_apply_plan(PrefillFp8Params& p, const Fp8TailPlan& tp, void* ws, size_t ws_bytes) {
    if (tp.n_tail == 0 || ws == nullptr || ws_bytes < tp.bytes || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
        return;
    p.n_full = tp.n_full;
    p.tail_s = tp.s;
    p.tail_tiles = tp.tiles;
    p.tail_part = static_cast<uint8_t*>(ws);
}

template <int D, bool CAUSAL, typename TQ, typename TO>
static int launch_fp8(const PrefillFp8Params& prm, hipStream_t stream) {
    PrefillFp8Params p = prm;
    p.n_qblocks = (p.Sq + 127) / 128;
    const int64_t blocks = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (blocks == 0) return DTATTN_OK;
    if (blocks > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: grid too large");
    const int64_t grid = p.tail_s > 1 ? p.n_full + (blocks - p.n_full) * p.tail_s : blocks;
    if (p.tail_s <= 1) p.n_full = (int32_t)blocks;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: grid too large");
    hipLaunchKernelGGL((prefill_fp8_kernel<D, CAUSAL, TQ, TO>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    const int st = check_launch("prefill_fp8_kernel");
    if (st != DTATTN_OK || CAUSAL || p.tail_s <= 1) return st;
    hipLaunchKernelGGL((fp8_tail_merge_kernel<D, TO>), dim3((unsigned)((blocks - p.n_full) * 4)), dim3(64), 0, stream, p);
    return check_launch("fp8_tail_merge_kernel");
}

template <typename TQ, typename TO>
static int dispatch_fp8(const PrefillFp8Params& p, int64_t D, bool causal, hipStream_t stream) {
    if (D == 128) return causal ? launch_fp8<128, true, TQ, TO>(p, stream) : launch_fp8<128, false, TQ, TO>(p, stream);
    if (D == 64) return causal ? launch_fp8<64, true, TQ, TO>(p, stream) : launch_fp8<64, false, TQ, TO>(p, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: head dim %lld not supported (64 or 128)", (long long)D);
}

// Kernel parameters from the ABI arguments; q/k/v pointers, strides and descales are the caller's.
static PrefillFp8Params fp8_params(const dtattn_prefill_args* a, float c, int32_t delta) {
    PrefillFp8Params p;
    memset(&p, 0, sizeof(p));
    p.q = a->q;
    p.k = reinterpret_cast<const uint8_t*>(a->k);
    p.v = reinterpret_cast<const uint8_t*>(a->v);
    p.o = a->o;
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
    p.q_and = 0xffffffffu;
    p.q_xor = 0u;
    p.tail_s = 1;
    return p;
}

static int stream_device_fp8(hipStream_t stream, int* dev) {
    return (stream == nullptr ? hipGetDevice(dev) : hipStreamGetDevice(stream, dev)) == hipSuccess ? DTATTN_OK
                                                                                               : DTATTN_ERR_DEVICE;
}

// Workspace dtattn_prefill_fwd can use for FP8 codes on `device`: the tail split's (0: none).
size_t prefill_fp8_workspace_size(const dtattn_prefill_args* a, int device) {
    if (a->B <= 0 || a->Sq <= 0 || a->Sk <= 0 || (a->D != 64 && a->D != 128)) return 0;
    return fp8_plan_for(a, device).bytes;
}

// dtattn_prefill_fwd with FP8 codes: output BF16 or FP16.
int prefill_fp8(const dtattn_prefill_args* a, float c, int32_t delta, uint32_t q_and, uint32_t q_xor,
                hipStream_t stream) {
    PrefillFp8Params p = fp8_params(a, c, delta);
    p.q_and = q_and;
    p.q_xor = q_xor;
    if (!a->causal && a->workspace != nullptr && a->Sk > 0 && (a->D == 64 || a->D == 128)) {
        int dev = 0;
        if (stream_device_fp8(stream, &dev) != DTATTN_OK) return fail(DTATTN_ERR_DEVICE, "prefill fp8: stream device");
        fp8_apply_plan(p, fp8_plan_for(a, dev), a->workspace, a->workspace_bytes);
    }
    const bool causal = a->causal != 0;
    if (a->o_dtype == DTATTN_FP16) return dispatch_fp8<uint8_t, f16_t>(p, a->D, causal, stream);
    return dispatch_fp8<uint8_t, bf16_t>(p, a->D, causal, stream);
}

// Workspace of dtattn_prefill_fp8: K and V codes [B, Hkv, Sk, D], then the per-head scales (q descale and
// factor, k and v descales) and the slice maxima of the three tensors, each region 256-byte aligned.
struct Fp8Workspace {
    size_t k8, v8, qd, qinv, kd, vd, qpart, kpart, vpart, total;
    size_t tail, tail_bytes;  // the tail split's region (after total; optional)
};
static Fp8Workspace fp8_workspace(const dtattn_prefill_args* a, int device) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    Fp8Workspace w;
    size_t off = 0;
    const size_t kv = (size_t)a->B * a->Hkv * a->Sk * a->D;
    w.k8 = off, off += up(kv);
    w.v8 = off, off += up(kv);
    w.qd = off, off += up((size_t)a->B * a->Hq * 4);
    w.qinv = off, off += up((size_t)a->B * a->Hq * 4);
    w.kd = off, off += up((size_t)a->B * a->Hkv * 4);
    w.vd = off, off += up((size_t)a->B * a->Hkv * 4);
    w.qpart = off, off += up((size_t)a->B * a->Hq * quant_slices(a->Sq) * 4);
    w.kpart = off, off += up((size_t)a->B * a->Hkv * quant_slices(a->Sk) * 4);
    w.vpart = off, off += up((size_t)a->B * a->Hkv * quant_slices(a->Sk) * 4);
    w.total = off;
    w.tail = off;
    w.tail_bytes = a->Sk > 0 && a->Sq > 0 && device >= 0 ? fp8_plan_for(a, device).bytes : 0;
    return w;
}

}  // namespace dtattn

using namespace dtattn;

extern "C" size_t dtattn_prefill_fp8_workspace_size(const dtattn_prefill_args* a) {
    if (a == nullptr || a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Sq < 0 || a->Sk < 0 || a->D <= 0) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    const Fp8Workspace w = fp8_workspace(a, a->D == 64 || a->D == 128 ? dev : -1);
    return w.total + w.tail_bytes;
}

extern "C" int dtattn_prefill_fp8(const dtattn_prefill_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill_fp8: args is NULL");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: inputs must be bf16 or fp16 (dtype %d)", a->dtype);
    if (a->o_dtype != a->dtype) return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: output dtype must equal input dtype");
    if (a->mask != nullptr) return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: an attention mask is not supported");
    if (a->B < 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Sq < 0 || a->Sk < 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill_fp8: bad sizes");
    if (a->Hq % a->Hkv != 0) return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill_fp8: Hq is not a multiple of Hkv");
    if (a->D != a->Dv || (a->D != 64 && a->D != 128))
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: head dim %lld / %lld not supported (64 or 128, D == Dv)",
                    (long long)a->D, (long long)a->Dv);
    if (a->Sq > (1 << 29) || a->Sk > (1 << 29) || a->B * a->Hq > 65535 || a->B * a->Hkv > 65535)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: sizes too large");
    if (a->B == 0 || a->Sq == 0) return DTATTN_OK;
    if (a->q == nullptr || a->o == nullptr || (a->Sk > 0 && (a->k == nullptr || a->v == nullptr)))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill_fp8: null tensor pointer");
    const int64_t* strides[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 3; ++j)
            if ((strides[i][j] * 2) % 16 != 0)
                return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: strides must be multiples of 16 bytes");
    if (((reinterpret_cast<uintptr_t>(a->q) | reinterpret_cast<uintptr_t>(a->k) | reinterpret_cast<uintptr_t>(a->v) |
          reinterpret_cast<uintptr_t>(a->o)) & 15u) != 0)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill_fp8: tensors must be 16-byte aligned");
    ScalePlan sp;
    const int sst = plan_scale(a->scale, a->D, kSign16, &sp);  // q is rounded from its 16-bit rows
    if (sst != DTATTN_OK) return sst;
    int dev = 0;
    if (stream_device_fp8(stream, &dev) != DTATTN_OK) return fail(DTATTN_ERR_DEVICE, "prefill_fp8: stream device");
    const Fp8Workspace w = fp8_workspace(a, dev);
    if (a->workspace == nullptr || a->workspace_bytes < w.total || (reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
        return fail(DTATTN_ERR_WORKSPACE, "prefill_fp8: a 256-byte aligned workspace of %zu bytes is required, %zu given",
                    w.total, a->workspace_bytes);
    char* ws = static_cast<char*>(a->workspace);

    // 1-2. per-head maxima of q, k, v; K/V codes and every scale (q: scales only)
    QuantParams qp;
    memset(&qp, 0, sizeof(qp));
    qp.B = (int32_t)a->B;
    qp.D = (int32_t)a->D;
    // tensors q (scales only), k, v; with no keys only q's scales are needed
    const void* src[3] = {a->q, a->k, a->v};
    const int64_t* st[3] = {a->q_stride, a->k_stride, a->v_stride};
    const int64_t H[3] = {a->Hq, a->Hkv, a->Hkv}, S[3] = {a->Sq, a->Sk, a->Sk};
    const size_t codes[3] = {0, w.k8, w.v8}, desc[3] = {w.qd, w.kd, w.vd}, part[3] = {w.qpart, w.kpart, w.vpart};
    for (int i = 0; i < 3; ++i) {
        QuantTensor& t = qp.t[i];
        t.x = src[i];
        t.x8 = i > 0 ? reinterpret_cast<uint8_t*>(ws + codes[i]) : nullptr;
        t.descale = reinterpret_cast<float*>(ws + desc[i]);
        t.inv = i == 0 ? reinterpret_cast<float*>(ws + w.qinv) : nullptr;
        t.part = reinterpret_cast<float*>(ws + part[i]);
        t.xs_b = st[i][0], t.xs_h = st[i][1], t.xs_s = st[i][2];
        t.H = (int32_t)H[i], t.S = (int32_t)S[i];
        t.nslice = quant_slices(S[i]);
    }
    const int rc = fp8_quantize_batch(qp, a->Sk > 0 ? 3 : 1, a->dtype, stream);
    if (rc != DTATTN_OK) return rc;

    // 3. attention on the codes, Q rounded in the kernel
    const float scale = sp.scale;
    int64_t delta64 = a->q_offset - a->k_offset;
    const int64_t lim = a->Sq + a->Sk + 1;
    delta64 = delta64 > lim ? lim : (delta64 < -lim ? -lim : delta64);
    dtattn_prefill_args codes_args = *a;
    codes_args.k = ws + w.k8;
    codes_args.v = ws + w.v8;
    codes_args.k_stride[0] = a->Hkv * a->Sk * a->D, codes_args.k_stride[1] = a->Sk * a->D, codes_args.k_stride[2] = a->D;
    codes_args.v_stride[0] = codes_args.k_stride[0], codes_args.v_stride[1] = codes_args.k_stride[1];
    codes_args.v_stride[2] = a->D;
    codes_args.q_descale = reinterpret_cast<const float*>(ws + w.qd);
    codes_args.k_descale = reinterpret_cast<const float*>(ws + w.kd);
    codes_args.v_descale = reinterpret_cast<const float*>(ws + w.vd);
    PrefillFp8Params p = fp8_params(&codes_args, scale * kLog2e, (int32_t)delta64);
    p.qinv = reinterpret_cast<const float*>(ws + w.qinv);
    p.q_and = sp.q_and;
    p.q_xor = sp.q_xor;
    const bool causal = a->causal != 0;
    if (!causal && a->Sk > 0) {
        const size_t room = a->workspace_bytes - w.tail;
        fp8_apply_plan(p, fp8_plan_for(a, dev), ws + w.tail, room);
    }
    if (a->dtype == DTATTN_BF16) return dispatch_fp8<bf16_t, bf16_t>(p, a->D, causal, stream);
    return dispatch_fp8<f16_t, f16_t>(p, a->D, causal, stream);
}
