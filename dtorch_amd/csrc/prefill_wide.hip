// Attention forward for wide heads (kernel head dims 256, 512) on bf16 / fp16 MFMA, with per-row LSE.
//
// The arithmetic of SdpaOp::Compute (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:
// 107-109) at head dims where the main kernel's plan (32 query rows per wave, Q and O of the full head
// in registers) needs more than 512 registers per wave.  The reference reaches it through the VAE
// mid-block attention of its diffusers ports: one head of block_out_channels[-1] = 512 dimensions
// (python/dtorch/applications/huggingface/diffusers/models/unets/unet_2d_blocks.py:126-140).
//
// Work decomposition: a workgroup of 2 NRG waves owns 32 NRG query rows of one (batch, query head): NRG
// row groups of 32 rows, each handled by a pair of waves that split the head dims in halves.  Wave
// (rg, dh) holds Q and accumulates O for rows 32 rg .. 32 rg + 31 and dims [dh D/2, (dh + 1) D/2):
//   - S^T = K Q^T is the sum of the pair's two halves: each wave computes its partial 32x32 tile with
//     v_mfma_f32_32x32x16, writes it to LDS, and after one barrier adds its partner's.  Both waves of
//     the pair then hold the same scores and run the same softmax, so no further exchange is needed.
//   - O^T = V^T P^T for the wave's half, with V^T read by ds_read_b64_tr_b16 as in the main kernel.
// Per 32-key tile a wave reads half of K and V plus one partner partial from LDS: about 40 KB per 32
// MFMAs at D = 512, against 36 KB per 16 MFMAs when four waves split the score reduction.
//   D = 256: NRG = 4, 8 waves (two per SIMD, one workgroup per CU), each K/V tile shared by 128 rows;
//            64 KB of tiles plus a 32 KB exchange.
//   D = 512: NRG = 2, 4 waves with up to 512 registers each (64 of Q and 128 of O per wave do not fit
//            the 256 of two waves per SIMD); 128 KB of tiles plus a 16 KB exchange, 64 rows per tile.
// Key tiles of 32 rows, K and V double-buffered through direct buffer->LDS loads.
#include "dtattn_common.hpp"
#include "prefill_params.hpp"

namespace dtattn {

// 16-byte chunk swizzle of LDS row r: distinct over any 16 consecutive rows (the K reads take one chunk of
// 16 rows per step) and differing above the low two bits for 4 consecutive rows (a transposed V read
// takes 4 aligned chunks of 4 rows); rows are whole multiples of 256 bytes, so every row starts on bank 0.
__device__ __forceinline__ int wswz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// PAD: real head dims below D (multiples of 8, Dv may differ from D), as in the main kernel: Q/K chunks
// past p.qk_ch and V chunks past p.v_ch load as zeros, O chunks past p.v_ch are not stored.
template <typename T, int D, int NRG, bool CAUSAL, bool MASKED, bool PAD>
__global__ void __launch_bounds__(64 * 2 * NRG, 1) prefill_wide_kernel(const PrefillParams p) {
    constexpr int NW = 2 * NRG;
    constexpr int BN = 32;           // keys per tile
    constexpr int BM = 32 * NRG;     // query rows per workgroup
    constexpr int DH = D / 2;        // dimensions per wave
    constexpr int DCH = D / 8;       // 16-byte chunks per row
    constexpr int KSTEPS = DH / 16;  // S^T k-steps per wave
    constexpr int DT = DH / 32;      // 32-row d tiles of the wave's O^T
    static_assert(D == 256 || D == 512, "wide head dims");
    static_assert(NRG >= 1 && NRG <= 4, "a tile buffer stages each row group's output");
    typedef typename Elem<T>::vec8 V8;
    typedef typename Elem<T>::vec4 V4;
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

    __shared__ __attribute__((aligned(16))) T Ka[BN * D];
    __shared__ __attribute__((aligned(16))) T Kb[BN * D];
    __shared__ __attribute__((aligned(16))) T Va[BN * D];
    __shared__ __attribute__((aligned(16))) T Vb[BN * D];
    // Partial scores, one 64 x 16 fp32 slab per wave; lane l's 16-byte chunk j at l * 16 + 4 (j ^ ((l >> 2) & 3)).
    // Lane l's slab starts on bank 16 (l & 3), so the XOR with bits 2-3 of the lane index puts the 16 lanes
    // of one 16-byte access pass on 16 distinct 16-byte bank groups.
    __shared__ __attribute__((aligned(16))) float Sx[NW * 64 * 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave >> 1;  // row group
    const int dh = wave & 1;   // half of the head dims
    const int l32 = lane & 31;
    const int hf = lane >> 5;
    const int d0 = dh * DH;    // first dimension of this wave's half

    const BlockCoord bc = block_coord<CAUSAL>(p);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;
    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const T* kp = reinterpret_cast<const T*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const T* vp = reinterpret_cast<const T*>(p.v) + b * p.vs_b + hk * p.vs_h;
    const int q0 = qb * BM;
    const int wq0 = q0 + rg * 32;  // first row of this wave's row group

    // Key block of this workgroup (the whole key range unless split): tiles t0 .. nt - 1, indexed from
    // key 0 so that tile t always holds keys 32 t .. 32 t + 31.
    const int split = blockIdx.y;
    const int kb0 = split * p.kblock;
    int kend = min(p.Sk, kb0 + p.kblock);
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;  // keys < lim can be visible
        kend = lim < 0 ? 0 : (lim < kend ? lim : kend);
    }
    const int t0 = kb0 / BN;
    const int nt = kend > kb0 ? (kend + BN - 1) / BN : t0;

    // Q fragment of the wave's half (B operand of S^T), loaded after the first tile's loads are issued
    V8 qf[KSTEPS];
    f32x16 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
    float mrow = kNegInf, lrow = 0.f;

    const int krow = (int)(p.ks_s * (int64_t)sizeof(T));
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(T));

    // Tile t -> LDS (lane l -> byte 16*l of a 1 KB block, 1024 / (2 D) rows per instruction), chunk c of
    // row r at c ^ wswz(r); rows past Sk read zeros, and so do chunks at or past valid_ch (PAD).  The
    // resource ends where the tile's last valid row ends.
    auto dma = [&](T* dst, const T* base, int pitch, int64_t stride, int t, int valid_ch) {
        constexpr int ROWS_PER_INSTR = 1024 / (2 * D);
        constexpr int INSTR = BN / ROWS_PER_INSTR / NW;
        static_assert(INSTR >= 1, "at least one load per wave");
        const int rows = min(BN, p.Sk - t * BN);
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + (PAD ? valid_ch * 16 : D * (int)sizeof(T)));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int r0 = (wave * INSTR + i) * ROWS_PER_INSTR;
            const int r = r0 + lane / DCH;
            const int c = (lane % DCH) ^ wswz(r);
            const uint32_t off = (PAD && c >= valid_ch) ? nbytes : (uint32_t)(r * pitch + c * 16);
            buf_ld16_lds_async(rs, dst + r0 * D, off);
        }
    };

    constexpr int DMA_ROWS = 1024 / (2 * D);             // rows per load instruction
    constexpr int DMA_INSTR = BN / DMA_ROWS / NW;  // per wave, per tensor and tile
    static_assert(DMA_INSTR >= 1, "at least one load per wave");
    // At D = 512 (one wave per SIMD) tile t+1's loads are spread over tile t's MFMAs: K's between the S
    // MFMAs, V's after the PV block.  Issued in one burst at the tile start, a wave's 16 one-row loads
    // stalled its issue for ~1,700 cycles while the memory pipeline took them, with no other wave on the
    // SIMD.  That form uses the compiler-tracked load, which the scheduler can place between MFMAs.  The
    // D = 256 kernels keep the untracked burst, and so do the masked ones: their mask loads are tracked too,
    // and since the memory counter retires in order, each wait for a mask value would also wait for the
    // tile loads issued before it (5 to 33 waits per tile in the generated code).  Causal D = 512 kernels
    // keep it as well: the spread form measured 28-31% slower there (1x8x2048, D = 512 and 320).
    constexpr bool kSpreadDma = D >= 512 && !MASKED && !CAUSAL;
    // Resource over tile t's rows below kend (the workgroup's key block, or the causal limit inside it).
    // Past the block's last tile it covers nothing: every load is then out of range, touches no memory and
    // lands zeros in a buffer no wave reads again.  Rows of the last tile at or past kend are masked for
    // every query of the workgroup, so they load as zeros too.
    auto dma_rs = [&](const T* base, int pitch, int64_t stride, int t, int valid_ch, uint32_t* nb) {
        const int rows = min(BN, kend - t * BN);
        *nb = rows > 0 ? (uint32_t)((rows - 1) * pitch + (PAD ? valid_ch * 16 : D * (int)sizeof(T))) : 0u;
        return make_rsrc(base + (rows > 0 ? (int64_t)t * BN * stride : 0), *nb);
    };
    // Load i of this wave's share of a tile, in the tracked form.
    auto dma_one = [&](T* dst, __amdgpu_buffer_rsrc_t rs, uint32_t nbytes, int pitch, int valid_ch, int i) {
        const int r0 = (wave * DMA_INSTR + i) * DMA_ROWS;
        const int r = r0 + lane / DCH;
        const int c = (lane % DCH) ^ wswz(r);
        const uint32_t off = (PAD && c >= valid_ch) ? nbytes : (uint32_t)(r * pitch + c * 16);
        buf_ld16_lds(rs, dst + r0 * D, off);
    };

    // V^T reads (ds_read_b64_tr_b16), as in the main kernel: within each 16-lane block, lane 4j+a
    // addresses key K0+j, d-segment D0+4a.
    const int blk = lane >> 4, bl = lane & 15;
    const int tr_key = bl >> 2;
    const int tr_d = 16 * (blk & 1) + 4 * (bl & 3);
    const int tr_k4 = 4 * (blk >> 1);

    const float* mbase_p = MASKED ? p.mask + b * p.ms_b + hq * p.ms_h : nullptr;
    const auto mrs = make_rsrc(mbase_p, MASKED ? (uint32_t)((((int64_t)(p.Sq - 1) * p.ms_l + p.Sk) * 4)) : 0u);
    const uint32_t mrow_off = MASKED ? (uint32_t)((int64_t)min(wq0 + l32, p.Sq - 1) * p.ms_l * 4) : 0u;

    float* sx_mine = Sx + (wave * 64 + lane) * 16;
    const float* sx_partner = Sx + ((wave ^ 1) * 64 + lane) * 16;
    const int sxs = (lane >> 2) & 3;  // chunk swizzle of this lane's slab

    auto tile = [&](const T* Kc, const T* Vc, T* Kn, T* Vn, int t) {
        wait_vmem();
        lds_barrier();  // tile t landed; every wave finished tile t-1, including its exchange reads
        uint32_t knb = 0, vnb = 0;
        const auto krs_n = dma_rs(kp, krow, p.ks_s, t + 1, p.qk_ch, &knb);
        const auto vrs_n = dma_rs(vp, vrow, p.vs_s, t + 1, p.v_ch, &vnb);
        if constexpr (!kSpreadDma) {
            if (t + 1 < nt) {
                dma(Kn, kp, krow, p.ks_s, t + 1, p.qk_ch);
                dma(Vn, vp, vrow, p.vs_s, t + 1, p.v_ch);
            }
        }
        const int kbase = t * BN;
        // Every row of this row group precedes the tile: the pair skips it together (both waves still
        // reach the exchange barrier below).
        const bool skip = CAUSAL && kbase > wq0 + 31 + p.delta;
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > wq0 + p.delta));
        u32x4 mraw[4];
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < 4; ++g) mraw[g] = buf_ld16(mrs, mrow_off + (uint32_t)((kbase + 8 * g + 4 * hf) * 4));
        }
        // partial S^T over this wave's half
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.f;
        if (skip) {
            if constexpr (kSpreadDma) {
#pragma unroll
                for (int i = 0; i < DMA_INSTR; ++i) dma_one(Kn, krs_n, knb, krow, p.qk_ch, i);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                const int r = l32;
                const int c = (d0 + ks * 16 + hf * 8) >> 3;
                const V8 a = *reinterpret_cast<const V8*>(Kc + r * D + 8 * (c ^ wswz(r)));
                s = Elem<T>::mfma32(a, qf[ks], s);
            }
            // K fragment reads run four MFMAs ahead of their use: at D = 512 the wave runs alone on its
            // SIMD, so an LDS read that has not returned stalls the matrix pipe (two ahead: 8% slower)
            if constexpr (kSpreadDma) {
                // tile t+1's K loads, one after every KSTEPS / DMA_INSTR MFMAs
#pragma unroll
                for (int i = 0; i < DMA_INSTR; ++i) dma_one(Kn, krs_n, knb, krow, p.qk_ch, i);
                constexpr int EVERY = KSTEPS / DMA_INSTR;
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
                for (int i = 0; i < KSTEPS; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (i < KSTEPS - 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (i % EVERY == EVERY - 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            } else {
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
                for (int i = 0; i < KSTEPS - 4; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(sx_mine + 4 * (j ^ sxs)) =
                    f32x4{s[4 * j], s[4 * j + 1], s[4 * j + 2], s[4 * j + 3]};
        }
        lds_barrier();  // every partial written
        if (skip) {
            if constexpr (kSpreadDma) {
#pragma unroll
                for (int i = 0; i < DMA_INSTR; ++i) dma_one(Vn, vrs_n, vnb, vrow, p.v_ch, i);
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(sx_partner + 4 * (j ^ sxs));
            s[4 * j] += x.x, s[4 * j + 1] += x.y, s[4 * j + 2] += x.z, s[4 * j + 3] += x.w;
        }
        // Element i of s holds key kbase + 8*(i/4) + 4*hf + i%4 of query wq0 + l32.
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 m = __builtin_bit_cast(f32x4, mraw[g]);
                s[4 * g + 0] += m.x * p.inv_scale;
                s[4 * g + 1] += m.y * p.inv_scale;
                s[4 * g + 2] += m.z * p.inv_scale;
                s[4 * g + 3] += m.w * p.inv_scale;
            }
        }
        if (need_mask) {
            int lim = p.Sk - 1 - kbase;
            if (CAUSAL) lim = min(lim, wq0 + l32 + p.delta - kbase);
            lim -= 4 * hf;
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (8 * (i >> 2) + (i & 3) > lim) s[i] = kNegInf;
        }
        float mx = kNegInf;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
        mx = max_xor32(mx);
        const float mcand = fmaxf(mrow, mx * p.c);
        if (__any(mcand - mrow > kRescaleThreshold)) {  // wave-uniform (and the same in both waves of the pair)
            const float alpha = fast_exp2(mrow - (mcand == kNegInf ? 0.f : mcand));
            mrow = mcand;
            lrow *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
        }
        const float mbase = (mrow == kNegInf) ? 0.f : mrow;
        V8 pb[2];
        float ls = lrow;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            V8 pk;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pv = fast_exp2(__builtin_fmaf(s[8 * half + e], p.c, -mbase));
                ls += pv;
                pk[e] = Elem<T>::from_f32(pv);
            }
            pb[half] = pk;
        }
        lrow = ls;
        // O^T (this wave's half) += V^T P^T: k-step ks covers keys 16 ks .. 16 ks + 15
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int d = d0 + dt * 32 + tr_d;
                const int k1 = ks * 16 + tr_k4 + tr_key;
                const int k2 = k1 + 8;
                const V4 lo = __builtin_bit_cast(
                    V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vc + k1 * D + 8 * ((d >> 3) ^ wswz(k1)) + (d & 7))));
                const V4 hi = __builtin_bit_cast(
                    V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vc + k2 * D + 8 * ((d >> 3) ^ wswz(k2)) + (d & 7))));
                const V8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                oacc[dt] = Elem<T>::mfma32(a, pb[ks], oacc[dt]);
            }
        }
        if constexpr (kSpreadDma) {  // tile t+1's V loads (they stay after the V^T reads of this buffer's twin)
#pragma unroll
            for (int i = 0; i < DMA_INSTR; ++i) dma_one(Vn, vrs_n, vnb, vrow, p.v_ch, i);
        }
        // V^T reads (two per MFMA) run two MFMAs ahead (one ahead: 8% slower at D = 512, 6-9% at D = 256;
        // three ahead: no faster).  Spreading the exponentials of P chunk 1 over these MFMAs measured
        // 4-7% slower than computing P first.
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 2 * DT - 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    };

    if (nt > t0) {
        if constexpr (kSpreadDma) {  // one form of the load per kernel: the tracked one sets m0 itself
            uint32_t kb0 = 0, vb0 = 0;
            const auto krs0 = dma_rs(kp, krow, p.ks_s, t0, p.qk_ch, &kb0);
            const auto vrs0 = dma_rs(vp, vrow, p.vs_s, t0, p.v_ch, &vb0);
#pragma unroll
            for (int i = 0; i < DMA_INSTR; ++i) dma_one(Ka, krs0, kb0, krow, p.qk_ch, i);
#pragma unroll
            for (int i = 0; i < DMA_INSTR; ++i) dma_one(Va, vrs0, vb0, vrow, p.v_ch, i);
        } else {
            dma(Ka, kp, krow, p.ks_s, t0, p.qk_ch);
            dma(Va, vp, vrow, p.vs_s, t0, p.v_ch);
        }
    }
    // Lane holds query l32, d = d0 + ks*16 + hf*8 .. +8.  Unconditional loads issue back to back and share
    // the first tile's memory latency (a branch per load serialised them).  Rows past Sq read row Sq-1 and
    // chunks past qk_ch read the half's first chunk; the mask zeroes both.
    {
        const int qrow = wq0 + l32;
        const bool row_ok = qrow < p.Sq;
        const T* qsrc = qp + (int64_t)(row_ok ? qrow : p.Sq - 1) * p.qs_s + d0;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const bool ok = row_ok && (!PAD || (d0 >> 3) + 2 * ks + hf < p.qk_ch);
            const u32x4 w = ld16(qsrc + (ok ? ks * 16 + hf * 8 : 0));
            qf[ks] = __builtin_bit_cast(V8, q_bits(w, ok ? p.q_and : 0u, ok ? p.q_xor : 0u));
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): Q and the first tile, visibly to the compiler
    for (int t = t0; t < nt; t += 2) {
        tile(Ka, Va, Kb, Vb, t);
        if (t + 1 < nt) tile(Kb, Vb, Ka, Va, t + 1);
    }

    // Epilogue: row group rg stages its 32 output rows in tile buffer rg (row r, 16-byte chunk c at
    // c ^ (r % 16)), each wave its half, then all threads store whole rows.
    static_assert(32 <= BN, "a tile buffer holds one row group's output rows");
    __syncthreads();
    T* Os = rg == 0 ? Ka : rg == 1 ? Kb : rg == 2 ? Va : Vb;
    {
        const float l = sum_xor32(lrow);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int row = l32;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                V4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = Elem<T>::from_f32(oacc[dt][4 * i4 + e] * inv);
                const int c = (d0 >> 3) + dt * 4 + i4;
                *reinterpret_cast<V4*>(Os + row * D + 8 * (c ^ (row & 15)) + 4 * hf) = o4;
            }
        if (dh == 0 && p.lse != nullptr && hf == 0) {
            const int qrow = wq0 + row;
            if (qrow < p.Sq)
                p.lse[split * p.lses_split + b * p.lses_b + hq * p.lses_h + qrow] =
                    l > 0.f ? (mrow + __log2f(l)) * kLn2 : kNegInf;
        }
    }
    __syncthreads();
    T* op = reinterpret_cast<T*>(p.o) + split * p.os_split + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < BM * DCH / (64 * NW); ++it) {
        const int id = it * 64 * NW + tid;
        const int row = id / DCH, c = id % DCH;  // row of the workgroup's BM
        const int qrow = q0 + row;
        const T* src = (row < 32 ? Ka : row < 64 ? Kb : row < 96 ? Va : Vb) + (row & 31) * D;
        if (qrow < p.Sq && (!PAD || c < p.v_ch))
            st16(op + (int64_t)qrow * p.os_s + c * 8, ld16(src + 8 * (c ^ (row & 15))));
    }
}

// Row groups per workgroup: see the kernel's header.
template <int D>
constexpr int wide_row_groups() { return D == 512 ? 2 : 4; }

template <typename T, int D, bool CAUSAL, bool MASKED, bool PAD>
static int launch_wide(const PrefillParams& prm, hipStream_t stream) {
    constexpr int NRG = wide_row_groups<D>();
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + 32 * NRG - 1) / (32 * NRG);
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_wide_kernel<T, D, NRG, CAUSAL, MASKED, PAD>), dim3((unsigned)grid, (unsigned)p.nsplit),
                       dim3(64 * 2 * NRG), 0, stream, p);
    return check_launch("prefill_wide_kernel");
}

template <typename T, bool MASKED, bool PAD>
static int dispatch_wide_m(const PrefillParams& p, int D, bool causal, hipStream_t stream) {
    if (D == 256)
        return causal ? launch_wide<T, 256, true, MASKED, PAD>(p, stream)
                      : launch_wide<T, 256, false, MASKED, PAD>(p, stream);
    if (D == 512)
        return causal ? launch_wide<T, 512, true, MASKED, PAD>(p, stream)
                      : launch_wide<T, 512, false, MASKED, PAD>(p, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill: kernel head dim %d not supported (64, 128, 256 or 512)", D);
}

template <typename T>
static int dispatch_wide(const PrefillParams& p, int D, bool causal, bool pad, hipStream_t stream) {
    if (pad)
        return p.mask != nullptr ? dispatch_wide_m<T, true, true>(p, D, causal, stream)
                                 : dispatch_wide_m<T, false, true>(p, D, causal, stream);
    return p.mask != nullptr ? dispatch_wide_m<T, true, false>(p, D, causal, stream)
                             : dispatch_wide_m<T, false, false>(p, D, causal, stream);
}

// Key blocks for a wide-head launch of kernel head dim D: the wide kernel runs one workgroup per CU, so
// a grid of at most half the CU count runs its keys as blocks of whole 32-key tiles (at least 256 keys,
// at most 8 blocks), in one launch with the blocks on grid.y, about one full round of workgroups.
int wide_key_splits(int64_t B, int64_t Hq, int64_t Sq, int64_t Sk, int D, int cu_count) {
    const int64_t rows = D == 512 ? 32 * wide_row_groups<512>() : 32 * wide_row_groups<256>();
    const int64_t wgs = (Sq + rows - 1) / rows * B * Hq;
    if (wgs <= 0 || cu_count <= 0 || wgs * 2 > cu_count) return 1;
    int64_t n = cu_count / wgs;
    n = n < Sk / 256 ? n : Sk / 256;
    n = n < 8 ? n : 8;
    return n > 1 ? (int)n : 1;
}

bool prefill_wide512_fits(const PrefillParams& p);
int prefill_wide512(const PrefillParams& p, bool f16, hipStream_t stream);

// Entry from dtattn_prefill_fwd for kernel head dims 256 / 512 with bf16 or fp16 inputs.  p.nsplit and
// p.kblock are set by the caller (1 and Sk when unsplit).  Non-causal head-dim-512 calls without mask or
// padding run the software-pipelined kernel of prefill_wide512.hip (the same arithmetic).
int prefill_wide(const PrefillParams& p, int D, bool causal, bool bf16, bool pad, hipStream_t stream) {
    if (D == 512 && !causal && !pad && p.mask == nullptr && prefill_wide512_fits(p))
        return prefill_wide512(p, !bf16, stream);
    return bf16 ? dispatch_wide<bf16_t>(p, D, causal, pad, stream) : dispatch_wide<f16_t>(p, D, causal, pad, stream);
}

}  // namespace dtattn
