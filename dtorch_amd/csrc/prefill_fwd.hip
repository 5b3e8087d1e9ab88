// Flash-style attention forward for gfx950 (bf16 / fp16 MFMA), with per-row LSE.
//
// Replaces the arithmetic of SdpaOp::Compute (the libtorch call at
// dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109) on the GPU.
//
// Work decomposition
//   One workgroup = 4 waves = 4*QT*32 consecutive query rows of one (batch, query head).  Each wave
//   owns QT tiles of 32 queries and keeps their Q fragments in registers for the whole kernel.
//   Key/value tiles of 64 rows are staged through LDS and shared by the 4 waves.
//
// Layout trick
//   The score tile is computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_{bf16,f16}: the
//   accumulator column (lane % 32) is the query, so each lane holds 16 keys of one query row and the
//   row max needs one cross-half exchange (v_permlane32_swap) instead of a 32-lane reduction.  The
//   output is accumulated transposed as well, O^T = V^T P^T: P^T comes straight from the score
//   registers (the MFMA reduction index is a free permutation, matched on both operands), and the V^T
//   operand is read from the row-major V tile with ds_read_b64_tr_b16 (LDS transpose read).  The
//   per-query rescale factor is then a per-lane scalar.
//
// LDS: K and V tiles of 64 rows, double-buffered, filled by direct buffer->LDS loads (no VGPR
// staging); 16-byte chunk c of row r sits at chunk c ^ kswz(r), which keeps both the 16-byte K reads
// and the 8-byte transposed V reads free of bank conflicts.
//
// Pipeline per key tile j (one barrier per tile):
//   wait own loads + barrier | K[j+1], V[j+1] -> LDS (async) | S^T = K[j] Q^T | softmax |
//   O^T += V^T(j) P^T(j)
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "dtattn_common.hpp"
#include "prefill_params.hpp"

namespace dtattn {

// XOR swizzle of the 16-byte chunk index of LDS row r (K and V tiles).  It is distinct over any 16
// consecutive rows (the 16-byte K reads take one chunk of 16 rows per step) and differs above the
// low two bits for 4 consecutive rows (a transposed V read takes 4 aligned chunks of 4 rows).  With
// 128-byte rows (D = 64) two rows share a 256-byte bank row, so the pattern is applied per row pair.
template <int D>
__device__ __forceinline__ int kswz(int r) {
    return D >= 128 ? 4 * (r & 3) + ((r >> 2) & 3) : 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}

// PAD: the real head dims are below D (any multiple of 8, Dv may differ from D); Q/K chunks past
// p.qk_ch and V chunks past p.v_ch load as zeros, and O chunks past p.v_ch are not stored.
template <typename T, int D, int QT, bool CAUSAL, bool MASKED, bool PAD>
__global__ void __launch_bounds__(256, 2) prefill_fwd_kernel(const PrefillParams p) {
    constexpr int NW = 4;
    constexpr int BN = 64;
    constexpr int BM = NW * 32;
    constexpr int DCH = D / 8;            // 16-byte chunks per row
    constexpr int KSTEPS = D / 16;        // MFMA k-steps of S^T = K Q^T
    constexpr int DT = D / 32;            // 32-row d tiles of O^T
    constexpr int KT = BN / 32;           // 32-key tiles per key block
    constexpr int PVS = BN / 16;          // MFMA k-steps of O^T = V^T P^T
    static_assert(QT == 1, "one 32-query tile per wave");
    typedef typename Elem<T>::vec8 V8;
    typedef typename Elem<T>::vec4 V4;
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

    // K and V tiles, double-buffered, each [64 keys][D] with 16-byte chunk c of row r at c ^ kswz(r).
    // Four distinct LDS objects so the compiler's alias analysis can tell an in-flight load into one
    // buffer from the reads of the others.
    __shared__ __attribute__((aligned(16))) T Ka[BN * D];
    __shared__ __attribute__((aligned(16))) T Kb[BN * D];
    __shared__ __attribute__((aligned(16))) T Va[BN * D];
    __shared__ __attribute__((aligned(16))) T Vb[BN * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS bases stay scalar
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const BlockCoord bc = block_coord<CAUSAL>(p);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;

    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const T* kp = reinterpret_cast<const T*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const T* vp = reinterpret_cast<const T*>(p.v) + b * p.vs_b + hk * p.vs_h;

    const int q0 = qb * BM;
    const int wq0 = q0 + wave * 32;

    int kend = p.Sk;
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;  // keys < lim can be visible
        kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
    }
    const int nt = (kend + BN - 1) / BN;

    V8 qf[KSTEPS];  // Q fragments (B operand of S^T = K Q^T), loaded after tile 0's loads are issued

    f32x16 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
    float mrow = kNegInf, lrow = 0.f;

    const int krow = (int)(p.ks_s * (int64_t)sizeof(T));  // row pitch in bytes (< 2^25, host-checked)
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(T));

    // Tile t of K or V -> LDS by direct buffer->LDS loads: one wave instruction fills 1 KB of LDS (lane
    // l -> byte 16*l), i.e. 1024/(2*D) rows, so lane l loads the global chunk that belongs at its LDS
    // slot, c = slot ^ kswz(row).  The buffer resource covers the tile's valid rows; rows past Sk
    // read zeros, and so do chunks at or past valid_ch (PAD), whose offset is the resource's size.
    auto dma = [&](T* dst, const T* base, int pitch, int64_t stride, int t, int valid_ch) {
        constexpr int ROWS_PER_INSTR = 1024 / (2 * D);
        constexpr int INSTR = BN / ROWS_PER_INSTR / NW;  // per wave
        const int rows = min(BN, p.Sk - t * BN);
        // the resource ends where the tile's last valid row ends (its real width under PAD)
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + (PAD ? valid_ch * 16 : D * (int)sizeof(T)));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int r0 = (wave * INSTR + i) * ROWS_PER_INSTR;
            const int r = r0 + lane / DCH;
            const int c = (lane % DCH) ^ kswz<D>(r);
            const uint32_t off = (PAD && c >= valid_ch) ? nbytes : (uint32_t)(r * pitch + c * 16);
            buf_ld16_lds_async(rs, dst + r0 * D, off);
        }
    };

    // V^T fragments for the PV MFMA come straight from the row-major V tile with ds_read_b64_tr_b16:
    // within each 16-lane block, lane 4j+a addresses key K0+j, d-segment D0+4a, and lane i then
    // receives V[K0..K0+3][D0+i] -- one d and four consecutive keys, the A-operand slot layout.
    const int blk = lane >> 4, bl = lane & 15;
    const int tr_key = bl >> 2;                 // j
    const int tr_d = 16 * (blk & 1) + 4 * (bl & 3);  // D0 offset within the 32-d tile + 4a
    const int tr_k4 = 4 * (blk >> 1);           // 4 * hf

    // MASKED: the mask slab of (b, hq) behind a buffer resource, so reads past its last row return 0
    // (those keys are hidden by the ragged-tail mask anyway).  Lane (l32, hf) reads, for query row
    // wq0 + l32, the four consecutive keys of each of its 4 groups per 32-key tile.
    const float* mbase_p = MASKED ? p.mask + b * p.ms_b + hq * p.ms_h : nullptr;
    const auto mrs = make_rsrc(mbase_p, MASKED ? (uint32_t)((((int64_t)(p.Sq - 1) * p.ms_l + p.Sk) * 4)) : 0u);
    const uint32_t mrow_off = MASKED ? (uint32_t)((int64_t)min(wq0 + l32, p.Sq - 1) * p.ms_l * 4) : 0u;

    // One key tile.  Kc/Vc hold tile t; Kn/Vn receive tile t+1.
    auto tile = [&](const T* Kc, const T* Vc, T* Kn, T* Vn, int t) {
        wait_vmem();
        lds_barrier();  // tile t landed everywhere; every wave finished tile t-1 (so Kn/Vn are free)
        auto next_tile = [&]() {
            if (t + 1 < nt) {
                dma(Kn, kp, krow, p.ks_s, t + 1, p.qk_ch);
                dma(Vn, vp, vrow, p.vs_s, t + 1, p.v_ch);
            }
        };
        // Issue point of the next tile's loads: at the tile start in the causal kernel; after this tile's
        // S block in the non-causal one (measured +2.5% at 256-512 keys, neutral on long rows; the causal
        // kernel would spill); masked kernels after the mask add (the compiler's wait for the mask values
        // would otherwise also wait for the tile loads).
        constexpr bool kLateLoads = MASKED || !CAUSAL;
        if constexpr (!kLateLoads) next_tile();
        const int kbase = t * BN;
        if (CAUSAL && kbase > wq0 + 31 + p.delta) {  // every row of this wave precedes the tile
            if constexpr (kLateLoads) next_tile();
            return;
        }
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > wq0 + p.delta));
        u32x4 mraw[KT * 4];
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < KT * 4; ++g)  // keys kbase + 32*(g/4) + 8*(g%4) + 4*hf .. +3
                mraw[g] = buf_ld16(mrs, mrow_off + (uint32_t)((kbase + 32 * (g >> 2) + 8 * (g & 3) + 4 * hf) * 4));
        }

        f32x16 s[KT];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[kt][i] = 0.f;
        // key tile kt=0 completes first, so its row max can overlap the MFMAs of kt=1
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                const int r = kt * 32 + l32;
                const int c = ks * 2 + hf;
                const V8 a = *reinterpret_cast<const V8*>(Kc + r * D + 8 * (c ^ kswz<D>(r)));
                s[kt] = Elem<T>::mfma32(a, qf[ks], s[kt]);
            }
        }
        // K fragment reads run 4 MFMAs ahead of their use
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < KT * KSTEPS - 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < KT * 4; ++g) {
                const f32x4 m = __builtin_bit_cast(f32x4, mraw[g]);
                s[g >> 2][4 * (g & 3) + 0] += m.x * p.inv_scale;
                s[g >> 2][4 * (g & 3) + 1] += m.y * p.inv_scale;
                s[g >> 2][4 * (g & 3) + 2] += m.z * p.inv_scale;
                s[g >> 2][4 * (g & 3) + 3] += m.w * p.inv_scale;
            }
        }
        if constexpr (kLateLoads) next_tile();
        if (need_mask) {
            // Element i of key tile kt holds key kbase + kt*32 + 8*(i/4) + 4*hf + i%4; it is visible
            // iff its compile-time offset kt*32 + 8*(i/4) + i%4 is <= lim.
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
        const float mcand = fmaxf(mrow, mx * p.c);
        if (__any(mcand - mrow > kRescaleThreshold)) {  // wave-uniform
            const float alpha = fast_exp2(mrow - (mcand == kNegInf ? 0.f : mcand));
            // A lane whose max is still -inf has seen no visible key: its O and l are exactly 0.  When
            // that holds for the whole wave (its first tile) the multiply is skipped.
            if (!__all(mrow == kNegInf)) {
                lrow *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
            }
            mrow = mcand;
        }
        // Wave priority: raised over the exponential/PV block of the non-causal kernel only.  Measured
        // A/B on one MI355X: MMDiT 1x24x4608 +4.5% against raising it over both blocks; the causal
        // kernels ran 1-3% faster with no raise at all.
        if constexpr (!CAUSAL) __builtin_amdgcn_s_setprio(1);
        const float mbase = (mrow == kNegInf) ? 0.f : mrow;
        V8 pb[PVS];
        float ls = lrow;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                V8 pk;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    // fp32 row sum: a sum of the rounded P would cost up to 2^-9 relative in the LSE of
                    // rows with few keys
                    const float pv = fast_exp2(__builtin_fmaf(s[kt][8 * half + e], p.c, -mbase));
                    ls += pv;
                    pk[e] = Elem<T>::from_f32(pv);
                }
                pb[2 * kt + half] = pk;
            }
        }
        lrow = ls;

        // k-step outer: the four MFMAs of step ks need only P chunk ks, so they can run while the
        // exponentials of the later chunks are still being computed
#pragma unroll
        for (int ks = 0; ks < PVS; ++ks) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int d = dt * 32 + tr_d;
                const int k1 = ks * 16 + tr_k4 + tr_key;  // slots 0-3: keys 16ks + 4hf + j
                const int k2 = k1 + 8;                    // slots 4-7: keys 16ks + 8 + 4hf + j
                const V4 lo = __builtin_bit_cast(
                    V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vc + k1 * D + 8 * ((d >> 3) ^ kswz<D>(k1)) + (d & 7))));
                const V4 hi = __builtin_bit_cast(
                    V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(Vc + k2 * D + 8 * ((d >> 3) ^ kswz<D>(k2)) + (d & 7))));
                const V8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                oacc[dt] = Elem<T>::mfma32(a, pb[ks], oacc[dt]);
            }
        }
        // Issue order of this block: the V^T reads of step 0 and P chunk 0, then each PV MFMA
        // followed by two V^T reads and a slice of the next chunk's exponentials.
        __builtin_amdgcn_sched_group_barrier(0x100, 4 * DT, 0);
        __builtin_amdgcn_sched_group_barrier(0x402, 28, 0);
#pragma unroll
        for (int i = 0; i < (PVS - 1) * DT; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x402, 7, 0);
        }
#pragma unroll
        for (int i = 0; i < DT; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (!CAUSAL) __builtin_amdgcn_s_setprio(0);
    };

    if (nt > 0) {
        dma(Ka, kp, krow, p.ks_s, 0, p.qk_ch);
        dma(Va, vp, vrow, p.vs_s, 0, p.v_ch);
    }
    // Q fragments: lane holds query l32, d = ks*16 + hf*8 .. +8.  Issued after tile 0's loads so that
    // the two share one memory latency.  The loads are unconditional, so they issue back to back (a
    // branch per load made the compiler wait for each in turn: 8 round trips, ~3.7 us of a C2
    // workgroup's start).  Rows past Sq read row Sq-1 and chunks past qk_ch read chunk 0; the mask
    // zeroes both.
    {
        const int qrow = wq0 + l32;
        const bool row_ok = qrow < p.Sq;
        const T* qsrc = qp + (int64_t)(row_ok ? qrow : p.Sq - 1) * p.qs_s;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const bool ok = row_ok && (!PAD || 2 * ks + hf < p.qk_ch);
            const u32x4 w = ld16(qsrc + (ok ? ks * 16 + hf * 8 : 0));
            qf[ks] = __builtin_bit_cast(V8, q_bits(w, ok ? p.q_and : 0u, ok ? p.q_xor : 0u));
        }
    }
    // Q fragments (and tile 0) complete here, visibly to the compiler, so that it inserts no load
    // waits inside the loop (where they would also drain the asynchronous tile loads).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    for (int t = 0; t < nt; t += 2) {  // unrolled by two so each tile names its buffers statically
        tile(Ka, Va, Kb, Vb, t);
        if (t + 1 < nt) tile(Kb, Vb, Ka, Va, t + 1);
    }

    // Epilogue: normalise, stage O through LDS (wave w in a 32-row slab of Ka/Kb; 16-byte chunk c of
    // row r at c ^ (r % DCH)) for 16-byte coalesced row stores, and write the LSE.
    __syncthreads();
    T* Os = (wave < 2 ? Ka : Kb) + (wave & 1) * 32 * D;
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
                const int c = dt * 4 + i4;
                *reinterpret_cast<V4*>(Os + row * D + 8 * (c ^ (row % DCH)) + 4 * hf) = o4;
            }
        if (p.lse != nullptr && hf == 0) {
            const int qrow = wq0 + row;
            if (qrow < p.Sq) {
                const float lse = l > 0.f ? (mrow + __log2f(l)) * kLn2 : kNegInf;
                p.lse[b * p.lses_b + hq * p.lses_h + qrow] = lse;
            }
        }
    }
    __syncthreads();
    T* op = reinterpret_cast<T*>(p.o) + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < 32 * DCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / DCH, c = id % DCH;
        const int qrow = wq0 + row;
        // non-temporal: measured +1.3 to 2.5% on short sequences (16x512, 32x256), +0.2 to 0.3% on long ones,
        // against plain stores, with back-to-back launches
        if (qrow < p.Sq && (!PAD || c < p.v_ch))
            __builtin_nontemporal_store(ld16(Os + row * D + 8 * (c ^ (row % DCH))),
                                        reinterpret_cast<u32x4*>(op + (int64_t)qrow * p.os_s + c * 8));
    }
}

// ------------------------------------------------------------------------------------------------

template <typename T, int D, int QT, bool CAUSAL, bool MASKED, bool PAD>
static int launch_prefill(const PrefillParams& prm, hipStream_t stream) {
    constexpr int BM = 4 * QT * 32;
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + BM - 1) / BM;
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_fwd_kernel<T, D, QT, CAUSAL, MASKED, PAD>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    return check_launch("prefill_fwd_kernel");
}

template <typename T, bool MASKED, bool PAD>
static int dispatch_prefill_m(const PrefillParams& p, int D, bool causal, hipStream_t stream) {
    if (D == 128) {
        return causal ? launch_prefill<T, 128, 1, true, MASKED, PAD>(p, stream)
                      : launch_prefill<T, 128, 1, false, MASKED, PAD>(p, stream);
    }
    if (D == 64) {
        return causal ? launch_prefill<T, 64, 1, true, MASKED, PAD>(p, stream)
                      : launch_prefill<T, 64, 1, false, MASKED, PAD>(p, stream);
    }
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill: kernel head dim %d not supported (64, 128, 256 or 512)", D);
}

int prefill_rows64(const PrefillParams& p, bool causal, bool f16, void* ws, size_t ws_bytes, hipStream_t stream);
bool prefill_rows64_fits(const PrefillParams& p);
size_t rows64_sk_workspace(const dtattn_prefill_args* a, int device);

// D is the kernel's head dim (64 or 128); pad: the real head dims are below it.  Head dim 128 without mask or
// padding runs the 64-rows-per-wave kernel (prefill_rows64.hip), which returns the same bits as
// prefill_fwd_kernel at 4-9% (non-causal) and 4-14% (causal) more throughput.
template <typename T>
static int dispatch_prefill(const PrefillParams& p, int D, bool causal, bool pad, void* ws, size_t ws_bytes,
                            hipStream_t stream) {
    if (D == 128 && !pad && p.mask == nullptr && prefill_rows64_fits(p))
        return prefill_rows64(p, causal, __is_same(T, f16_t), ws, ws_bytes, stream);
    if (pad)
        return p.mask != nullptr ? dispatch_prefill_m<T, true, true>(p, D, causal, stream)
                                 : dispatch_prefill_m<T, false, true>(p, D, causal, stream);
    return p.mask != nullptr ? dispatch_prefill_m<T, true, false>(p, D, causal, stream)
                             : dispatch_prefill_m<T, false, false>(p, D, causal, stream);
}

int prefill_fp8(const dtattn_prefill_args* a, float c, int32_t delta, uint32_t q_and, uint32_t q_xor,
                hipStream_t stream);
size_t prefill_fp8_workspace_size(const dtattn_prefill_args* a, int device);
int prefill_f32(const PrefillParams& p, int D, bool causal, bool pad, hipStream_t stream);
int prefill_wide(const PrefillParams& p, int D, bool causal, bool bf16, bool pad, hipStream_t stream);
int wide_key_splits(int64_t B, int64_t Hq, int64_t Sq, int64_t Sk, int D, int cu_count);

// Kernel head dim of a bf16/fp16 call: the smallest of 64, 128, 256, 512 holding both real head dims.
static int kernel_head_dim(int64_t D, int64_t Dv) {
    const int64_t dmax = D > Dv ? D : Dv;
    return dmax <= 64 ? 64 : dmax <= 128 ? 128 : dmax <= 256 ? 256 : dmax <= 512 ? 512 : 0;
}

// Key blocks of a wide-head call on `device` (1: unsplit) and the workspace their partials need:
// O parts [splits][B][Hq][Sq][Dv] in the input dtype, then (256-byte aligned) LSE parts
// [splits][B][Hq][Sq] fp32.
static int wide_plan(const dtattn_prefill_args* a, int device, size_t* bytes, size_t* lse_off) {
    *bytes = 0;
    *lse_off = 0;
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16) return 1;
    if (a->D % 8 != 0 || a->Dv % 8 != 0 || a->B <= 0 || a->Sq <= 0 || a->Sk <= 0) return 1;
    const int Dk = kernel_head_dim(a->D, a->Dv);
    if (Dk < 256) return 1;
    dtattn_device_peaks pk;
    if (dtattn_get_device_peaks(device, &pk) != DTATTN_OK) return 1;
    const int splits = wide_key_splits(a->B, a->Hq, a->Sq, a->Sk, Dk, pk.cu_count);
    if (splits <= 1) return 1;
    const size_t o_bytes = (size_t)splits * a->B * a->Hq * a->Sq * a->Dv * 2;
    *lse_off = (o_bytes + 255) & ~(size_t)255;
    *bytes = *lse_off + (size_t)splits * a->B * a->Hq * a->Sq * sizeof(float);
    return splits;
}

static int stream_device(hipStream_t stream, int* dev) {
    return (stream == nullptr ? hipGetDevice(dev) : hipStreamGetDevice(stream, dev)) == hipSuccess ? DTATTN_OK
                                                                                               : DTATTN_ERR_DEVICE;
}

static bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace dtattn

using namespace dtattn;

extern "C" int dtattn_prefill_fwd(const dtattn_prefill_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill: args is NULL");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (a->B < 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Sq < 0 || a->Sk < 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill: bad sizes B=%lld Hq=%lld Hkv=%lld Sq=%lld Sk=%lld",
                    (long long)a->B, (long long)a->Hq, (long long)a->Hkv, (long long)a->Sq, (long long)a->Sk);
    if (a->Hq % a->Hkv != 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill: Hq=%lld is not a multiple of Hkv=%lld", (long long)a->Hq,
                    (long long)a->Hkv);
    if (a->D <= 0 || a->Dv <= 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill: bad head dims D=%lld Dv=%lld", (long long)a->D,
                    (long long)a->Dv);
    const bool sixteen_bit = a->dtype == DTATTN_BF16 || a->dtype == DTATTN_FP16;
    if (a->D != a->Dv && !sixteen_bit && a->dtype != DTATTN_FP32)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: D=%lld != Dv=%lld is supported for bf16/fp16/fp32 only",
                    (long long)a->D, (long long)a->Dv);
    if (sixteen_bit && (a->D % 8 != 0 || a->Dv % 8 != 0))
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: head dims must be multiples of 8 (D=%lld, Dv=%lld)",
                    (long long)a->D, (long long)a->Dv);
    if (a->dtype == DTATTN_FP32 && (a->D % 4 != 0 || a->Dv % 4 != 0 || a->D > 512 || a->Dv > 512))
        return fail(DTATTN_ERR_UNSUPPORTED,
                    "prefill: fp32 head dims must be multiples of 4 up to 512 (D=%lld, Dv=%lld)", (long long)a->D,
                    (long long)a->Dv);
    // Sequence lengths up to 2^29 keep every causal index expression of the kernels in int32.
    if (a->Sq > (1 << 29) || a->Sk > (1 << 29) || a->B * a->Hq > 0x3fffffff)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: sequence length exceeds 2^29");
    if (a->B == 0 || a->Sq == 0) return DTATTN_OK;
    if (a->q == nullptr || a->o == nullptr || (a->Sk > 0 && (a->k == nullptr || a->v == nullptr)))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill: null tensor pointer");
    const int64_t* strides[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
    const int esz_in = a->dtype == DTATTN_FP8_E4M3FN ? 1 : (a->dtype == DTATTN_FP32 ? 4 : 2);
    const int esz_out = a->o_dtype == DTATTN_FP32 ? 4 : 2;
    for (int i = 0; i < 4; ++i) {
        const int esz = i == 3 ? esz_out : esz_in;
        for (int j = 0; j < 3; ++j)
            if ((strides[i][j] * esz) % 16 != 0)
                return fail(DTATTN_ERR_UNSUPPORTED,
                            "prefill: tensor %d stride[%d]=%lld is not a multiple of 16 bytes", i, j,
                            (long long)strides[i][j]);
    }
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o))
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: tensors must be 16-byte aligned");
    // key/value tiles are addressed with 32-bit byte offsets: 64 rows x row pitch < 2^31
    if (a->k_stride[2] * esz_in * 64 >= (int64_t)1 << 31 || a->v_stride[2] * esz_in * 64 >= (int64_t)1 << 31)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: key/value row pitch exceeds 32 MB");
    ScalePlan sp;
    {
        const uint32_t sign = a->dtype == DTATTN_FP32 ? kSign32 : a->dtype == DTATTN_FP8_E4M3FN ? kSign8 : kSign16;
        const int st = plan_scale(a->scale, a->D, sign, &sp);
        if (st != DTATTN_OK) return st;
    }
    const float scale = sp.scale;
    const float c = scale * kLog2e;
    int64_t delta64 = a->q_offset - a->k_offset;
    const int64_t lim = a->Sq + a->Sk + 1;
    if (delta64 > lim) delta64 = lim;
    if (delta64 < -lim) delta64 = -lim;
    const int32_t delta = (int32_t)delta64;

    if (a->mask != nullptr) {
        if (a->dtype == DTATTN_FP8_E4M3FN)
            return fail(DTATTN_ERR_UNSUPPORTED, "prefill: an attention mask is not supported with fp8 inputs");
        for (int j = 0; j < 3; ++j)
            if (a->mask_stride[j] < 0 || a->mask_stride[j] % 4 != 0)
                return fail(DTATTN_ERR_UNSUPPORTED, "prefill: mask stride[%d]=%lld must be a non-negative multiple of 4",
                            j, (long long)a->mask_stride[j]);
        if ((reinterpret_cast<uintptr_t>(a->mask) & 15u) != 0)
            return fail(DTATTN_ERR_UNSUPPORTED, "prefill: mask must be 16-byte aligned");
        // one (b, h) slab of the mask is addressed with 32-bit byte offsets
        if (((a->Sq - 1) * a->mask_stride[2] + a->Sk + 64) * 4 >= ((int64_t)1 << 32))
            return fail(DTATTN_ERR_UNSUPPORTED, "prefill: mask slab of one (batch, head) exceeds 4 GB");
    }
    if (a->dtype == DTATTN_FP8_E4M3FN) {
        if (a->o_dtype != DTATTN_BF16 && a->o_dtype != DTATTN_FP16)
            return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: output must be bf16 or fp16");
        if (a->q_descale == nullptr || a->k_descale == nullptr || a->v_descale == nullptr)
            return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill fp8: descale pointers are required");
        return prefill_fp8(a, c, delta, sp.q_and, sp.q_xor, stream);
    }
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16 && a->dtype != DTATTN_FP32)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: dtype %d not supported (bf16, fp16, fp32, fp8_e4m3fn)",
                    a->dtype);
    if (a->o_dtype != a->dtype) return fail(DTATTN_ERR_UNSUPPORTED, "prefill: output dtype must equal input dtype");

    PrefillParams p;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->o;
    p.lse = a->lse;
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
    p.mask = a->mask;
    p.ms_b = a->mask_stride[0], p.ms_h = a->mask_stride[1], p.ms_l = a->mask_stride[2];
    p.inv_scale = 1.0f / scale;
    p.nsplit = 1;
    p.kblock = (int32_t)(a->Sk > 0 ? a->Sk : 1);
    p.os_split = 0;
    p.lses_split = 0;
    p.q_and = sp.q_and;
    p.q_xor = sp.q_xor;
    const bool causal = a->causal != 0;
    if (a->dtype == DTATTN_FP32) {
        // kernel head dim 64, 128, 256 or 512 (the last two on the wide fp32 kernel); smaller real dims
        // (multiples of 4, D and Dv independent) are padded
        const int Dk = kernel_head_dim(a->D, a->Dv);
        p.qk_ch = (int32_t)(a->D / 4);
        p.v_ch = (int32_t)(a->Dv / 4);
        return prefill_f32(p, Dk, causal, a->D != Dk || a->Dv != Dk, stream);
    }
    // bf16 / fp16: the kernel head dim is the smallest of 64, 128, 256, 512 that holds both real head
    // dims; smaller real dims (multiples of 8, D and Dv independent) run the padded instantiations.
    const int Dk = kernel_head_dim(a->D, a->Dv);
    if (Dk == 0)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: head dim %lld exceeds 512",
                    (long long)(a->D > a->Dv ? a->D : a->Dv));
    p.qk_ch = (int32_t)(a->D / 8);
    p.v_ch = (int32_t)(a->Dv / 8);
    const bool pad = a->D != Dk || a->Dv != Dk;
    if (Dk >= 256) {
        int splits = 1;
        size_t need = 0, lse_off = 0;
        if (a->workspace != nullptr && a->workspace_bytes > 0 && (reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0) {
            int dev = 0;
            if (stream_device(stream, &dev) != DTATTN_OK) return fail(DTATTN_ERR_DEVICE, "prefill: stream device");
            splits = wide_plan(a, dev, &need, &lse_off);
            if (need > a->workspace_bytes) splits = 1;
        }
        if (splits <= 1) return prefill_wide(p, Dk, causal, a->dtype == DTATTN_BF16, pad, stream);
        // Key blocks in one launch, then their (O, LSE) merged by LSE into the caller's outputs.
        const int64_t tiles = (a->Sk + 31) / 32;
        p.kblock = (int32_t)((tiles + splits - 1) / splits * 32);
        p.nsplit = (int32_t)((a->Sk + p.kblock - 1) / p.kblock);
        char* ws = static_cast<char*>(a->workspace);
        p.o = ws;
        p.os_b = a->Hq * a->Sq * a->Dv, p.os_h = a->Sq * a->Dv, p.os_s = a->Dv;
        p.os_split = a->B * a->Hq * a->Sq * a->Dv;
        p.lse = reinterpret_cast<float*>(ws + lse_off);
        p.lses_b = a->Hq * a->Sq, p.lses_h = a->Sq;
        p.lses_split = a->B * a->Hq * a->Sq;
        const int st = prefill_wide(p, Dk, causal, a->dtype == DTATTN_BF16, pad, stream);
        if (st != DTATTN_OK) return st;
        dtattn_merge_args m;
        memset(&m, 0, sizeof(m));
        m.n_blocks = p.nsplit;
        for (int i = 0; i < p.nsplit; ++i) {
            m.o_blocks[i] = ws + (size_t)i * p.os_split * 2;
            m.lse_blocks[i] = reinterpret_cast<const float*>(ws + lse_off) + (size_t)i * p.lses_split;
        }
        m.B = a->B, m.H = a->Hq, m.S = a->Sq, m.D = a->Dv;
        m.block_o_stride[0] = p.os_b, m.block_o_stride[1] = p.os_h, m.block_o_stride[2] = p.os_s;
        m.block_lse_stride[0] = p.lses_b, m.block_lse_stride[1] = p.lses_h;
        m.block_dtype = a->dtype;
        m.o = a->o;
        m.o_stride[0] = a->o_stride[0], m.o_stride[1] = a->o_stride[1], m.o_stride[2] = a->o_stride[2];
        m.lse = a->lse;
        m.lse_stride[0] = a->lse_stride[0], m.lse_stride[1] = a->lse_stride[1];
        m.o_dtype = a->o_dtype;
        return dtattn_lse_merge(&m, stream);
    }
    if (a->dtype == DTATTN_BF16) return dispatch_prefill<bf16_t>(p, Dk, causal, pad, a->workspace, a->workspace_bytes, stream);
    return dispatch_prefill<f16_t>(p, Dk, causal, pad, a->workspace, a->workspace_bytes, stream);
}

extern "C" size_t dtattn_prefill_workspace_size(const dtattn_prefill_args* a) {
    if (a == nullptr) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (a->dtype == DTATTN_FP8_E4M3FN) return prefill_fp8_workspace_size(a, dev);
    size_t bytes = 0, lse_off = 0;
    wide_plan(a, dev, &bytes, &lse_off);
    const size_t sk = rows64_sk_workspace(a, dev);
    return bytes > sk ? bytes : sk;
}
