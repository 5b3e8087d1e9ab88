// fp32 attention forward for gfx950 on the fp32 matrix cores (v_mfma_f32_32x32x2_f32), with per-row
// LSE.
//
// This is the fp32 branch of SdpaOp::Compute: the libtorch call at
// dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109 computes fp32 inputs in
// fp32, and DTorch's own Llama test (python/dtorch/test/modules/test_llama.py:26-64) runs the model
// in fp32 on the GPU at a 1e-4 tolerance.  Q K^T, the softmax, P and P V therefore all stay in fp32
// here; nothing is rounded to a 16-bit type.
//
// Work decomposition and layout follow the bf16 kernel (prefill_fwd.hip): a workgroup is 4 waves of
// 32 query rows of one (batch, query head); Q fragments stay in registers; S^T = K Q^T and
// O^T = V^T P^T, so each lane owns one query column and the per-query softmax state is a per-lane
// scalar.  What differs:
//   - Key tiles of 32 rows (an fp32 row is twice the bytes): K and V tiles [32][D] fp32,
//     double-buffered, 64 KB per workgroup at D = 128, two workgroups per CU.
//   - The MFMA reduction index is 2 wide.  In S^T step s, lane half h contributes dimension
//     d = (D/2) h + s, so a lane's Q fragment and its K reads are contiguous runs of D/2 floats.
//     Row i of the d-block `blk` of O^T is dimension d = DT i + blk (DT = D / 32), so one LDS read of
//     DT consecutive floats of a V row feeds the DT MFMAs of a PV step.
//   - LDS rows keep 16-byte chunk c at c ^ (r & 15): a 16-lane group of K reads (16 rows, one chunk
//     each) and of V reads (one row, 16 consecutive chunks) touches 16 distinct bank groups.
//
// Pipeline per key tile j (one barrier per tile), as in the bf16 kernel:
//   wait own loads + barrier | K[j+1], V[j+1] -> LDS (async) | S^T = K[j] Q^T | softmax |
//   O^T += V^T(j) P^T(j)
//
// PAD: the real head dims are below the kernel's D (any multiples of 4, Dv may differ from D), as in
// the bf16 kernel: Q/K chunks past p.qk_ch and V chunks past p.v_ch load as zeros (adding nothing to
// the scores, giving O columns that are never stored), and O chunks past p.v_ch are not written.
#include "dtattn_common.hpp"
#include "prefill_params.hpp"

namespace dtattn {

template <int D, bool CAUSAL, bool MASKED, bool PAD>
__global__ void __launch_bounds__(256, 2) prefill_f32_kernel(const PrefillParams p) {
    constexpr int NW = 4;
    constexpr int BN = 32;           // keys per tile
    constexpr int BM = NW * 32;      // query rows per workgroup
    constexpr int DCH = D / 4;       // 16-byte chunks per row
    constexpr int HD = D / 2;        // S^T k-steps: dimensions per lane half
    constexpr int DT = D / 32;       // 32-row d blocks of O^T
    static_assert(D == 64 || D == 128, "head dim 64 or 128");
    typedef float fvec __attribute__((ext_vector_type(DT)));

    __shared__ __attribute__((aligned(16))) float Ka[BN * D];
    __shared__ __attribute__((aligned(16))) float Kb[BN * D];
    __shared__ __attribute__((aligned(16))) float Va[BN * D];
    __shared__ __attribute__((aligned(16))) float Vb[BN * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const BlockCoord bc = block_coord<CAUSAL>(p);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;

    const float* qp = reinterpret_cast<const float*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const float* kp = reinterpret_cast<const float*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const float* vp = reinterpret_cast<const float*>(p.v) + b * p.vs_b + hk * p.vs_h;

    const int q0 = qb * BM;
    const int wq0 = q0 + wave * 32;

    int kend = p.Sk;
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;  // keys < lim can be visible
        kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
    }
    const int nt = (kend + BN - 1) / BN;

    // Q fragment (B operand of S^T = K Q^T), loaded after the first tile's loads are issued
    float qf[HD];

    f32x16 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
    float mrow = kNegInf, lrow = 0.f;

    const int krow = (int)(p.ks_s * (int64_t)sizeof(float));  // row pitch in bytes (host-checked)
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(float));

    // Tile t -> LDS by direct buffer->LDS loads: one wave instruction fills 1 KB (lane l -> byte 16*l),
    // i.e. 1024 / (4 D) rows; lane l loads the global chunk that belongs at its LDS slot,
    // c = slot ^ (row & 15).  The buffer resource covers the tile's valid rows; rows past Sk read zeros,
    // and so do chunks at or past valid_ch (PAD), whose offset lies past the resource.
    auto dma = [&](float* dst, const float* base, int pitch, int64_t stride, int t, int valid_ch) {
        constexpr int ROWS_PER_INSTR = 1024 / (4 * D);
        constexpr int INSTR = BN / ROWS_PER_INSTR / NW;  // per wave
        const int rows = min(BN, p.Sk - t * BN);
        // the resource ends where the tile's last valid row ends (its real width under PAD)
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + (PAD ? valid_ch * 16 : D * 4));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int r0 = (wave * INSTR + i) * ROWS_PER_INSTR;
            const int r = r0 + lane / DCH;
            const int c = (lane % DCH) ^ (r & 15);
            // 2^31 lies past every tile's resource (the host keeps 64 row pitches below 2^31)
            const uint32_t off = (PAD && c >= valid_ch) ? 0x80000000u : (uint32_t)(r * pitch + c * 16);
            buf_ld16_lds_async(rs, dst + r0 * D, off);
        }
    };

    // MASKED: lane (l32, hf) reads, for query row wq0 + l32, keys kbase + 8g + 4hf .. +3 (g < 4) of
    // the (b, hq) mask slab, behind a buffer resource (reads past its last row return 0; those keys
    // are hidden by the ragged-tail mask anyway).
    const float* mbase_p = MASKED ? p.mask + b * p.ms_b + hq * p.ms_h : nullptr;
    const auto mrs = make_rsrc(mbase_p, MASKED ? (uint32_t)((((int64_t)(p.Sq - 1) * p.ms_l + p.Sk) * 4)) : 0u);
    const uint32_t mrow_off = MASKED ? (uint32_t)((int64_t)min(wq0 + l32, p.Sq - 1) * p.ms_l * 4) : 0u;

    auto tile = [&](const float* Kc, const float* Vc, float* Kn, float* Vn, int t) {
        wait_vmem();
        lds_barrier();  // tile t landed everywhere; every wave finished tile t-1 (so Kn/Vn are free)
        auto next_tile = [&]() {
            if (t + 1 < nt) {
                dma(Kn, kp, krow, p.ks_s, t + 1, p.qk_ch);
                dma(Vn, vp, vrow, p.vs_s, t + 1, p.v_ch);
            }
        };
        if constexpr (!MASKED) next_tile();
        const int kbase = t * BN;
        if (CAUSAL && kbase > wq0 + 31 + p.delta) {  // every row of this wave precedes the tile
            if constexpr (MASKED) next_tile();
            return;
        }
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > wq0 + p.delta));
        u32x4 mraw[4];
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < 4; ++g) mraw[g] = buf_ld16(mrs, mrow_off + (uint32_t)((kbase + 8 * g + 4 * hf) * 4));
        }

        // S^T = K Q^T: lane (l32, hf) supplies K[kbase + l32][HD*hf + s] at step s.
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.f;
        {
            const int r = l32;
#pragma unroll
            for (int g = 0; g < HD / 4; ++g) {
                const int c = (HD / 4) * hf + g;
                const f32x4 kv = *reinterpret_cast<const f32x4*>(Kc + r * D + 4 * (c ^ (r & 15)));
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * g + 0], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * g + 1], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * g + 2], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * g + 3], s, 0, 0, 0);
            }
            // K reads run two groups of four MFMAs ahead of their use (hoisting them all would cost
            // 4 D registers)
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int g = 0; g < HD / 4 - 2; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
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
            next_tile();
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
        if (__any(mcand - mrow > kRescaleThreshold)) {  // wave-uniform
            const float alpha = fast_exp2(mrow - (mcand == kNegInf ? 0.f : mcand));
            mrow = mcand;
            lrow *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
        }
        const float mbase = (mrow == kNegInf) ? 0.f : mrow;
        float pr[16];
        float ls = lrow;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pr[i] = fast_exp2(__builtin_fmaf(s[i], p.c, -mbase));
            ls += pr[i];
        }
        lrow = ls;

        // O^T += V^T P^T over 16 steps: step (jj, rr) pairs key 8jj + rr (lane half 0) with key
        // 8jj + 4 + rr (half 1), the keys of the lane's own score element 4jj + rr.
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int key = 8 * jj + 4 * hf + rr;
                const int e = DT * l32;  // first of the DT consecutive floats this lane reads
                const fvec vv = *reinterpret_cast<const fvec*>(Vc + key * D + 4 * ((e >> 2) ^ (key & 15)) + (e & 3));
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[dt], pr[4 * jj + rr], oacc[dt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < 14; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, DT, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * DT, 0);
    };

    if (nt > 0) {
        dma(Ka, kp, krow, p.ks_s, 0, p.qk_ch);
        dma(Va, vp, vrow, p.vs_s, 0, p.v_ch);
    }
    // Lane (l32, hf) holds Q[wq0 + l32][HD*hf + s], s < HD.  Unconditional loads issue back to back and
    // share the first tile's memory latency (a branch per load serialised them); rows past Sq read row
    // Sq-1 and are zeroed by the mask; so are chunks at or past qk_ch (PAD), which read chunk 0.
    {
        const int qrow = wq0 + l32;
        const bool row_ok = qrow < p.Sq;
        const float* qsrc = qp + (int64_t)(row_ok ? qrow : p.Sq - 1) * p.qs_s;
#pragma unroll
        for (int g = 0; g < HD / 4; ++g) {
            const int ch = (HD / 4) * hf + g;  // 16-byte chunk of the row
            const bool ok = row_ok && (!PAD || ch < p.qk_ch);
            const float* src = (!PAD || ch < p.qk_ch) ? qsrc + 4 * ch : qsrc;
            const u32x4 raw = q_bits(ld16(src), ok ? p.q_and : 0u, ok ? p.q_xor : 0u);
            const f32x4 x = __builtin_bit_cast(f32x4, raw);
            qf[4 * g + 0] = x.x, qf[4 * g + 1] = x.y, qf[4 * g + 2] = x.z, qf[4 * g + 3] = x.w;
        }
    }
    // Q fragments (and tile 0) complete here, visibly to the compiler, so that it inserts no load
    // waits inside the loop (where they would also drain the asynchronous tile loads).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    for (int t = 0; t < nt; t += 2) {  // unrolled by two so each tile names its buffers statically
        tile(Ka, Va, Kb, Vb, t);
        if (t + 1 < nt) tile(Kb, Vb, Ka, Va, t + 1);
    }

    // Epilogue: element i of O^T block dt is O[wq0 + l32][DT * (8*(i/4) + 4*hf + i%4) + dt], so the
    // DT blocks of one element index form DT consecutive floats of the output row.
    const float l = sum_xor32(lrow);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int qrow = wq0 + l32;
    if (qrow < p.Sq) {
        float* orow = reinterpret_cast<float*>(p.o) + b * p.os_b + hq * p.os_h + (int64_t)qrow * p.os_s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            fvec o;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] = oacc[dt][i] * inv;
            const int col = DT * (8 * (i >> 2) + 4 * hf + (i & 3));  // DT <= 4 floats within one 16-byte chunk
            if (!PAD || col < 4 * p.v_ch) *reinterpret_cast<fvec*>(orow + col) = o;
        }
        if (p.lse != nullptr && hf == 0)
            p.lse[b * p.lses_b + hq * p.lses_h + qrow] = l > 0.f ? (mrow + __log2f(l)) * kLn2 : kNegInf;
    }
}

template <int D, bool CAUSAL, bool MASKED, bool PAD>
static int launch_prefill_f32(const PrefillParams& prm, hipStream_t stream) {
    constexpr int BM = 4 * 32;
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + BM - 1) / BM;
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_f32_kernel<D, CAUSAL, MASKED, PAD>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    return check_launch("prefill_f32_kernel");
}

// ------------------------------------------------------------------------------------------------
// fp32 at kernel head dims 256 and 512 (the diffusers VAE attention, one head of 512, run in fp32).
//
// Q fragments of D/2 floats per lane and O^T accumulators of D/2 registers no longer fit one wave, so
// the head dims are split across the workgroup instead: a workgroup is 4 waves over the same 32 query
// rows, and wave w owns dims [w D/4, (w+1) D/4) of both Q K^T and O.  Per 32-key tile:
//   1. wave w computes its partial S^T over its dims (D/8 MFMA steps, lane half h contributing dims
//      w D/4 + (D/8) h + s) and writes it to its slab of an LDS exchange;
//   2. barrier; K(t+1) starts loading into the K buffer, which every wave has finished reading;
//   3. every wave adds the four partials in wave order (the same fp32 additions in every wave, so all
//      four hold bit-identical scores), applies the mask and runs the same softmax;
//   4. wait for V(t) (issued one tile earlier) + barrier, then O^T += V^T P^T for the wave's dims;
//   5. barrier; V(t+1) starts loading into the V buffer.
// K and V tiles are single-buffered ([32][D] fp32 each, 64 KB at D = 512) and the two loads of a tile
// overlap the other half of the previous tile's work: 144 KB of LDS with the 16 KB exchange at D = 512.
// Row i of the d-block dt of a wave's O^T is dimension w D/4 + DQ i + dt (DQ = D/128 blocks), so one
// LDS read of DQ consecutive floats of a V row feeds the DQ MFMAs of a PV step, as in the kernel above.
template <int N>
__device__ __forceinline__ void wait_vm_n() {
    static_assert(N == 0 || N == 8 || N == 16, "vmcnt immediates used by the wide fp32 kernel");
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    if constexpr (N == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

template <int D, bool CAUSAL, bool MASKED, bool PAD>
__global__ void __launch_bounds__(256, 1) prefill_f32_wide_kernel(const PrefillParams p) {
    constexpr int NW = 4;
    constexpr int BN = 32;           // keys per tile
    constexpr int BM = 32;           // query rows per workgroup (shared by the 4 waves)
    constexpr int DCH = D / 4;       // 16-byte chunks per row
    constexpr int HQ = D / 8;        // S^T k-steps per wave: dimensions per lane half of the wave's quarter
    constexpr int DQ = D / 128;      // 32-row d blocks of the wave's O^T
    constexpr int INSTR = BN * D * 4 / 1024 / NW;  // 1 KB tile-load instructions per wave per tile
    static_assert(D == 256 || D == 512, "head dim 256 or 512");
    typedef float fvec __attribute__((ext_vector_type(DQ)));

    __shared__ __attribute__((aligned(16))) float Kt[BN * D];
    __shared__ __attribute__((aligned(16))) float Vt[BN * D];
    __shared__ __attribute__((aligned(16))) float X[NW * 64 * 16];  // partial S^T of each wave

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const BlockCoord bc = block_coord<CAUSAL>(p);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;
    const float* qp = reinterpret_cast<const float*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const float* kp = reinterpret_cast<const float*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const float* vp = reinterpret_cast<const float*>(p.v) + b * p.vs_b + hk * p.vs_h;

    const int q0 = qb * BM;
    int kend = p.Sk;
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;
        kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
    }
    const int nt = (kend + BN - 1) / BN;
    const int qoff = wave * (D / 4);  // first dim of the wave's quarter

    float qf[HQ];
    f32x16 oacc[DQ];
#pragma unroll
    for (int dt = 0; dt < DQ; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
    float mrow = kNegInf, lrow = 0.f;

    const int krow = (int)(p.ks_s * (int64_t)sizeof(float));
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(float));
    // Tile t -> LDS as in the kernel above: lane l of instruction i fills 16-byte slot l of 1 KB, the
    // global chunk c = slot ^ (row & 15) of its row; rows past Sk and (PAD) chunks past valid_ch read 0.
    auto dma = [&](float* dst, const float* base, int pitch, int64_t stride, int t, int valid_ch) {
        constexpr int ROWS_PER_INSTR = 1024 / (4 * D);
        const int rows = min(BN, p.Sk - t * BN);
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + (PAD ? valid_ch * 16 : D * 4));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
        constexpr int LANES_PER_ROW = DCH > 64 ? 64 : DCH;
        constexpr int INSTR_PER_ROW = DCH / LANES_PER_ROW;  // 1 KB holds 1/INSTR_PER_ROW of a row
        static_assert(ROWS_PER_INSTR == 0 || INSTR_PER_ROW == 1, "");
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int ins = wave * INSTR + i;         // 1 KB piece of the tile
            const int r = ins / INSTR_PER_ROW;        // its row
            const int c = (ins % INSTR_PER_ROW) * 64 + lane;  // its chunk, unswizzled slot
            const int cg = c ^ (r & 15);              // global chunk held at slot c
            const uint32_t off = (PAD && cg >= valid_ch) ? 0x80000000u : (uint32_t)(r * pitch + cg * 16);
            buf_ld16_lds_async(rs, dst + ins * 256, off);
        }
    };
    static_assert(DCH >= 64, "one 1 KB load instruction covers at most one row");

    const float* mbase_p = MASKED ? p.mask + b * p.ms_b + hq * p.ms_h : nullptr;
    const auto mrs = make_rsrc(mbase_p, MASKED ? (uint32_t)((((int64_t)(p.Sq - 1) * p.ms_l + p.Sk) * 4)) : 0u);
    const uint32_t mrow_off = MASKED ? (uint32_t)((int64_t)min(q0 + l32, p.Sq - 1) * p.ms_l * 4) : 0u;

    // Exchange slab: lane l's 16 floats as four 16-byte chunks, chunk j at j ^ ((l >> 2) & 3), so the 16
    // lanes of one access pass hit 16 distinct bank groups.
    auto xoff = [&](int w, int j) { return (w * 64 + lane) * 16 + 4 * (j ^ ((lane >> 2) & 3)); };

    if (nt > 0) {
        dma(Kt, kp, krow, p.ks_s, 0, p.qk_ch);
        dma(Vt, vp, vrow, p.vs_s, 0, p.v_ch);
    }
    // Lane (l32, hf) holds Q[q0 + l32][qoff + HQ hf + s], s < HQ; rows past Sq read row Sq-1 and padded
    // chunks read chunk 0, both zeroed by the mask of the scale plan.
    {
        const int qrow = q0 + l32;
        const bool row_ok = qrow < p.Sq;
        const float* qsrc = qp + (int64_t)(row_ok ? qrow : p.Sq - 1) * p.qs_s;
#pragma unroll
        for (int g = 0; g < HQ / 4; ++g) {
            const int ch = (qoff + HQ * hf) / 4 + g;
            const bool ok = row_ok && (!PAD || ch < p.qk_ch);
            const float* src = (!PAD || ch < p.qk_ch) ? qsrc + 4 * ch : qsrc;
            const u32x4 raw = q_bits(ld16(src), ok ? p.q_and : 0u, ok ? p.q_xor : 0u);
            const f32x4 x = __builtin_bit_cast(f32x4, raw);
            qf[4 * g + 0] = x.x, qf[4 * g + 1] = x.y, qf[4 * g + 2] = x.z, qf[4 * g + 3] = x.w;
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): Q, K(0) and V(0)
    lds_barrier();

    for (int t = 0; t < nt; ++t) {
        const int kbase = t * BN;
        const bool more = t + 1 < nt;
        u32x4 mraw[4];
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < 4; ++g) mraw[g] = buf_ld16(mrs, mrow_off + (uint32_t)((kbase + 8 * g + 4 * hf) * 4));
        }
        // 1. partial S^T over the wave's dims
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.f;
        {
            const int r = l32;
#pragma unroll
            for (int g = 0; g < HQ / 4; ++g) {
                const int c = (qoff + HQ * hf) / 4 + g;
                const f32x4 kv = *reinterpret_cast<const f32x4*>(Kt + r * D + 4 * (c ^ (r & 15)));
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * g + 0], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * g + 1], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * g + 2], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * g + 3], s, 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int g = 0; g < HQ / 4 - 2; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<f32x4*>(X + xoff(wave, j)) = f32x4{s[4 * j], s[4 * j + 1], s[4 * j + 2], s[4 * j + 3]};
        // 2. every partial written, every K(t) read done: K(t+1) may land
        lds_barrier();
        if (more) dma(Kt, kp, krow, p.ks_s, t + 1, p.qk_ch);
        // 3. scores in wave order, mask, softmax
        f32x16 sum;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 a = *reinterpret_cast<const f32x4*>(X + xoff(0, j));
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                const f32x4 bq = *reinterpret_cast<const f32x4*>(X + xoff(w, j));
                a = f32x4{a.x + bq.x, a.y + bq.y, a.z + bq.z, a.w + bq.w};
            }
            sum[4 * j] = a.x, sum[4 * j + 1] = a.y, sum[4 * j + 2] = a.z, sum[4 * j + 3] = a.w;
        }
        if constexpr (MASKED) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 m = __builtin_bit_cast(f32x4, mraw[g]);
                sum[4 * g + 0] += m.x * p.inv_scale;
                sum[4 * g + 1] += m.y * p.inv_scale;
                sum[4 * g + 2] += m.z * p.inv_scale;
                sum[4 * g + 3] += m.w * p.inv_scale;
            }
        }
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > q0 + p.delta));
        if (need_mask) {
            int lim = p.Sk - 1 - kbase;
            if (CAUSAL) lim = min(lim, q0 + l32 + p.delta - kbase);
            lim -= 4 * hf;
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (8 * (i >> 2) + (i & 3) > lim) sum[i] = kNegInf;
        }
        float mx = kNegInf;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sum[i]);
        mx = max_xor32(mx);
        const float mcand = fmaxf(mrow, mx * p.c);
        if (__any(mcand - mrow > kRescaleThreshold)) {  // wave-uniform (and the same in every wave)
            const float alpha = fast_exp2(mrow - (mcand == kNegInf ? 0.f : mcand));
            if (!__all(mrow == kNegInf)) {
                lrow *= alpha;
#pragma unroll
                for (int dt = 0; dt < DQ; ++dt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
            }
            mrow = mcand;
        }
        const float mbase = (mrow == kNegInf) ? 0.f : mrow;
        float pr[16];
        float ls = lrow;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pr[i] = fast_exp2(__builtin_fmaf(sum[i], p.c, -mbase));
            ls += pr[i];
        }
        lrow = ls;
        // 4. V(t) landed everywhere (the K(t+1) loads issued after it may stay in flight)
        if (more)
            wait_vm_n<INSTR>();
        else
            wait_vm_n<0>();
        lds_barrier();
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int key = 8 * jj + 4 * hf + rr;
                const int e = qoff + DQ * l32;
                const fvec vv = *reinterpret_cast<const fvec*>(Vt + key * D + 4 * ((e >> 2) ^ (key & 15)) + (e & 3));
#pragma unroll
                for (int dt = 0; dt < DQ; ++dt)
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[dt], pr[4 * jj + rr], oacc[dt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < 14; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, DQ, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * DQ, 0);
        // 5. every V(t) read done: V(t+1) may land; then K(t+1) (issued before it) must have landed
        lds_barrier();
        if (more) {
            dma(Vt, vp, vrow, p.vs_s, t + 1, p.v_ch);
            wait_vm_n<INSTR>();
            lds_barrier();
        }
    }

    // Epilogue: element i of the wave's O^T block dt is O[q0 + l32][qoff + DQ (8 (i/4) + 4 hf + i%4) + dt].
    const float l = sum_xor32(lrow);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int qrow = q0 + l32;
    if (qrow < p.Sq) {
        float* orow = reinterpret_cast<float*>(p.o) + b * p.os_b + hq * p.os_h + (int64_t)qrow * p.os_s;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            fvec o;
#pragma unroll
            for (int dt = 0; dt < DQ; ++dt) o[dt] = oacc[dt][i] * inv;
            const int col = qoff + DQ * (8 * (i >> 2) + 4 * hf + (i & 3));  // DQ <= 4 floats of one chunk
            if (!PAD || col < 4 * p.v_ch) *reinterpret_cast<fvec*>(orow + col) = o;
        }
        if (p.lse != nullptr && hf == 0 && wave == 0)
            p.lse[b * p.lses_b + hq * p.lses_h + qrow] = l > 0.f ? (mrow + __log2f(l)) * kLn2 : kNegInf;
    }
}

template <int D, bool CAUSAL, bool MASKED, bool PAD>
static int launch_prefill_f32_wide(const PrefillParams& prm, hipStream_t stream) {
    constexpr int BM = 32;
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + BM - 1) / BM;
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_f32_wide_kernel<D, CAUSAL, MASKED, PAD>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    return check_launch("prefill_f32_wide_kernel");
}

template <bool MASKED, bool PAD>
static int dispatch_prefill_f32_m(const PrefillParams& p, int D, bool causal, hipStream_t stream) {
    if (D == 128)
        return causal ? launch_prefill_f32<128, true, MASKED, PAD>(p, stream)
                      : launch_prefill_f32<128, false, MASKED, PAD>(p, stream);
    if (D == 64)
        return causal ? launch_prefill_f32<64, true, MASKED, PAD>(p, stream)
                      : launch_prefill_f32<64, false, MASKED, PAD>(p, stream);
    if (D == 256)
        return causal ? launch_prefill_f32_wide<256, true, MASKED, PAD>(p, stream)
                      : launch_prefill_f32_wide<256, false, MASKED, PAD>(p, stream);
    if (D == 512)
        return causal ? launch_prefill_f32_wide<512, true, MASKED, PAD>(p, stream)
                      : launch_prefill_f32_wide<512, false, MASKED, PAD>(p, stream);
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill: fp32 kernel head dim %d not supported (64, 128, 256 or 512)", D);
}

// Entry from dtattn_prefill_fwd once the arguments are validated and `p` is filled.  D is the kernel's
// head dim (64, 128, 256 or 512); pad: the real head dims (p.qk_ch, p.v_ch chunks of 4 floats) are below it.
int prefill_f32(const PrefillParams& p, int D, bool causal, bool pad, hipStream_t stream) {
    if (pad)
        return p.mask != nullptr ? dispatch_prefill_f32_m<true, true>(p, D, causal, stream)
                                 : dispatch_prefill_f32_m<false, true>(p, D, causal, stream);
    return p.mask != nullptr ? dispatch_prefill_f32_m<true, false>(p, D, causal, stream)
                             : dispatch_prefill_f32_m<false, false>(p, D, causal, stream);
}

}  // namespace dtattn
