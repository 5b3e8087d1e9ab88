// Flash-style attention forward with 64 query rows per wave (bf16 / fp16, head dim 128, no mask, no padding).
//
// Replaces the arithmetic of SdpaOp::Compute (the libtorch call at
// dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109) on the GPU, for the calls
// prefill_fwd_kernel would otherwise take at head dim 128 without mask or padding.
//
// Why a second kernel.  prefill_fwd_kernel runs two waves of 32 query rows per SIMD; per 64-key tile a wave
// reads 32 KB of K and V^T fragments from LDS for 32 MFMAs, and the softmax of one wave only partly overlaps
// the MFMAs of the other.  Here a wave owns 64 rows (blocks A and B), so every K and V^T fragment feeds two
// MFMAs, and one wave per SIMD overlaps its own softmax with its MFMAs by software pipelining:
//   phase A of tile t: S(t+1) = K(t+1) Q^T   ||  P(t) chunks 0-1, the next tiles' loads
//   phase B of tile t: O += V(t)^T P(t)      ||  P(t) chunks 2-3, the row max of S(t+1)
// That register plan (O and Q in 192 accumulation registers, two score tiles, P and fragment temporaries in
// 200 vector registers) does not survive the compiler's allocator, so the tile loop is one inline-asm
// program written out by gen_prefill_rows64.py (the build runs it).  Its arithmetic is that of
// prefill_fwd_kernel step for step, with the same lazy rescale per 32-row block: the two kernels return
// identical bits.
//
// Workgroups: grouped-query calls (groups of 4k heads, positive scale) run prefill_rows64_gqa_kernel, whose
// 4 waves are 4 query heads over the same 64 rows, persistent over its work items.  Other calls run
// prefill_rows64_kernel: NW waves x 64 consecutive rows of one (batch, query head), NW = 2 for causal calls
// (two workgroups per CU), 4 otherwise.  K and V tiles of 64 keys are double-buffered in LDS and filled by
// direct buffer->LDS loads spread over phase A; the epilogue is prefill_fwd_kernel's.
#include "dtattn_common.hpp"
#include "prefill_params.hpp"
#include "prefill_rows64_asm.inc"

namespace dtattn {

namespace {

typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int kswz128(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

template <int NW>
struct DmaOffsets;
template <>
struct DmaOffsets<4> {
    typedef u32x8 type;
};
template <>
struct DmaOffsets<2> {
    typedef u32x16 type;
};

}  // namespace

template <typename T, bool CAUSAL, int NW>
__global__ void __launch_bounds__(64 * NW, 1) prefill_rows64_kernel(const PrefillParams p) {
    typedef typename Elem<T>::vec4 V4;
    constexpr int D = 128, BN = 64, BM = NW * 64, DCH = 16, INSTR = 16 / NW;
    // K0, K1, V0, V1: [64 keys][128] each, 16-byte chunk c of row r at c ^ kswz128(r)
    __shared__ __attribute__((aligned(16))) T smem[4 * BN * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const BlockCoord bc = block_coord<CAUSAL>(p);
    const int b = bc.b, hq = bc.hq, hk = bc.hk;
    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const T* kp = reinterpret_cast<const T*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const T* vp = reinterpret_cast<const T*>(p.v) + b * p.vs_b + hk * p.vs_h;

    const int q0 = bc.qb * BM;
    const int wq0 = q0 + wave * 64;
    int kend = p.Sk;
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;  // keys < lim can be visible to the workgroup
        kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
    }
    const int nt = (kend + BN - 1) / BN;
    int tw = nt;  // tiles this wave computes; the others it only loads and waits through
    if (CAUSAL) {
        const int last = wq0 + 63 + p.delta;
        tw = last < 0 ? 0 : min(nt, last / BN + 1);
    }
    tw = __builtin_amdgcn_readfirstlane(tw);

    const int krow = (int)(p.ks_s * (int64_t)sizeof(T));  // row pitches in bytes
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(T));
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;

    // This wave's share of a tile load: INSTR 1 KB instructions per tensor, lane l -> LDS byte 16 l of
    // rows 4i .. 4i+3 of the wave's slice; the global chunk is the one that belongs at that LDS slot.
    typename DmaOffsets<NW>::type doff;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
        const int r = (wave * INSTR + i) * 4 + lane / DCH;
        const int cc = (lane % DCH) ^ kswz128(r);
        doff[i] = (uint32_t)(r * krow + cc * 16);
        doff[INSTR + i] = (uint32_t)(r * vrow + cc * 16);
    }
    auto dma = [&](int buf, const T* base, int pitch, int64_t stride, int t, int first) {
        const int rows = min(BN, p.Sk - t * BN);
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + D * (int)sizeof(T));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
        T* dst = smem + buf * BN * D;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) buf_ld16_lds_async(rs, dst + (wave * INSTR + i) * 4 * D, doff[first + i]);
    };

    // LDS addresses of the fragment reads: K row l32 chunk (2 ks + hf) per k-step; the V^T reads of
    // ds_read_b64_tr_b16 (in each 16-lane block lane 4j+a addresses key j, d-segment 4a) per 32-d tile
    u32x16 addr;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) addr[ks] = sbase + (uint32_t)(l32 * D + 8 * ((2 * ks + hf) ^ kswz128(l32))) * 2u;
    {
        const int blk = lane >> 4, bl = lane & 15;
        const int tr_key = bl >> 2, tr_d = 16 * (blk & 1) + 4 * (bl & 3), tr_k4 = 4 * (blk >> 1);
        const int k1 = tr_k4 + tr_key, k2 = k1 + 8;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int d = dt * 32 + tr_d;
            addr[8 + dt] = sbase + (uint32_t)(k1 * D + 8 * ((d >> 3) ^ kswz128(k1)) + (d & 7)) * 2u;
            addr[12 + dt] = sbase + (uint32_t)(k2 * D + 8 * ((d >> 3) ^ kswz128(k2)) + (d & 7)) * 2u;
        }
    }
    // Mask limits of blocks A and B (lane's row, keys of its half): key offset o of tile j is hidden when
    // o > lim - 64 j.
    u32x2 lim;
#pragma unroll
    for (int X = 0; X < 2; ++X) {
        int v = p.Sk - 1;
        if (CAUSAL) v = min(v, wq0 + 32 * X + l32 + p.delta);
        lim[X] = (uint32_t)(v - 4 * hf);
    }

    if (nt > 0) {
        dma(0, kp, krow, p.ks_s, 0, 0);
        dma(2, vp, vrow, p.vs_s, 0, INSTR);
        if (nt > 1) dma(1, kp, krow, p.ks_s, 1, 0);
    }
    // Q of blocks A and B: lane holds row l32 (+32), d = ks*16 + hf*8 .. +8 per k-step.  Unconditional loads:
    // rows past Sq read row Sq-1 and the scale plan's mask zeroes them.
    u32x32 QA, QB;
#pragma unroll
    for (int X = 0; X < 2; ++X) {
        const int qrow = wq0 + 32 * X + l32;
        const bool ok = qrow < p.Sq;
        const T* qsrc = qp + (int64_t)(ok ? qrow : p.Sq - 1) * p.qs_s;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const u32x4 q = q_bits(ld16(qsrc + ks * 16 + hf * 8), ok ? p.q_and : 0u, ok ? p.q_xor : 0u);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (X == 0)
                    QA[4 * ks + j] = q[j];
                else
                    QB[4 * ks + j] = q[j];
            }
        }
    }
    f32x32 OA01, OA23, OB01, OB23;
#pragma unroll
    for (int i = 0; i < 32; ++i) OA01[i] = 0.f, OA23[i] = 0.f, OB01[i] = 0.f, OB23[i] = 0.f;
    float mA = kNegInf, mB = kNegInf, lA = 0.f, lB = 0.f;
    const float c = p.c;
    const int kd = wq0 + p.delta;
    const uint64_t kb64 = (uint64_t)(uintptr_t)kp, vb64 = (uint64_t)(uintptr_t)vp;
    const uint32_t klo = (uint32_t)kb64, khi = (uint32_t)(kb64 >> 32);
    const uint32_t vlo = (uint32_t)vb64, vhi = (uint32_t)(vb64 >> 32);
    const uint32_t m0base = __builtin_amdgcn_readfirstlane(sbase + (uint32_t)(wave * INSTR * 1024));

    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): Q and the first tiles
    lds_barrier();
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is named as clobbered: the program sets it for its loads
    if (nt > 0) {
#define DTATTN_ROWS64_OPERANDS                                                                                 \
    : "+{a[0:31]}"(OA01), "+{a[32:63]}"(OA23), "+{a[64:95]}"(OB01), "+{a[96:127]}"(OB23), [mA] "+v"(mA),       \
      [mB] "+v"(mB), [lA] "+v"(lA), [lB] "+v"(lB)                                                                \
    : "{a[128:159]}"(QA), "{a[160:191]}"(QB), "{v[200:215]}"(addr), [nt] "s"(nt), [tw] "s"(tw), [c] "s"(c),    \
      [sk] "s"(p.Sk), [kd] "s"(kd), [kp] "s"(krow), [vp] "s"(vrow), [klo] "s"(klo), [khi] "s"(khi),            \
      [vlo] "s"(vlo), [vhi] "s"(vhi), [m0base] "s"(m0base)
#define DTATTN_ROWS64_RUN(PROG)                                                                                \
    if constexpr (NW == 4)                                                                                     \
        asm volatile(PROG DTATTN_ROWS64_OPERANDS, "{v[216:223]}"(doff), "{v[224:225]}"(lim)                    \
                     : DTATTN_ROWS64_CLOBBERS);                                                                \
    else                                                                                                       \
        asm volatile(PROG DTATTN_ROWS64_OPERANDS, "{v[216:231]}"(doff), "{v[232:233]}"(lim)                    \
                     : DTATTN_ROWS64_CLOBBERS);
        constexpr bool F16 = __is_same(T, f16_t);
        if constexpr (F16 && CAUSAL && NW == 2) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_F16_2_1) }
        else if constexpr (F16 && CAUSAL) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_F16_4_1) }
        else if constexpr (F16 && NW == 2) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_F16_2_0) }
        else if constexpr (F16) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_F16_4_0) }
        else if constexpr (CAUSAL && NW == 2) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_BF16_2_1) }
        else if constexpr (CAUSAL) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_BF16_4_1) }
        else if constexpr (NW == 2) { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_BF16_2_0) }
        else { DTATTN_ROWS64_RUN(DTATTN_ROWS64_PROGRAM_BF16_4_0) }
#undef DTATTN_ROWS64_RUN
#undef DTATTN_ROWS64_OPERANDS
    }
#pragma clang diagnostic pop

    // Epilogue: normalise, stage O through LDS (wave w in rows [64w, 64w + 64); 16-byte chunk c of row r at
    // c ^ (r % 16)) for 16-byte coalesced row stores, and write the LSE.
    __syncthreads();
    T* Os = smem + wave * 64 * D;
#pragma unroll
    for (int X = 0; X < 2; ++X) {
        const float l = sum_xor32(X == 0 ? lA : lB);
        const float m = X == 0 ? mA : mB;
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int row = 32 * X + l32;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                V4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 16 * (dt & 1) + 4 * i4 + e;
                    const float ov = X == 0 ? (dt < 2 ? OA01[k] : OA23[k]) : (dt < 2 ? OB01[k] : OB23[k]);
                    o4[e] = Elem<T>::from_f32(ov * inv);
                }
                const int cc = dt * 4 + i4;
                *reinterpret_cast<V4*>(Os + row * D + 8 * (cc ^ (row % DCH)) + 4 * hf) = o4;
            }
        if (p.lse != nullptr && hf == 0) {
            const int qrow = wq0 + row;
            if (qrow < p.Sq) p.lse[b * p.lses_b + hq * p.lses_h + qrow] = l > 0.f ? (m + __log2f(l)) * kLn2 : kNegInf;
        }
    }
    __syncthreads();
    T* op = reinterpret_cast<T*>(p.o) + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < 64 * DCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / DCH, cc = id % DCH;
        const int qrow = wq0 + row;
        if (qrow < p.Sq)
            __builtin_nontemporal_store(ld16(Os + row * D + 8 * (cc ^ (row % DCH))),
                                        reinterpret_cast<u32x4*>(op + (int64_t)qrow * p.os_s + cc * 8));
    }
}

// Grouped-query form, persistent.  A workgroup's 4 waves are 4 query heads of one kv head over the same 64
// rows, so they share every K/V tile and all see the same causal tile count (no wave idles through the
// others' diagonal tiles).  One workgroup per CU loops over work items (64 rows x 4 heads) in a snake order
// within its XCD, so consecutive items balance in length; the next item's Q and first K/V tiles load while
// the current item's epilogue runs, with O staged through its own 64 KB of LDS.  Q goes straight into its
// accumulation registers (rows past Sq load row Sq-1; their outputs are not stored), so the scale plan must
// be the identity (a positive scale).
__device__ __forceinline__ int gqa_item(int w, int k, int G, int xcd_map) {
    if (xcd_map) {  // items x + 8 j run on XCD x; workgroup w is on XCD w % 8
        const int x = w & 7, u = w >> 3, gx = G >> 3;
        return x + 8 * ((k & 1) ? (k + 1) * gx - 1 - u : k * gx + u);
    }
    return (k & 1) ? (k + 1) * G - 1 - w : k * G + w;
}

template <typename T, bool CAUSAL>
__global__ void __launch_bounds__(256, 1) prefill_rows64_gqa_kernel(const PrefillParams p, int n_items) {
    typedef typename Elem<T>::vec4 V4;
    constexpr int D = 128, BN = 64, DCH = 16, INSTR = 4;
    __shared__ __attribute__((aligned(16))) T smem[4 * BN * D];    // K0, K1, V0, V1
    __shared__ __attribute__((aligned(16))) T ostage[4 * 64 * D];  // O staging: 64 rows per wave

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hf = lane >> 5;
    const int G = gridDim.x;
    const int nsub = p.group / 4;  // 4-head subgroups per kv head (the host checks group % 4 == 0)

    const int krow = (int)(p.ks_s * (int64_t)sizeof(T));
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(T));
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;
    u32x8 doff;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
        const int r = (wave * INSTR + i) * 4 + lane / DCH;
        const int cc = (lane % DCH) ^ kswz128(r);
        doff[i] = (uint32_t)(r * krow + cc * 16);
        doff[INSTR + i] = (uint32_t)(r * vrow + cc * 16);
    }
    const uint32_t m0base = __builtin_amdgcn_readfirstlane(sbase + (uint32_t)(wave * INSTR * 1024));

    struct Item {
        int b, hq, q0, nt;
        const T *qp, *kp, *vp;
    };
    auto item_at = [&](int bid) {
        const BlockCoord bc = block_coord_at<CAUSAL>(bid, p.B, p.Hkv * nsub, p.Hkv, nsub, p.n_qblocks, p.xcd_map);
        Item it;
        it.b = bc.b;
        it.hq = bc.hk * p.group + (bc.hq - bc.hk * nsub) * 4 + wave;
        it.q0 = bc.qb * 64;
        int kend = p.Sk;
        if (CAUSAL) {
            const int lim = it.q0 + 64 + p.delta;
            kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
        }
        it.nt = (kend + BN - 1) / BN;
        it.qp = reinterpret_cast<const T*>(p.q) + it.b * p.qs_b + it.hq * p.qs_h;
        it.kp = reinterpret_cast<const T*>(p.k) + it.b * p.ks_b + bc.hk * p.ks_h;
        it.vp = reinterpret_cast<const T*>(p.v) + it.b * p.vs_b + bc.hk * p.vs_h;
        return it;
    };
    auto dma = [&](int buf, const T* base, int pitch, int64_t stride, int t, int first) {
        const int rows = min(BN, p.Sk - t * BN);
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + D * (int)sizeof(T));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
        T* dst = smem + buf * BN * D;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) buf_ld16_lds_async(rs, dst + (wave * INSTR + i) * 4 * D, doff[first + i]);
    };
    u32x32 QA, QB;
    auto prefetch = [&](const Item& it) {
        if (it.nt > 0) {
            dma(0, it.kp, krow, p.ks_s, 0, 0);
            dma(2, it.vp, vrow, p.vs_s, 0, INSTR);
            if (it.nt > 1) dma(1, it.kp, krow, p.ks_s, 1, 0);
        }
        const T* qa = it.qp + (int64_t)min(it.q0 + l32, p.Sq - 1) * p.qs_s + hf * 8;
        const T* qb = it.qp + (int64_t)min(it.q0 + 32 + l32, p.Sq - 1) * p.qs_s + hf * 8;
        asm volatile(
            "global_load_dwordx4 a[128:131], %2, off\n\tglobal_load_dwordx4 a[132:135], %2, off offset:32\n\t"
            "global_load_dwordx4 a[136:139], %2, off offset:64\n\tglobal_load_dwordx4 a[140:143], %2, off offset:96\n\t"
            "global_load_dwordx4 a[144:147], %2, off offset:128\n\tglobal_load_dwordx4 a[148:151], %2, off offset:160\n\t"
            "global_load_dwordx4 a[152:155], %2, off offset:192\n\tglobal_load_dwordx4 a[156:159], %2, off offset:224\n\t"
            "global_load_dwordx4 a[160:163], %3, off\n\tglobal_load_dwordx4 a[164:167], %3, off offset:32\n\t"
            "global_load_dwordx4 a[168:171], %3, off offset:64\n\tglobal_load_dwordx4 a[172:175], %3, off offset:96\n\t"
            "global_load_dwordx4 a[176:179], %3, off offset:128\n\tglobal_load_dwordx4 a[180:183], %3, off offset:160\n\t"
            "global_load_dwordx4 a[184:187], %3, off offset:192\n\tglobal_load_dwordx4 a[188:191], %3, off offset:224"
            : "={a[128:159]}"(QA), "={a[160:191]}"(QB)
            : "v"(qa), "v"(qb)
            : "memory");
    };

    if ((int)blockIdx.x >= n_items) return;
    int k = 0;
    Item it = item_at(gqa_item(blockIdx.x, 0, G, p.xcd_map));
    prefetch(it);
    while (true) {
        u32x16 addr;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) addr[ks] = sbase + (uint32_t)(l32 * D + 8 * ((2 * ks + hf) ^ kswz128(l32))) * 2u;
        {
            const int blk = lane >> 4, bl = lane & 15;
            const int tr_key = bl >> 2, tr_d = 16 * (blk & 1) + 4 * (bl & 3), tr_k4 = 4 * (blk >> 1);
            const int k1 = tr_k4 + tr_key, k2 = k1 + 8;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int d = dt * 32 + tr_d;
                addr[8 + dt] = sbase + (uint32_t)(k1 * D + 8 * ((d >> 3) ^ kswz128(k1)) + (d & 7)) * 2u;
                addr[12 + dt] = sbase + (uint32_t)(k2 * D + 8 * ((d >> 3) ^ kswz128(k2)) + (d & 7)) * 2u;
            }
        }
        u32x2 lim;
#pragma unroll
        for (int X = 0; X < 2; ++X) {
            int v = p.Sk - 1;
            if (CAUSAL) v = min(v, it.q0 + 32 * X + l32 + p.delta);
            lim[X] = (uint32_t)(v - 4 * hf);
        }
        f32x32 OA01, OA23, OB01, OB23;
#pragma unroll
        for (int i = 0; i < 32; ++i) OA01[i] = 0.f, OA23[i] = 0.f, OB01[i] = 0.f, OB23[i] = 0.f;
        float mA = kNegInf, mB = kNegInf, lA = 0.f, lB = 0.f;
        const float c = p.c;
        const int kd = it.q0 + p.delta;
        const int nt = __builtin_amdgcn_readfirstlane(it.nt), tw = nt;
        const uint64_t kb64 = (uint64_t)(uintptr_t)it.kp, vb64 = (uint64_t)(uintptr_t)it.vp;
        const uint32_t klo = __builtin_amdgcn_readfirstlane((uint32_t)kb64);
        const uint32_t khi = __builtin_amdgcn_readfirstlane((uint32_t)(kb64 >> 32));
        const uint32_t vlo = __builtin_amdgcn_readfirstlane((uint32_t)vb64);
        const uint32_t vhi = __builtin_amdgcn_readfirstlane((uint32_t)(vb64 >> 32));
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this item's Q and first tiles (and the last stores)
        lds_barrier();
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is named as clobbered: the program sets it for its loads
        if (nt > 0) {
#define DTATTN_ROWS64_GQA_OPERANDS                                                                             \
    : "+{a[0:31]}"(OA01), "+{a[32:63]}"(OA23), "+{a[64:95]}"(OB01), "+{a[96:127]}"(OB23), [mA] "+v"(mA),       \
      [mB] "+v"(mB), [lA] "+v"(lA), [lB] "+v"(lB)                                                                \
    : "{a[128:159]}"(QA), "{a[160:191]}"(QB), "{v[200:215]}"(addr), [nt] "s"(nt), [tw] "s"(tw), [c] "s"(c),    \
      [sk] "s"(p.Sk), [kd] "s"(kd), [kp] "s"(krow), [vp] "s"(vrow), [klo] "s"(klo), [khi] "s"(khi),            \
      [vlo] "s"(vlo), [vhi] "s"(vhi), [m0base] "s"(m0base), "{v[216:223]}"(doff), "{v[224:225]}"(lim)
            constexpr bool F16 = __is_same(T, f16_t);
            if constexpr (F16 && CAUSAL) asm volatile(DTATTN_ROWS64_PROGRAM_F16_4_1 DTATTN_ROWS64_GQA_OPERANDS : DTATTN_ROWS64_CLOBBERS);
            else if constexpr (F16) asm volatile(DTATTN_ROWS64_PROGRAM_F16_4_0 DTATTN_ROWS64_GQA_OPERANDS : DTATTN_ROWS64_CLOBBERS);
            else if constexpr (CAUSAL) asm volatile(DTATTN_ROWS64_PROGRAM_BF16_4_1 DTATTN_ROWS64_GQA_OPERANDS : DTATTN_ROWS64_CLOBBERS);
            else asm volatile(DTATTN_ROWS64_PROGRAM_BF16_4_0 DTATTN_ROWS64_GQA_OPERANDS : DTATTN_ROWS64_CLOBBERS);
#undef DTATTN_ROWS64_GQA_OPERANDS
        }
#pragma clang diagnostic pop
        // every wave is past its last K/V read: the buffers take the next item's tiles during this epilogue
        lds_barrier();
        const Item cur = it;
        ++k;
        const int nbid = gqa_item(blockIdx.x, k, G, p.xcd_map);
        const bool more = nbid < n_items;
        if (more) {
            it = item_at(nbid);
            prefetch(it);
        }
        // Epilogue: normalise, stage O through this wave's 64 rows of LDS (16-byte chunk c of row r at
        // c ^ (r % 16)) for 16-byte coalesced row stores, LSE
        T* Os = ostage + wave * 64 * D;
#pragma unroll
        for (int X = 0; X < 2; ++X) {
            const float l = sum_xor32(X == 0 ? lA : lB);
            const float m = X == 0 ? mA : mB;
            const float inv = l > 0.f ? 1.f / l : 0.f;
            const int row = 32 * X + l32;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    V4 o4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int kk = 16 * (dt & 1) + 4 * i4 + e;
                        const float ov = X == 0 ? (dt < 2 ? OA01[kk] : OA23[kk]) : (dt < 2 ? OB01[kk] : OB23[kk]);
                        o4[e] = Elem<T>::from_f32(ov * inv);
                    }
                    const int cc = dt * 4 + i4;
                    *reinterpret_cast<V4*>(Os + row * D + 8 * (cc ^ (row % DCH)) + 4 * hf) = o4;
                }
            if (p.lse != nullptr && hf == 0) {
                const int qrow = cur.q0 + row;
                if (qrow < p.Sq)
                    p.lse[cur.b * p.lses_b + cur.hq * p.lses_h + qrow] = l > 0.f ? (m + __log2f(l)) * kLn2 : kNegInf;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave reads back only its own staged rows
        T* op = reinterpret_cast<T*>(p.o) + cur.b * p.os_b + cur.hq * p.os_h;
#pragma unroll
        for (int i = 0; i < 64 * DCH / 64; ++i) {
            const int id = i * 64 + lane;
            const int row = id / DCH, cc = id % DCH;
            const int qrow = cur.q0 + row;
            if (qrow < p.Sq)
                __builtin_nontemporal_store(ld16(Os + row * D + 8 * (cc ^ (row % DCH))),
                                            reinterpret_cast<u32x4*>(op + (int64_t)qrow * p.os_s + cc * 8));
        }
        if (!more) break;
    }
}

template <typename T, bool CAUSAL, int NW>
static int launch_rows64(const PrefillParams& prm, hipStream_t stream) {
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + 64 * NW - 1) / (64 * NW);
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_rows64_kernel<T, CAUSAL, NW>), dim3((unsigned)grid), dim3(64 * NW), 0, stream, p);
    return check_launch("prefill_rows64_kernel");
}

// Whether a head-dim-128 call without mask or padding can take the 64-row kernel: its tile loop computes the
// byte offset of a K/V tile in 32-bit scalar arithmetic.
bool prefill_rows64_fits(const PrefillParams& p) {
    const int64_t pitch = (p.ks_s > p.vs_s ? p.ks_s : p.vs_s) * 2;
    return p.ks_s >= 0 && p.vs_s >= 0 && ((int64_t)p.Sk + 128) * pitch < ((int64_t)1 << 31);
}

static int rows64_stream_device(hipStream_t stream, int* dev) {
    return (stream == nullptr ? hipGetDevice(dev) : hipStreamGetDevice(stream, dev)) == hipSuccess ? DTATTN_OK
                                                                                               : DTATTN_ERR_DEVICE;
}

template <typename T, bool CAUSAL>
static int launch_rows64_gqa(const PrefillParams& prm, int cus, hipStream_t stream) {
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + 63) / 64;
    const int64_t n_items = (int64_t)p.n_qblocks * p.B * (p.Hq / 4);
    if (n_items == 0) return DTATTN_OK;
    if (n_items > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill: too many work items");
    int grid = n_items < cus ? (int)n_items : cus;
    if (p.xcd_map) grid &= ~7;  // the item map deals items to XCDs in groups of 8 (n_items is a multiple of 8)
    hipLaunchKernelGGL((prefill_rows64_gqa_kernel<T, CAUSAL>), dim3((unsigned)grid), dim3(256), 0, stream, p,
                       (int)n_items);
    return check_launch("prefill_rows64_gqa_kernel");
}

int prefill_rows64(const PrefillParams& p, bool causal, bool f16, hipStream_t stream) {
    // grouped-query calls with groups of 4k heads and a positive scale take the persistent form
    if (p.group >= 4 && p.group % 4 == 0 && p.q_and == 0xffffffffu && p.q_xor == 0u) {
        int dev = 0;
        dtattn_device_peaks pk;
        if (rows64_stream_device(stream, &dev) == DTATTN_OK && dtattn_get_device_peaks(dev, &pk) == DTATTN_OK &&
            pk.cu_count >= 8) {
            if (f16)
                return causal ? launch_rows64_gqa<f16_t, true>(p, pk.cu_count, stream)
                              : launch_rows64_gqa<f16_t, false>(p, pk.cu_count, stream);
            return causal ? launch_rows64_gqa<bf16_t, true>(p, pk.cu_count, stream)
                          : launch_rows64_gqa<bf16_t, false>(p, pk.cu_count, stream);
        }
    }
    if (f16)
        return causal ? launch_rows64<f16_t, true, 2>(p, stream) : launch_rows64<f16_t, false, 4>(p, stream);
    return causal ? launch_rows64<bf16_t, true, 2>(p, stream) : launch_rows64<bf16_t, false, 4>(p, stream);
}

}  // namespace dtattn
