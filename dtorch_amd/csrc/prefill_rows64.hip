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
#include <cmath>

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

// Stream-K form of the persistent layouts (non-causal, positive scale).  Work items of the row layout (4 waves x
// 64 consecutive rows of one head) or of the grouped-query form (the 4 query heads of a kv head over 64 rows)
// run one workgroup per CU; a grid of items that does not fill whole rounds of the CUs leaves part of the chip
// idle (128 items on 256 CUs: half of it).  Here each workgroup takes an equal, contiguous share of all (item,
// key tile) units, items in order with the query block fastest, and runs it as segments: whole items end in
// the usual epilogue, and the at most two segments of a share that cut an item (its first and its last) leave
// O over their own row sums, the row maxima and the row sums in a workspace record, which a second launch
// merges by the row maxima.  Shares are dealt XCD by XCD (workgroup w on XCD w % 8 takes share (w % 8) G/8 +
// w / 8), so an XCD walks consecutive query blocks of the same heads and their K/V stay in its L2.
struct Rows64Sk {
    int64_t units;  // n_items * nt
    int32_t nt;     // key tiles per item
    int32_t nqb;    // query blocks per item column: of 256 rows (row layout) or 64 rows (grouped-query form)
    int32_t G;      // workgroups (a multiple of 8)
    char* ws;       // 2 G records of kRows64SkRec bytes
};

// Batch, query head and first row of wave `wave` in item i.  Row layout: 4 waves x 64 consecutive rows of one
// head, items (b, hq, 256-row block).  Grouped-query form (GQA): the 4 query heads of one kv head over the
// same 64 rows, items (b, kv head, 4-head subgroup, 64-row block).  The query block runs fastest in both.
template <bool GQA>
__device__ __forceinline__ void sk_item(const PrefillParams& p, const Rows64Sk& sk, int i, int wave, int* b,
                                        int* hq, int* q0) {
    const int qb = i % sk.nqb, rest = i / sk.nqb;
    if constexpr (GQA) {
        const int nsub = p.group / 4;
        *b = rest / (p.Hkv * nsub);
        const int r2 = rest % (p.Hkv * nsub);
        *hq = (r2 / nsub) * p.group + (r2 % nsub) * 4 + wave;
        *q0 = qb * 64;
    } else {
        *b = rest / p.Hq;
        *hq = rest % p.Hq;
        *q0 = qb * 256 + wave * 64;
    }
}
// One record: lane l of wave w holds O / l of its 128 accumulators in the input dtype, as the blockwise ring
// step keeps its key blocks' outputs before their LSE merge (the epilogue's order: 16-byte chunk
// q = 8 X + 2 dt + i4 / 2 at (16 w + q) 64 + l), then, in fp32, its rows' (max A, max B, sum A, sum B) at byte
// 65536 + 16 (64 w + l).
constexpr int kRows64SkRec = 4 * 64 * 128 * 2 + 4 * 64 * 16;

__device__ __forceinline__ int64_t sk_start(int64_t units, int G, int r) { return units * r / G; }

template <typename T, bool GQA>
__global__ void __launch_bounds__(256, 1) prefill_rows64_sk_kernel(const PrefillParams p, const Rows64Sk sk) {
    typedef typename Elem<T>::vec4 V4;
    constexpr int D = 128, BN = 64, DCH = 16, INSTR = 4;
    __shared__ __attribute__((aligned(16))) T smem[4 * BN * D];    // K0, K1, V0, V1
    __shared__ __attribute__((aligned(16))) T ostage[4 * 64 * D];  // O staging: 64 rows per wave

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hf = lane >> 5;
    const int G = sk.G;
    const int rank = (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3);
    const int64_t u0 = sk_start(sk.units, G, rank), u1 = sk_start(sk.units, G, rank + 1);
    if (u0 >= u1) return;  // workgroup-uniform

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

    // segment: tiles t0 .. t1-1 of item i (this wave: rows q0 .. q0+63 of head hq); its keys start at key
    // 64 t0, so K/V are addressed from there and the program sees skr = Sk - 64 t0 keys
    struct Seg {
        int b, hq, q0, nt, skr, slot;
        bool whole;
        const T *qp, *kp, *vp;
    };
    auto seg_at = [&](int64_t u) {
        Seg s;
        const int i = (int)(u / sk.nt);
        const int t0 = (int)(u - (int64_t)i * sk.nt);
        const int t1 = (int)min((int64_t)sk.nt, (int64_t)t0 + (u1 - u));
        sk_item<GQA>(p, sk, i, wave, &s.b, &s.hq, &s.q0);
        const int hk = s.hq / p.group;
        s.nt = t1 - t0;
        s.skr = p.Sk - t0 * BN;
        s.whole = t0 == 0 && t1 == sk.nt;
        s.slot = 2 * rank + (u == u0 ? 0 : 1);
        s.qp = reinterpret_cast<const T*>(p.q) + s.b * p.qs_b + s.hq * p.qs_h;
        s.kp = reinterpret_cast<const T*>(p.k) + s.b * p.ks_b + hk * p.ks_h + (int64_t)t0 * BN * p.ks_s;
        s.vp = reinterpret_cast<const T*>(p.v) + s.b * p.vs_b + hk * p.vs_h + (int64_t)t0 * BN * p.vs_s;
        return s;
    };
    auto dma = [&](int buf, const T* base, int pitch, int64_t stride, int t, int skr, int first) {
        const int rows = min(BN, skr - t * BN);
        const uint32_t nbytes = (uint32_t)((rows - 1) * pitch + D * (int)sizeof(T));
        const auto rs = make_rsrc(base + (int64_t)t * BN * stride, nbytes);
        T* dst = smem + buf * BN * D;
#pragma unroll
        for (int i = 0; i < INSTR; ++i) buf_ld16_lds_async(rs, dst + (wave * INSTR + i) * 4 * D, doff[first + i]);
    };
    u32x32 QA, QB;
    auto prefetch = [&](const Seg& s) {
        dma(0, s.kp, krow, p.ks_s, 0, s.skr, 0);
        dma(2, s.vp, vrow, p.vs_s, 0, s.skr, INSTR);
        if (s.nt > 1) dma(1, s.kp, krow, p.ks_s, 1, s.skr, 0);
        const T* qa = s.qp + (int64_t)min(s.q0 + l32, p.Sq - 1) * p.qs_s + hf * 8;
        const T* qb = s.qp + (int64_t)min(s.q0 + 32 + l32, p.Sq - 1) * p.qs_s + hf * 8;
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

    int64_t u = u0;
    Seg s = seg_at(u);
    prefetch(s);
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
        lim[0] = lim[1] = (uint32_t)(s.skr - 1 - 4 * hf);
        f32x32 OA01, OA23, OB01, OB23;
#pragma unroll
        for (int i = 0; i < 32; ++i) OA01[i] = 0.f, OA23[i] = 0.f, OB01[i] = 0.f, OB23[i] = 0.f;
        float mA = kNegInf, mB = kNegInf, lA = 0.f, lB = 0.f;
        const float c = p.c;
        const int kd = 0;  // causal offsets only
        const int nt = __builtin_amdgcn_readfirstlane(s.nt), tw = nt;
        const int skr = __builtin_amdgcn_readfirstlane(s.skr);
        const uint64_t kb64 = (uint64_t)(uintptr_t)s.kp, vb64 = (uint64_t)(uintptr_t)s.vp;
        const uint32_t klo = __builtin_amdgcn_readfirstlane((uint32_t)kb64);
        const uint32_t khi = __builtin_amdgcn_readfirstlane((uint32_t)(kb64 >> 32));
        const uint32_t vlo = __builtin_amdgcn_readfirstlane((uint32_t)vb64);
        const uint32_t vhi = __builtin_amdgcn_readfirstlane((uint32_t)(vb64 >> 32));
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this segment's Q and first tiles (and the last stores)
        lds_barrier();
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is named as clobbered: the program sets it for its loads
#define DTATTN_ROWS64_SK_OPERANDS                                                                              \
    : "+{a[0:31]}"(OA01), "+{a[32:63]}"(OA23), "+{a[64:95]}"(OB01), "+{a[96:127]}"(OB23), [mA] "+v"(mA),       \
      [mB] "+v"(mB), [lA] "+v"(lA), [lB] "+v"(lB)                                                                \
    : "{a[128:159]}"(QA), "{a[160:191]}"(QB), "{v[200:215]}"(addr), [nt] "s"(nt), [tw] "s"(tw), [c] "s"(c),    \
      [sk] "s"(skr), [kd] "s"(kd), [kp] "s"(krow), [vp] "s"(vrow), [klo] "s"(klo), [khi] "s"(khi),             \
      [vlo] "s"(vlo), [vhi] "s"(vhi), [m0base] "s"(m0base), "{v[216:223]}"(doff), "{v[224:225]}"(lim)
        if constexpr (__is_same(T, f16_t)) asm volatile(DTATTN_ROWS64_PROGRAM_F16_4_0 DTATTN_ROWS64_SK_OPERANDS : DTATTN_ROWS64_CLOBBERS);
        else asm volatile(DTATTN_ROWS64_PROGRAM_BF16_4_0 DTATTN_ROWS64_SK_OPERANDS : DTATTN_ROWS64_CLOBBERS);
#undef DTATTN_ROWS64_SK_OPERANDS
#pragma clang diagnostic pop
        // every wave is past its last K/V read: the buffers take the next segment's tiles during this epilogue
        lds_barrier();
        const Seg cur = s;
        u += cur.nt;
        const bool more = u < u1;
        if (more) {
            s = seg_at(u);
            prefetch(s);
        }
        if (!cur.whole) {
            // a cut item: O over this segment's row sums, the row maxima and the row sums go to its record
            char* rec = sk.ws + (int64_t)cur.slot * kRows64SkRec;
            float ls[2];
#pragma unroll
            for (int X = 0; X < 2; ++X) {
                const float l = sum_xor32(X == 0 ? lA : lB);
                const float inv = l > 0.f ? 1.f / l : 0.f;
                ls[X] = l;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                    for (int i8 = 0; i8 < 2; ++i8) {
                        float v[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int kk = 16 * (dt & 1) + 8 * i8 + e;
                            const float ov = X == 0 ? (dt < 2 ? OA01[kk] : OA23[kk]) : (dt < 2 ? OB01[kk] : OB23[kk]);
                            v[e] = ov * inv;
                        }
                        reinterpret_cast<u32x4*>(rec)[(16 * wave + 8 * X + 2 * dt + i8) * 64 + lane] = pack8<T>(v);
                    }
            }
            reinterpret_cast<f32x4*>(rec + 65536)[64 * wave + lane] = f32x4{mA, mB, ls[0], ls[1]};
            if (!more) break;
            continue;
        }
        // Epilogue of a whole item: prefill_rows64_gqa_kernel's, for this wave's rows of head cur.hq
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

// Merge of the items the shares cut.  Workgroup r - 1 takes the share boundary r; it merges the item that
// boundary falls in (unless an earlier boundary falls in the same item), combining the records of every
// share that covers part of it by their row maxima, in share order, then writes O and the LSE as the
// epilogue of an uncut item would.
template <typename T, bool GQA>
__global__ void __launch_bounds__(256) rows64_sk_merge_kernel(const PrefillParams p, const Rows64Sk sk) {
    typedef typename Elem<T>::vec4 V4;
    constexpr int D = 128, DCH = 16;
    __shared__ __attribute__((aligned(16))) T ostage[4 * 64 * D];
    const int G = sk.G;
    const int r = (int)blockIdx.x + 1;
    const int64_t ub = sk_start(sk.units, G, r);
    const int i = (int)(ub / sk.nt);
    const int64_t ib = (int64_t)i * sk.nt, ie = ib + sk.nt;
    if (ub == ib) return;                                   // the boundary is an item edge
    if (r >= 2 && sk_start(sk.units, G, r - 1) > ib) return;  // an earlier boundary merges this item

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hf = lane >> 5;
    // running (M, L, o) per row block: o = sum_p l_p 2^(m_p - M) O_p, L = sum_p l_p 2^(m_p - M)
    float o[128];
    float mA = kNegInf, mB = kNegInf, lA = 0.f, lB = 0.f;
#pragma unroll
    for (int k = 0; k < 128; ++k) o[k] = 0.f;
    for (int q = r - 1; q < G && sk_start(sk.units, G, q) < ie; ++q) {
        const int slot = 2 * q + ((q == r - 1 && sk_start(sk.units, G, q) < ib) ? 1 : 0);
        const char* rec = sk.ws + (int64_t)slot * kRows64SkRec;
        const f32x4 ml = reinterpret_cast<const f32x4*>(rec + 65536)[64 * wave + lane];
        const float nA = fmaxf(mA, ml[0]), nB = fmaxf(mB, ml[1]);
        // a max of -inf carries no keys: weight 0
        const float aA = mA == kNegInf ? 0.f : exp2f(mA - nA), bA = ml[0] == kNegInf ? 0.f : ml[2] * exp2f(ml[0] - nA);
        const float aB = mB == kNegInf ? 0.f : exp2f(mB - nB), bB = ml[1] == kNegInf ? 0.f : ml[3] * exp2f(ml[1] - nB);
        lA = lA * aA + bA;
        lB = lB * aB + bB;
        mA = nA;
        mB = nB;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            float v[8];
            unpack8<T>(reinterpret_cast<const u32x4*>(rec)[(16 * wave + c) * 64 + lane], v);
            const float a = c < 8 ? aA : aB, w = c < 8 ? bA : bB;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[8 * c + e] = o[8 * c + e] * a + v[e] * w;
        }
    }
    // the item's rows and head, as the main kernel derives them
    int b, hq, q0;
    sk_item<GQA>(p, sk, i, wave, &b, &hq, &q0);
    T* Os = ostage + wave * 64 * D;
#pragma unroll
    for (int X = 0; X < 2; ++X) {
        const float l = X == 0 ? lA : lB;  // whole row sums already
        const float m = X == 0 ? mA : mB;
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int row = 32 * X + l32;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                V4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = Elem<T>::from_f32(o[64 * X + 16 * dt + 4 * i4 + e] * inv);
                const int cc = dt * 4 + i4;
                *reinterpret_cast<V4*>(Os + row * D + 8 * (cc ^ (row % DCH)) + 4 * hf) = o4;
            }
        if (p.lse != nullptr && hf == 0) {
            const int qrow = q0 + row;
            if (qrow < p.Sq) p.lse[b * p.lses_b + hq * p.lses_h + qrow] = l > 0.f ? (m + __log2f(l)) * kLn2 : kNegInf;
        }
    }
    __syncthreads();
    T* op = reinterpret_cast<T*>(p.o) + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < 64 * DCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / DCH, cc = id % DCH;
        const int qrow = q0 + row;
        if (qrow < p.Sq)
            __builtin_nontemporal_store(ld16(Os + row * D + 8 * (cc ^ (row % DCH))),
                                        reinterpret_cast<u32x4*>(op + (int64_t)qrow * p.os_s + cc * 8));
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

// Shares of the stream-K form for a non-causal call (B, Hq, Sq, Sk; grouped-query items when gqa) on `cus` CUs,
// and the workspace its records need; false unless the model below says the shares beat the plain grid by 5%.
// Times in key tiles (of 64 keys for every wave of a CU): an item costs nt + 4 (Q load, first tiles, epilogue);
// a share its tiles plus 4 per segment, plus 14 for writing and merging the records (~36 MB at 256 CUs;
// measured 13-20 on the shapes of the tests).  By it, 1 x 8 x 4096 (128 items on 256 CUs) gains 26-30% and
// 1 x 24 x 4096 (384 items) 10%, while 1 x 24 x 4608 (432 items of 72 tiles) keeps the plain grid, where
// stream-K measured 1-3% slower.
bool rows64_sk_plan(int64_t B, int64_t Hq, int64_t Sq, int64_t Sk, bool gqa, int cus, Rows64Sk* sk, size_t* bytes) {
    const int G = cus & ~7;
    if (G < 8 || B <= 0 || Hq <= 0 || Sq <= 0 || Sk <= 0) return false;
    const int64_t nqb = gqa ? (Sq + 63) / 64 : (Sq + 255) / 256;
    const int64_t n_items = nqb * B * (gqa ? Hq / 4 : Hq), nt = (Sk + 63) / 64;
    if (n_items > 0x7fffffff || n_items * nt > ((int64_t)1 << 40)) return false;
    const int64_t units = n_items * nt;
    const double per = (double)units / G;
    if (per < 8.0) return false;
    const double plain = (double)((n_items + G - 1) / G) * (double)(nt + 4);
    const double segs = std::ceil(per / (double)nt) + 1.0;
    if (std::ceil(per) + 4.0 * segs + 14.0 >= 0.95 * plain) return false;
    sk->units = units;
    sk->nt = (int32_t)nt;
    sk->nqb = (int32_t)nqb;
    sk->G = G;
    sk->ws = nullptr;
    *bytes = (size_t)2 * G * kRows64SkRec;
    return true;
}

// Workspace the stream-K form can use for a prefill call on `device` (0: the call does not take it): bf16 /
// fp16 at head dims D = Dv = 128, non-causal, no mask, a positive scale, and tile offsets that fit the program's
// 32-bit arithmetic; items of the row layout, or of the grouped-query form for groups of 4k heads.
size_t rows64_sk_workspace(const dtattn_prefill_args* a, int device) {
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16) return 0;
    if (a->D != 128 || a->Dv != 128 || a->causal != 0 || a->mask != nullptr || a->scale <= 0.f) return 0;
    if (a->Hkv <= 0 || a->Hq % a->Hkv != 0) return 0;
    const int64_t group = a->Hq / a->Hkv;
    const bool gqa = group >= 4 && group % 4 == 0;
    const int64_t ks = a->k_stride[2], vs = a->v_stride[2];
    if (ks < 0 || vs < 0 || (a->Sk + 128) * (ks > vs ? ks : vs) * 2 >= ((int64_t)1 << 31)) return 0;
    dtattn_device_peaks pk;
    if (dtattn_get_device_peaks(device, &pk) != DTATTN_OK) return 0;
    Rows64Sk sk;
    size_t bytes = 0;
    return rows64_sk_plan(a->B, a->Hq, a->Sq, a->Sk, gqa, pk.cu_count, &sk, &bytes) ? bytes : 0;
}

template <typename T, bool GQA>
static int launch_rows64_sk(const PrefillParams& p, const Rows64Sk& sk, hipStream_t stream) {
    hipLaunchKernelGGL((prefill_rows64_sk_kernel<T, GQA>), dim3((unsigned)sk.G), dim3(256), 0, stream, p, sk);
    const int st = check_launch("prefill_rows64_sk_kernel");
    if (st != DTATTN_OK) return st;
    hipLaunchKernelGGL((rows64_sk_merge_kernel<T, GQA>), dim3((unsigned)(sk.G - 1)), dim3(256), 0, stream, p, sk);
    return check_launch("rows64_sk_merge_kernel");
}

// ws / ws_bytes: the caller's workspace (may be NULL); non-causal row-layout calls whose grid would leave a
// ragged last round take the stream-K form when it holds the records.
int prefill_rows64(const PrefillParams& p, bool causal, bool f16, void* ws, size_t ws_bytes, hipStream_t stream) {
    const bool positive = p.q_and == 0xffffffffu && p.q_xor == 0u;
    const bool gqa_form = p.group >= 4 && p.group % 4 == 0;
    if (!causal && positive && ws != nullptr && (reinterpret_cast<uintptr_t>(ws) & 255u) == 0) {
        int dev = 0;
        dtattn_device_peaks pk;
        Rows64Sk sk;
        size_t need = 0;
        if (rows64_stream_device(stream, &dev) == DTATTN_OK && dtattn_get_device_peaks(dev, &pk) == DTATTN_OK &&
            rows64_sk_plan(p.B, p.Hq, p.Sq, p.Sk, gqa_form, pk.cu_count, &sk, &need) && need <= ws_bytes) {
            sk.ws = static_cast<char*>(ws);
            if (gqa_form)
                return f16 ? launch_rows64_sk<f16_t, true>(p, sk, stream) : launch_rows64_sk<bf16_t, true>(p, sk, stream);
            return f16 ? launch_rows64_sk<f16_t, false>(p, sk, stream) : launch_rows64_sk<bf16_t, false>(p, sk, stream);
        }
    }
    // grouped-query calls with groups of 4k heads and a positive scale take the persistent form
    if (gqa_form && positive) {
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
