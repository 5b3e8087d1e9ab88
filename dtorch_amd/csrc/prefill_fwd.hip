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
//   row max / row sum need one cross-half exchange (lane ^ 32) instead of a 32-lane reduction.  The
//   output is accumulated transposed as well, O^T = V^T P^T: P^T comes straight from the score
//   registers (the MFMA reduction index is a free permutation, matched on both operands), and V is
//   written transposed into LDS so each lane reads 4 consecutive keys of one d with one 8-byte read.
//   The per-query rescale factor is then a per-lane scalar.
//
// LDS layouts (bank-conflict free for the 16-byte K reads and the 8-byte V^T reads/writes)
//   K  tile: [64 keys][D], 16-byte chunk c of row r stored at chunk c ^ kswz(r).
//   V^T tile: [D][64 keys], 4-key group g of row d stored at group g ^ ((d & 15) ^ ((d >> 4) & 15)).
//
// Pipeline per key tile j (K double-buffered in LDS and filled by direct global->LDS loads, V
// prefetched one tile ahead in registers and transposed into a single V^T buffer):
//   wait + barrier | V[j] regs -> V^T | V[j+1] -> regs (async) | K[j+1] -> LDS (async) |
//   S = K[j] Q^T | softmax | barrier | O^T += V^T P^T
#include <stdarg.h>
#include <stdio.h>

#include "dtattn_common.hpp"

namespace dtattn {

struct PrefillParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int64_t qs_b, qs_h, qs_s;
    int64_t ks_b, ks_h, ks_s;
    int64_t vs_b, vs_h, vs_s;
    int64_t os_b, os_h, os_s;
    int64_t lses_b, lses_h;
    int32_t B, Hq, Hkv, Sq, Sk, group;
    int32_t n_qblocks;
    int32_t delta;  // key j visible to query i iff j <= i + delta (causal only)
    float c;        // softmax scale * log2(e)
    int32_t xcd_map;  // 1: group the workgroups of each (batch, kv head) slice on one XCD
};

// Workgroup -> (query block, batch, query head).  Causal launches take the longest query blocks
// first.  Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8), each with its own L2;
// with xcd_map the slices (b, kv head) are dealt to XCDs so that every workgroup reading a slice's
// K/V runs on the same XCD and the slice is fetched from HBM once per L2 instead of once per XCD.
struct BlockCoord {
    int qb, b, hq, hk;
};

template <bool CAUSAL>
__device__ __forceinline__ BlockCoord block_coord(const PrefillParams& p) {
    const int bid = blockIdx.x;
    BlockCoord r;
    if (p.xcd_map) {
        const int x = bid & 7, j = bid >> 3;
        const int per_rank = (p.B * p.Hkv / 8) * p.group;  // workgroups per query-block rank per XCD
        const int rank = j / per_rank, rem = j % per_rank;
        const int slice = (rem / p.group) * 8 + x;
        r.b = slice / p.Hkv;
        r.hk = slice % p.Hkv;
        r.hq = r.hk * p.group + rem % p.group;
        r.qb = CAUSAL ? (p.n_qblocks - 1 - rank) : rank;
    } else {
        const int bh = p.B * p.Hq;
        const int rest = bid % bh;
        r.qb = CAUSAL ? (p.n_qblocks - 1 - bid / bh) : (bid / bh);
        r.hq = rest % p.Hq;
        r.b = rest / p.Hq;
        r.hk = r.hq / p.group;
    }
    return r;
}

// Lazy rescaling: the running max only moves (and O, l are only rescaled) when some row's max grew
// by more than 2^8; otherwise P is taken against the stale max (values up to 2^8, exact in the
// normalisation, which uses the same max for O and l).
constexpr float kRescaleThreshold = 8.0f;

template <int D>
__device__ __forceinline__ int kswz(int r) {
    return D >= 128 ? (r & 15) : (r & 7);
}

__device__ __forceinline__ int vswz(int d) { return (d & 15) ^ ((d >> 4) & 15); }

// Pack the (e)-th 16-bit half of two dwords into one dword: low half from a, high half from b.
__device__ __forceinline__ uint32_t pack_half(uint32_t a, uint32_t b, int e) {
    return __builtin_amdgcn_perm(b, a, e ? 0x07060302u : 0x05040100u);
}

template <typename T, int D, int QT, bool CAUSAL>
__global__ void __launch_bounds__(256, 2) prefill_fwd_kernel(const PrefillParams p) {
    constexpr int NW = 4;
    constexpr int BN = 64;
    constexpr int BM = NW * QT * 32;
    constexpr int DCH = D / 8;            // 16-byte chunks per row
    constexpr int KSTEPS = D / 16;        // MFMA k-steps of S = K Q^T
    constexpr int DT = D / 32;            // 32-row d tiles of O^T
    constexpr int KT = BN / 32;           // 32-key tiles per key block
    constexpr int PVS = BN / 16;          // MFMA k-steps of O^T = V^T P^T
    constexpr int NVB = (BN / 4) * DCH;   // 4-key x 8-d blocks of V per tile
    static_assert((BN * DCH) % 256 == 0, "tile/thread mismatch");
    static_assert(NVB <= 256, "one V block per thread at most");
    static_assert(QT == 1, "the output staging reuses the two K buffers: 2 waves x 32 rows each");
    typedef typename Elem<T>::vec8 V8;

    // Three distinct LDS objects so the compiler's alias analysis can tell the in-flight K load
    // (into one buffer) from the reads of the other buffer and from the V^T writes.
    __shared__ __attribute__((aligned(16))) T Ksa[BN * D];
    __shared__ __attribute__((aligned(16))) T Ksb[BN * D];
    __shared__ __attribute__((aligned(16))) T VTs[D * BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hf = lane >> 5;

    const BlockCoord bc = block_coord<CAUSAL>(p);
    const int qb = bc.qb, b = bc.b, hq = bc.hq, hk = bc.hk;

    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const T* kp = reinterpret_cast<const T*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const T* vp = reinterpret_cast<const T*>(p.v) + b * p.vs_b + hk * p.vs_h;

    const int q0 = qb * BM;
    const int wq0 = q0 + wave * QT * 32;

    int kend = p.Sk;
    if (CAUSAL) {
        const int lim = q0 + BM + p.delta;  // keys < lim can be visible
        kend = lim < 0 ? 0 : (lim < p.Sk ? lim : p.Sk);
    }
    const int nt = (kend + BN - 1) / BN;

    // Q fragments (B operand of S^T = K Q^T): lane holds query l32, d = ks*16 + hf*8 .. +8.
    V8 qf[QT][KSTEPS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qrow = wq0 + qt * 32 + l32;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (qrow < p.Sq) raw = ld16(qp + (int64_t)qrow * p.qs_s + ks * 16 + hf * 8);
            qf[qt][ks] = __builtin_bit_cast(V8, raw);
        }
    }

    f32x16 oacc[QT][DT];
    float mrow[QT], lrow[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        mrow[qt] = kNegInf;
        lrow[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[qt][dt][i] = 0.f;
    }

    u32x4 vreg[4];
    const int krow = (int)(p.ks_s * (int64_t)sizeof(T));  // row pitch in bytes (< 2^25, host-checked)
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(T));

    // Buffer resource over the valid rows of key tile t: offsets past the last row read zeros.
    auto tile_rsrc = [&](const T* base, int pitch, int64_t stride, int t) {
        const int rows = min(BN, p.Sk - t * BN);
        return make_rsrc(base + (int64_t)t * BN * stride, (uint32_t)((rows - 1) * pitch + D * (int)sizeof(T)));
    };

    // K tile t -> LDS by direct buffer->LDS loads: one wave instruction fills 1 KB of LDS (lane l ->
    // byte 16*l), i.e. 1024/(2*D) rows; lane l therefore loads the global chunk that belongs at its
    // LDS slot, c = slot ^ kswz(row).
    auto dma_k = [&](T* dst, int t) {
        constexpr int ROWS_PER_INSTR = 1024 / (2 * D);
        constexpr int INSTR = BN / ROWS_PER_INSTR / NW;  // per wave
        const auto rs = tile_rsrc(kp, krow, p.ks_s, t);
#pragma unroll
        for (int i = 0; i < INSTR; ++i) {
            const int r0 = (wave * INSTR + i) * ROWS_PER_INSTR;
            const int r = r0 + lane / DCH;
            const int c = (lane % DCH) ^ kswz<D>(r);
            buf_ld16_lds(rs, dst + r0 * D, (uint32_t)(r * krow + c * 16));
        }
    };
    auto load_v = [&](int t) {
        if (NVB == 256 || tid < NVB) {
            const int g = tid / DCH, c = tid % DCH;
            const auto rs = tile_rsrc(vp, vrow, p.vs_s, t);
#pragma unroll
            for (int i = 0; i < 4; ++i) vreg[i] = buf_ld16(rs, (uint32_t)((4 * g + i) * vrow + c * 16));
        }
    };
    auto store_v = [&]() {
        if (NVB == 256 || tid < NVB) {
            const int g = tid / DCH, c = tid % DCH;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int d = c * 8 + 2 * w + e;
                    u32x2 pr;
                    pr.x = pack_half(vreg[0][w], vreg[1][w], e);
                    pr.y = pack_half(vreg[2][w], vreg[3][w], e);
                    *reinterpret_cast<u32x2*>(VTs + d * BN + 4 * (g ^ vswz(d))) = pr;
                }
            }
        }
    };

    // One key tile.  Kcur holds K[t]; Knext receives K[t+1] while this tile computes.
    auto tile = [&](const T* Kcur, T* Knext, int t) {
        // K[t] (direct-to-LDS) and V[t] (registers) have landed for this wave; after the barrier
        // every wave's share is visible and every wave has finished tile t-1.
        wait_vmem();
        lds_barrier();
        store_v();
        if (t + 1 < nt) {
            load_v(t + 1);
            dma_k(Knext, t + 1);
        }

        const int kbase = t * BN;
        const bool wave_skip = CAUSAL && (kbase > wq0 + QT * 32 - 1 + p.delta);
        const bool need_mask = (kbase + BN > p.Sk) || (CAUSAL && (kbase + BN - 1 > wq0 + p.delta));

        V8 pb[QT][PVS];
        if (!wave_skip) {
            f32x16 s[QT][KT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[qt][kt][i] = 0.f;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    const int r = kt * 32 + l32;
                    const int c = ks * 2 + hf;
                    V8 a = *reinterpret_cast<const V8*>(Kcur + r * D + 8 * (c ^ kswz<D>(r)));
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) s[qt][kt] = Elem<T>::mfma32(a, qf[qt][ks], s[qt][kt]);
                }
            }
            if (need_mask) {
                // Element i of key tile kt holds key kbase + kt*32 + 8*(i/4) + 4*hf + i%4; it is
                // visible iff its compile-time offset kt*32 + 8*(i/4) + i%4 is <= lim.
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    int lim = p.Sk - 1 - kbase;
                    if (CAUSAL) lim = min(lim, wq0 + qt * 32 + l32 + p.delta - kbase);
                    lim -= 4 * hf;
#pragma unroll
                    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            if (kt * 32 + 8 * (i >> 2) + (i & 3) > lim) s[qt][kt][i] = kNegInf;
                }
            }
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                float mx = kNegInf;
#pragma unroll
                for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[qt][kt][i]);
                mx = max_xor32(mx);
                const float mcand = fmaxf(mrow[qt], mx * p.c);
                if (__any(mcand - mrow[qt] > kRescaleThreshold)) {  // wave-uniform
                    const float alpha = fast_exp2(mrow[qt] - (mcand == kNegInf ? 0.f : mcand));
                    mrow[qt] = mcand;
                    lrow[qt] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                        for (int i = 0; i < 16; ++i) oacc[qt][dt][i] *= alpha;
                }
                const float mbase = (mrow[qt] == kNegInf) ? 0.f : mrow[qt];
                float ls = lrow[qt];
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        V8 pk;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const float pv = fast_exp2(__builtin_fmaf(s[qt][kt][8 * half + e], p.c, -mbase));
                            ls += pv;
                            pk[e] = Elem<T>::from_f32(pv);
                        }
                        pb[qt][2 * kt + half] = pk;
                    }
                }
                lrow[qt] = ls;
            }
        }

        lds_barrier();  // V^T of tile t visible

        if (!wave_skip) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int d = dt * 32 + l32;
                const int sw = vswz(d);
#pragma unroll
                for (int ks = 0; ks < PVS; ++ks) {
                    const int g1 = ks * 4 + hf, g2 = ks * 4 + 2 + hf;
                    const u32x2 lo = *reinterpret_cast<const u32x2*>(VTs + d * BN + 4 * (g1 ^ sw));
                    const u32x2 hi = *reinterpret_cast<const u32x2*>(VTs + d * BN + 4 * (g2 ^ sw));
                    const u32x4 raw = {lo.x, lo.y, hi.x, hi.y};
                    const V8 a = __builtin_bit_cast(V8, raw);
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) oacc[qt][dt] = Elem<T>::mfma32(a, pb[qt][ks], oacc[qt][dt]);
                }
            }
        }
    };

    if (nt > 0) {
        dma_k(Ksa, 0);
        load_v(0);
    }
    for (int t = 0; t < nt; t += 2) {  // unrolled by two so each tile names its K buffers statically
        tile(Ksa, Ksb, t);
        if (t + 1 < nt) tile(Ksb, Ksa, t + 1);
    }

    // Epilogue: normalise, stage O through LDS (waves 0-1 in Ksa, 2-3 in Ksb; 16-byte chunk c of
    // row r at c ^ (r % DCH)) for 16-byte coalesced row stores, and write the LSE.
    __syncthreads();
    T* Os = (wave < 2 ? Ksa : Ksb) + (wave & 1) * 32 * D;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float l = sum_xor32(lrow[qt]);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int row = qt * 32 + l32;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                typename Elem<T>::vec4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) o4[e] = Elem<T>::from_f32(oacc[qt][dt][4 * i4 + e] * inv);
                const int c = dt * 4 + i4;
                *reinterpret_cast<typename Elem<T>::vec4*>(Os + row * D + 8 * (c ^ (row % DCH)) + 4 * hf) = o4;
            }
        if (p.lse != nullptr && hf == 0) {
            const int qrow = wq0 + row;
            if (qrow < p.Sq) {
                const float lse = l > 0.f ? (mrow[qt] + __log2f(l)) * kLn2 : kNegInf;
                p.lse[b * p.lses_b + hq * p.lses_h + qrow] = lse;
            }
        }
    }
    __syncthreads();
    T* op = reinterpret_cast<T*>(p.o) + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int it = 0; it < QT * 32 * DCH / 64; ++it) {
        const int id = it * 64 + lane;
        const int row = id / DCH, c = id % DCH;
        const int qrow = wq0 + row;
        if (qrow < p.Sq) st16(op + (int64_t)qrow * p.os_s + c * 8, ld16(Os + row * D + 8 * (c ^ (row % DCH))));
    }
}

// ------------------------------------------------------------------------------------------------

template <typename T, int D, int QT, bool CAUSAL>
static int launch_prefill(const PrefillParams& prm, hipStream_t stream) {
    constexpr int BM = 4 * QT * 32;
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + BM - 1) / BM;
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_fwd_kernel<T, D, QT, CAUSAL>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    return check_launch("prefill_fwd_kernel");
}

template <typename T>
static int dispatch_prefill(const PrefillParams& p, int D, bool causal, hipStream_t stream) {
    if (D == 128) {
        return causal ? launch_prefill<T, 128, 1, true>(p, stream) : launch_prefill<T, 128, 1, false>(p, stream);
    }
    if (D == 64) {
        return causal ? launch_prefill<T, 64, 1, true>(p, stream) : launch_prefill<T, 64, 1, false>(p, stream);
    }
    return fail(DTATTN_ERR_UNSUPPORTED, "prefill: head dim %d not supported (64 or 128)", D);
}

int prefill_fp8(const dtattn_prefill_args* a, float c, int32_t delta, hipStream_t stream);

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
    if (a->D != a->Dv)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: D=%lld != Dv=%lld not supported", (long long)a->D,
                    (long long)a->Dv);
    // Sequence lengths up to 2^29 keep every causal index expression of the kernels in int32.
    if (a->Sq > (1 << 29) || a->Sk > (1 << 29) || a->B * a->Hq > 0x3fffffff)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: sequence length exceeds 2^29");
    if (a->B == 0 || a->Sq == 0) return DTATTN_OK;
    if (a->q == nullptr || a->o == nullptr || (a->Sk > 0 && (a->k == nullptr || a->v == nullptr)))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill: null tensor pointer");
    const int64_t* strides[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
    const int esz_in = a->dtype == DTATTN_FP8_E4M3FN ? 1 : 2;
    for (int i = 0; i < 4; ++i) {
        const int esz = i == 3 ? 2 : esz_in;
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
    const float scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)a->D);
    const float c = scale * kLog2e;
    int64_t delta64 = a->q_offset - a->k_offset;
    const int64_t lim = a->Sq + a->Sk + 1;
    if (delta64 > lim) delta64 = lim;
    if (delta64 < -lim) delta64 = -lim;
    const int32_t delta = (int32_t)delta64;

    if (a->dtype == DTATTN_FP8_E4M3FN) {
        if (a->o_dtype != DTATTN_BF16) return fail(DTATTN_ERR_UNSUPPORTED, "prefill fp8: output must be bf16");
        if (a->q_descale == nullptr || a->k_descale == nullptr || a->v_descale == nullptr)
            return fail(DTATTN_ERR_INVALID_ARGUMENT, "prefill fp8: descale pointers are required");
        return prefill_fp8(a, c, delta, stream);
    }
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16)
        return fail(DTATTN_ERR_UNSUPPORTED, "prefill: dtype %d not supported (bf16, fp16, fp8_e4m3fn)", a->dtype);
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
    const int D = (int)a->D;
    const bool causal = a->causal != 0;
    if (a->dtype == DTATTN_BF16) return dispatch_prefill<bf16_t>(p, D, causal, stream);
    return dispatch_prefill<f16_t>(p, D, causal, stream);
}
