// Split-KV single-token decode for gfx950.
//
// Semantics: for each sequence b, O_b = softmax(scale * q_b K_b[:L_b]^T) V_b[:L_b] with GQA
// (query head h reads kv head h / (Hq/Hkv)); i.e. SdpaOp::Compute's arithmetic
// (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109) at Lq = 1,
// is_causal = False, over the true length.  The reference has no KV cache or decode op.
//
// Kernel 1 (decode_kernel): a workgroup owns (b, kv head, chunk of C tokens, head subgroup of G query
// heads); the G heads share every K/V byte read.  A token row (D * 2 bytes) is read by D/8 lanes with
// 16-byte buffer loads (whole rows per load instruction; rows past L_b read zeros without touching
// memory).  Scores: v_dot2_f32 chain + a DPP row sum; online softmax per wave; P V with v_dot2 over
// token pairs (P rounded to the element type, as the prefill's PV MFMA does); the 4 waves combine
// through LDS and write a partial (O, LSE) per chunk -- or the final output when the sequence is a
// single chunk.
// Kernel 2 (decode_merge_kernel): one wave per (b, query head) merges the ceil(L_b / C) partials by
// LSE.  (Merging inside kernel 1 by the last workgroup needs device-scope fences; on gfx950 each one
// writes back and invalidates the XCD's L2, which costs far more than the second launch.)
#include <mutex>

#include "dtattn_common.hpp"

namespace dtattn {

struct DecodeParams {
    const void* q;
    const void* k;
    const void* v;
    const int32_t* lengths;
    void* o;
    float* lse;
    float* part_o;    // [B, Hq, nsplit, D]
    float* part_lse;  // [B, Hq, nsplit]
    int64_t qs_b, qs_h;
    int64_t ks_b, ks_h, ks_s;
    int64_t vs_b, vs_h, vs_s;
    int64_t os_b, os_h;
    int64_t lses_b;
    int32_t B, Hq, Hkv, S_max, group;
    int32_t chunk, nsplit;
    float c;  // scale * log2(e)
    // paged cache: token t of sequence b is row t & (2^page_shift - 1) of page
    // block_table[b * bt_s + (t >> page_shift)]; ks_b / vs_b are then the page strides
    const int32_t* block_table;
    int64_t bt_s;
    int32_t page_shift, num_pages;
    // bytes from a kv head's base to the end of its last page row (K, V), when every page offset fits 32 bits
    // (strides >= 0, span < 2^32): the paged loads then go through buffer resources; 0: 64-bit flat loads
    uint32_t kspan, vspan;
    // real head dim (<= the kernel's D; a multiple of 16 bytes of elements) and its 16-byte chunks
    int32_t d_real, d_ch;
    uint32_t q_and, q_xor;  // applied to q's words at load, as in ScalePlan
};

constexpr int kDecodeChunk = 128;  // smallest split; workspace queries with chunk 0 size for it

// Split length picked for chunk = 0: 128 tokens for the 8-head workgroups (8 heads per workgroup
// leave no registers for longer splits: 3.0 TB/s at 128 against 2.1-2.3 TB/s at 256); 384 for
// 16-bit rows (each wave then keeps 1.5x the K/V bytes in flight of a 256-token split, using the
// registers that 2 waves per SIMD leave free); 256 for fp32 rows.  Measured on one MI355X over batch
// 1-128, contexts 2K-128K, 4 heads per workgroup: 384 was 1-8% faster than 256 at D = 64 and 128
// everywhere except one 8K sequence (-1 to -2%); 256 had been best or within 2% of 128 and 512.
static int32_t auto_chunk(int64_t Hq, int64_t Hkv, int64_t esz) {
    if ((Hq / Hkv) % 8 == 0 && Hkv % 8 != 0) return 128;
    return esz == 2 ? 384 : 256;
}

// Kernel head dim for a real head dim: 64 or 128 (0: unsupported).  Smaller real dims run the
// kernel of the next size, reading a valid chunk in place of each padded one with its query chunk
// zeroed, so the padding adds nothing to the scores; the padded output columns are not stored.
static int decode_kernel_dim(int64_t D) { return D <= 0 ? 0 : D <= 64 ? 64 : D <= 128 ? 128 : 0; }

size_t decode_ws_parts(int64_t B, int64_t Hq, int64_t S_max, int64_t D_real, int32_t chunk, int64_t* nsplit_out) {
    const int64_t D = decode_kernel_dim(D_real) > 0 ? decode_kernel_dim(D_real) : D_real;  // partials are kernel-wide
    const int64_t nsplit = (S_max + chunk - 1) / chunk;
    if (nsplit_out) *nsplit_out = nsplit;
    const size_t o_bytes = (size_t)B * Hq * nsplit * D * sizeof(float);
    const size_t lse_bytes = (size_t)B * Hq * nsplit * sizeof(float);
    return ((o_bytes + 255) & ~(size_t)255) + ((lse_bytes + 255) & ~(size_t)255);
}

// G heads per workgroup, D head dim, TPW tokens per wave (chunk = 4 * TPW, in sub-blocks per wave;
// all trip counts are compile-time so each sub-block's loads issue together).
// PAGED: 0, rows of a contiguous cache through a buffer resource over the chunk's rows; 1, rows of a paged
// cache through the block table, with 64-bit loads of clamped token indices; 2, the same through a buffer
// resource over the kv head's pages with 32-bit offsets, when they fit (DecodeParams::kspan); 3, 4 and 5, as
// 2 for 16-, 32- and larger pages of 16-bit rows, with each wave's page ids in scalar registers (loaded with
// lengths[b]);
// otherwise through a buffer resource over the chunk's rows.
// The sub-block loop of one fp32 instantiation (three 32-token sub-blocks per wave) is too large to
// unroll fully and stays a loop; each iteration still issues its sub-block's loads together.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
template <typename T, int D, int G, int TPW, int PAGED>
__global__ void __launch_bounds__(256) decode_kernel(const DecodeParams p) {
    constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk: 8 (bf16, fp16) or 4 (fp32)
    constexpr int LPT = D / EPC;          // lanes per token row
    constexpr int TPI = 64 / LPT;         // tokens per wave-wide load
    // Sub-blocks of at most 64 tokens and 16 K + 16 V loads per lane; 96-token waves (384-token
    // splits) of 16-bit rows take one sub-block of 96 (24 + 24 loads per lane at D = 128), fp32 rows
    // three of 32.
    constexpr int SBMAX = TPW == 96 ? (EPC == 8 ? 96 : 32) : (16 * TPI < 64 ? 16 * TPI : 64);
    constexpr int SB = TPW < SBMAX ? TPW : SBMAX;
    constexpr int NSB = TPW / SB;         // sub-blocks per wave
    constexpr int NI = SB / TPI;          // K (and V) loads per lane per sub-block
    constexpr int C = 4 * TPW;
    static_assert(NI >= 2 && NI % 2 == 0 && TPW % SB == 0, "bad chunk");
    __shared__ float red_o[4][G][D];
    __shared__ float red_m[4][G];
    __shared__ float red_l[4][G];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int split = blockIdx.z;
    const int hk = blockIdx.x % p.Hkv;
    const int sg = blockIdx.x / p.Hkv;   // head subgroup within the kv group
    const int b = blockIdx.y;
    const int t0 = split * C;
    // PAGED >= 3 (16-bit rows): the wave's page ids are scalar loads issued together with lengths[b] (the
    // empty asm keeps the compiler from sinking them past the exits below), so the cache loads follow
    // lengths by one round trip, as in the contiguous kernel, instead of two.  16- and 32-token pages
    // (3, 4): a wave's tokens are whole pages.  Pages of 64 tokens or more (5): a wave's tokens start
    // anywhere in a page and span at most 3 of them.
    constexpr int PSH = PAGED == 4 ? 5 : 4;  // log2 of the page size (3, 4)
    constexpr int NPW = PAGED == 5 ? 3 : (PAGED >= 3 ? TPW >> PSH : 1);
    static_assert(PAGED < 3 || PAGED == 5 || (TPW % (1 << PSH) == 0 && (1 << PSH) % TPI == 0), "whole pages per wave");
    static_assert(PAGED != 5 || (TPW <= 128 && 64 % TPI == 0), "a wave spans at most 3 pages of 64+ tokens");
    const int sh = PAGED == 5 ? p.page_shift : PSH;
    const int wbase = t0 + __builtin_amdgcn_readfirstlane(tid >> 6) * TPW;  // the wave's first token
    int pgw[NPW];
    int Lraw;
    if constexpr (PAGED >= 3) {
        typedef const __attribute__((address_space(4))) int32_t cint32;
        const int pb = wbase >> sh;
        const int plast = (p.S_max >> sh) - 1;  // the table row holds S_max / page_size pages
        cint32* btc = (cint32*)(p.block_table + (int64_t)b * p.bt_s);
#pragma unroll
        for (int j = 0; j < NPW; ++j) pgw[j] = btc[min(pb + j, plast)];
        Lraw = p.lengths[b];
#pragma unroll
        for (int j = 0; j < NPW; ++j) asm volatile("" : "+s"(Lraw) : "s"(pgw[j]));
    } else {
        Lraw = p.lengths[b];
    }
    const int L = min(max(Lraw, 0), p.S_max);  // never read past the cache
    const int ns = (L + C - 1) / C;      // chunks of this sequence
    const int hq0 = hk * p.group + sg * G;
    T* obase = reinterpret_cast<T*>(p.o) + b * p.os_b;
    if (L == 0) {  // empty sequence: O = 0, LSE = -inf
        if (split == 0)
            for (int idx = tid; idx < G * D; idx += 256) {
                if (idx % D < p.d_real) obase[(hq0 + idx / D) * p.os_h + idx % D] = Elem<T>::from_f32(0.f);
                if (p.lse != nullptr && idx % D == 0) p.lse[b * p.lses_b + hq0 + idx / D] = kNegInf;
            }
        return;
    }
    if (t0 >= L) return;
    const int n_tok = min(C, L - t0);
    const int c8r = lane % LPT;          // 16-byte chunk of the row this lane covers
    const bool cvalid = c8r < p.d_ch;    // false only for a padded head dim
    const int c8 = cvalid ? c8r : 0;     // the chunk it reads: a valid one (its query chunk is zero)
    const int tsub = lane / LPT;

    u32x4 qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        qv[g] = q_bits(ld16(reinterpret_cast<const T*>(p.q) + b * p.qs_b + (hq0 + g) * p.qs_h + c8 * EPC), p.q_and, p.q_xor);
        if (!cvalid) qv[g] = u32x4{0u, 0u, 0u, 0u};
    }

    const int kpitch = (int)(p.ks_s * (int64_t)sizeof(T));
    const int vpitch = (int)(p.vs_s * (int64_t)sizeof(T));
    const int64_t kbo = PAGED ? 0 : b * p.ks_b + (int64_t)t0 * p.ks_s;
    const int64_t vbo = PAGED ? 0 : b * p.vs_b + (int64_t)t0 * p.vs_s;
    const T* kp = reinterpret_cast<const T*>(p.k) + hk * p.ks_h + kbo;
    const T* vp = reinterpret_cast<const T*>(p.v) + hk * p.vs_h + vbo;
    // the resources end where the chunk's last valid row ends (at the real head dim)
    const auto krs = make_rsrc(kp, (uint32_t)((n_tok - 1) * kpitch + p.d_real * (int)sizeof(T)));
    const auto vrs = make_rsrc(vp, (uint32_t)((n_tok - 1) * vpitch + p.d_real * (int)sizeof(T)));
    const int32_t* bt = PAGED ? p.block_table + b * p.bt_s : nullptr;

    float m[G], l[G], acc[G][EPC];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = kNegInf;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] = 0.f;
    }

#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
        u32x4 kr[NI], vr[NI];
        if constexpr (PAGED >= 3) {
            // Load i covers tokens wbase + sb*SB + i*TPI + tsub, which lie in one page: the wave's page
            // (sb*SB + i*TPI) / page_size (3, 4), or the one of 3 its token index names (5).  Pages past the
            // sequence end hold any id: clamped to the pool, their rows are read but get score -inf and
            // V = 0 below.
            const auto kprs = make_rsrc(kp, p.kspan);
            const auto vprs = make_rsrc(vp, p.vspan);
            const uint32_t kpb = (uint32_t)(p.ks_b * sizeof(T)), kps = (uint32_t)(p.ks_s * sizeof(T));
            const uint32_t vpb = (uint32_t)(p.vs_b * sizeof(T)), vps = (uint32_t)(p.vs_s * sizeof(T));
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                int page_id, rowi;
                if constexpr (PAGED == 5) {
                    const int tok = wbase + sb * SB + i * TPI;  // wave-uniform
                    const int j = (tok >> sh) - (wbase >> sh);
                    page_id = j == 0 ? pgw[0] : (j == 1 ? pgw[1] : pgw[2]);
                    rowi = (tok & ((1 << sh) - 1)) + tsub;
                } else {
                    page_id = pgw[(sb * SB + i * TPI) >> PSH];
                    rowi = (sb * SB + i * TPI + tsub) & ((1 << PSH) - 1);
                }
                const uint32_t pg = (uint32_t)min(max(page_id, 0), p.num_pages - 1);
                const uint32_t row = (uint32_t)rowi;
                kr[i] = buf_ld16_nt(kprs, pg * kpb + row * kps + (uint32_t)c8 * 16u);
                vr[i] = buf_ld16_nt(vprs, pg * vpb + row * vps + (uint32_t)c8 * 16u);
            }
        } else if constexpr (PAGED) {
            // Token indices past the sequence end are clamped to its last token (L >= 1 here), so every
            // block-table and cache load is unconditional and a sub-block's loads issue together; those
            // rows get score -inf below and P = 0.  Rows at or past lengths[b] are never read.
            int pg[NI], tr[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                tr[i] = min(t0 + wave * TPW + sb * SB + i * TPI + tsub, L - 1);
                pg[i] = min(max(bt[tr[i] >> p.page_shift], 0), p.num_pages - 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            const int rmask = (1 << p.page_shift) - 1;
            if constexpr (PAGED == 2) {
                // 32-bit byte offsets into a resource over the head's pages: fewer address registers and
                // instructions than 64-bit flat addresses (measured 4% faster on 16-token pages)
                const auto kprs = make_rsrc(kp, p.kspan);
                const auto vprs = make_rsrc(vp, p.vspan);
                const uint32_t kpb = (uint32_t)(p.ks_b * sizeof(T)), kps = (uint32_t)(p.ks_s * sizeof(T));
                const uint32_t vpb = (uint32_t)(p.vs_b * sizeof(T)), vps = (uint32_t)(p.vs_s * sizeof(T));
#pragma unroll
                for (int i = 0; i < NI; ++i) {  // the cache is read once per call
                    const uint32_t row = (uint32_t)(tr[i] & rmask);
                    kr[i] = buf_ld16_nt(kprs, (uint32_t)pg[i] * kpb + row * kps + (uint32_t)c8 * 16u);
                    vr[i] = buf_ld16_nt(vprs, (uint32_t)pg[i] * vpb + row * vps + (uint32_t)c8 * 16u);
                }
            } else {
#pragma unroll
                for (int i = 0; i < NI; ++i) {  // the cache is read once per call
                    kr[i] = ld16_nt(kp + pg[i] * p.ks_b + (tr[i] & rmask) * p.ks_s + c8 * EPC);
                    vr[i] = ld16_nt(vp + pg[i] * p.vs_b + (tr[i] & rmask) * p.vs_s + c8 * EPC);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int tl = wave * TPW + sb * SB + i * TPI + tsub;
                kr[i] = buf_ld16_nt(krs, (uint32_t)(tl * kpitch + c8 * 16));  // the cache is read once per call
                vr[i] = buf_ld16_nt(vrs, (uint32_t)(tl * vpitch + c8 * 16));
            }
        }
        // Every K and V load of the sub-block is in flight before the first use: left alone, the
        // scheduler issues the V loads only after the QK products, which costs a second memory
        // round trip per workgroup (measured: 4.42 -> 4.67 TB/s on the random-length batch).
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PAGED >= 3) {
            if (n_tok < C) {  // the sequence's last chunk: rows past its end hold any value
#pragma unroll
                for (int i = 0; i < NI; ++i)
                    if (wave * TPW + sb * SB + i * TPI + tsub >= n_tok) vr[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        float sc[NI][G];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const bool ok = wave * TPW + sb * SB + i * TPI + tsub < n_tok;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float a = 0.f;
                if constexpr (EPC == 8) {
                    a = Elem<T>::dot2(kr[i].x, qv[g].x, a);
                    a = Elem<T>::dot2(kr[i].y, qv[g].y, a);
                    a = Elem<T>::dot2(kr[i].z, qv[g].z, a);
                    a = Elem<T>::dot2(kr[i].w, qv[g].w, a);
                } else {
                    const f32x4 kf = __builtin_bit_cast(f32x4, kr[i]), qf = __builtin_bit_cast(f32x4, qv[g]);
                    a = __builtin_fmaf(kf.x, qf.x, a);
                    a = __builtin_fmaf(kf.y, qf.y, a);
                    a = __builtin_fmaf(kf.z, qf.z, a);
                    a = __builtin_fmaf(kf.w, qf.w, a);
                }
                a = group_sum<LPT>(a);
                sc[i][g] = ok ? a * p.c : kNegInf;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mx = kNegInf;
#pragma unroll
            for (int i = 0; i < NI; ++i) mx = fmaxf(mx, sc[i][g]);
            mx = max_across_groups<LPT>(mx);
            const float mnew = fmaxf(m[g], mx);
            const float mbase = mnew == kNegInf ? 0.f : mnew;
            const float alpha = fast_exp2(m[g] - mbase);
            m[g] = mnew;
            float ls = l[g] * alpha;
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc[g][e] *= alpha;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float pw = fast_exp2(sc[i][g] - mbase);
                sc[i][g] = pw;
                ls += pw;
            }
            l[g] = ls;
        }
        if constexpr (EPC == 8) {
            // P V over token pairs (loads i, i+1 hold tokens t, t+TPI of the same row chunk): pack
            // (v_t[e], v_t'[e]) and (p_t, p_t') as element pairs and accumulate with v_dot2.
#pragma unroll
            for (int i = 0; i < NI; i += 2) {
                uint32_t vp2[8];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    vp2[2 * w] = pack_lo_hi(vr[i][w], vr[i + 1][w], 0);
                    vp2[2 * w + 1] = pack_lo_hi(vr[i][w], vr[i + 1][w], 1);
                }
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const uint32_t pp = pack2<T>(sc[i][g], sc[i + 1][g]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[g][e] = Elem<T>::dot2(vp2[e], pp, acc[g][e]);
                }
            }
        } else {  // fp32: P and V stay fp32
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const f32x4 vf = __builtin_bit_cast(f32x4, vr[i]);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    acc[g][0] = __builtin_fmaf(sc[i][g], vf.x, acc[g][0]);
                    acc[g][1] = __builtin_fmaf(sc[i][g], vf.y, acc[g][1]);
                    acc[g][2] = __builtin_fmaf(sc[i][g], vf.z, acc[g][2]);
                    acc[g][3] = __builtin_fmaf(sc[i][g], vf.w, acc[g][3]);
                }
            }
        }
    }
    // reduce across the TPI token lanes of each row position (same c8), then across waves
#pragma unroll
    for (int g = 0; g < G; ++g) {
        l[g] = sum_across_groups<LPT>(l[g]);
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] = sum_across_groups<LPT>(acc[g][e]);
    }
    if (tsub == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPC; ++e) red_o[wave][g][c8 * EPC + e] = acc[g][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            red_m[wave][g] = m[g];
            red_l[wave][g] = l[g];
        }
    }
    __syncthreads();
    const bool single = ns == 1;  // the whole sequence is this chunk: write the final output
    for (int idx = tid; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx % D;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w][g]);
        float Lsum = 0.f, val = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = red_m[w][g] == kNegInf ? 0.f : fast_exp2(red_m[w][g] - M);
            Lsum += f * red_l[w][g];
            val += f * red_o[w][g][d];
        }
        const int hq = hq0 + g;
        if (single) {  // the whole sequence was this chunk: final output
            if (d < p.d_real) obase[hq * p.os_h + d] = Elem<T>::from_f32(val / Lsum);
            if (p.lse != nullptr && d == 0) p.lse[b * p.lses_b + hq] = (M + __log2f(Lsum)) * kLn2;
        } else {
            p.part_o[(((int64_t)b * p.Hq + hq) * p.nsplit + split) * D + d] = val / Lsum;
            if (d == 0) p.part_lse[((int64_t)b * p.Hq + hq) * p.nsplit + split] = (M + __log2f(Lsum)) * kLn2;
        }
    }
}

#pragma clang diagnostic pop

// One wave per (b, query head): merge the ceil(L_b / C) partials by LSE (sequences that fit in one
// chunk were written directly by decode_kernel).
template <typename T, int D>
__global__ void __launch_bounds__(256) decode_merge_kernel(const DecodeParams p) {
    constexpr int DPL = D / 64;  // d values per lane
    const int lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (pair >= (int64_t)p.B * p.Hq) return;
    const int b = (int)(pair / p.Hq), hq = (int)(pair % p.Hq);
    const int L = min(max(p.lengths[b], 0), p.S_max);
    const int ns = (L + p.chunk - 1) / p.chunk;
    if (ns <= 1) return;
    const float* pl = p.part_lse + pair * p.nsplit;
    const float* po = p.part_o + pair * p.nsplit * D;
    float mx = kNegInf;
    for (int s = lane; s < ns; s += 64) mx = fmaxf(mx, pl[s]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int s = lane; s < ns; s += 64) sum += __expf(pl[s] - mx);
    sum = wave_sum(sum);
    float acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
    const float inv = 1.f / sum;
    // batches of MB partials: every load of a batch is issued before the first is used, so the
    // wave waits for one memory latency per batch instead of one per partial
    constexpr int MB = 8;
    for (int s0 = 0; s0 < ns; s0 += MB) {
        float lw[MB], v[MB][DPL];
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const int s = min(s0 + j, ns - 1);  // clamped: in bounds, weight zeroed below
            lw[j] = pl[s];
#pragma unroll
            for (int e = 0; e < DPL; ++e) v[j][e] = po[(int64_t)s * D + lane * DPL + e];
        }
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const float w = s0 + j < ns ? __expf(lw[j] - mx) * inv : 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] = __builtin_fmaf(w, v[j][e], acc[e]);
        }
    }
    T* op = reinterpret_cast<T*>(p.o) + b * p.os_b + hq * p.os_h;
#pragma unroll
    for (int e = 0; e < DPL; ++e)
        if (lane * DPL + e < p.d_real) op[lane * DPL + e] = Elem<T>::from_f32(acc[e]);
    if (p.lse != nullptr && lane == 0) p.lse[b * p.lses_b + hq] = mx + __logf(sum);
}

template <typename T, int D, int G, int TPW, int PAGED>
static int launch_decode(const DecodeParams& p, hipStream_t stream) {
    // Split index slowest: workgroups dispatched together read the same chunk of many sequences (and
    // the empty chunks of short sequences gather at the end of the grid).  Measured against split
    // fastest: +4% on random lengths, +31% on equal lengths of 4428 tokens.
    dim3 grid((unsigned)(p.Hkv * (p.group / G)), (unsigned)p.B, (unsigned)p.nsplit);
    hipLaunchKernelGGL((decode_kernel<T, D, G, TPW, PAGED>), grid, dim3(256), 0, stream, p);
    int st = check_launch("decode_kernel");
    if (st != DTATTN_OK) return st;
    const int64_t pairs = (int64_t)p.B * p.Hq;
    hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, stream, p);
    return check_launch("decode_merge_kernel");
}

template <typename T, int D, int G, int PAGED>
static int dispatch_chunk(const DecodeParams& p, hipStream_t stream) {
    switch (p.chunk) {
        case 128: return launch_decode<T, D, G, 32, PAGED>(p, stream);
        case 256: return launch_decode<T, D, G, 64, PAGED>(p, stream);
        case 384: return launch_decode<T, D, G, 96, PAGED>(p, stream);
        case 512: return launch_decode<T, D, G, 128, PAGED>(p, stream);
        default: return fail(DTATTN_ERR_UNSUPPORTED, "decode: chunk %d not supported (128, 256, 384, 512)", p.chunk);
    }
}

template <typename T, int D, int PAGED>
static int dispatch_group(const DecodeParams& p, hipStream_t stream) {
    const int g = p.group;
    // Groups of 8 heads: with Hkv a multiple of 8 the two 4-head subgroups of a kv head have workgroup
    // ids 8 apart, i.e. run on the same XCD, so the second read of each chunk hits that XCD's L2 and
    // the lighter 4-head kernel takes the longer default splits of 16-bit rows (measured +5-13% at
    // Hq 64, Hkv 8); otherwise one 8-head workgroup reads the chunk once (128-token splits).
    if (g % 8 == 0 && p.Hkv % 8 != 0) return dispatch_chunk<T, D, 8, PAGED>(p, stream);
    if (g % 4 == 0) return dispatch_chunk<T, D, 4, PAGED>(p, stream);
    if (g % 2 == 0) return dispatch_chunk<T, D, 2, PAGED>(p, stream);
    return dispatch_chunk<T, D, 1, PAGED>(p, stream);
}

// D: the real head dim (a multiple of 16 bytes of elements, up to 128).
template <typename T, int PAGED>
static int dispatch_decode(DecodeParams p, int D, hipStream_t stream) {
    const int Dk = decode_kernel_dim(D);
    if (Dk == 0 || (D * (int)sizeof(T)) % 16 != 0)
        return fail(DTATTN_ERR_UNSUPPORTED, "decode: head dim %d not supported (a multiple of %d up to 128)", D,
                    16 / (int)sizeof(T));
    p.d_real = D;
    p.d_ch = D * (int)sizeof(T) / 16;
    if (Dk == 128) return dispatch_group<T, 128, PAGED>(p, stream);
    return dispatch_group<T, 64, PAGED>(p, stream);
}

}  // namespace dtattn

using namespace dtattn;

extern "C" size_t dtattn_decode_workspace_size(int64_t B, int64_t Hq, int64_t S_max, int64_t D, int32_t chunk) {
    if (chunk <= 0) chunk = kDecodeChunk;
    if (B <= 0 || Hq <= 0 || S_max <= 0 || D <= 0) return 0;
    return decode_ws_parts(B, Hq, S_max, D, chunk, nullptr);
}

namespace dtattn {
namespace {

// Scratch of the allocation-free decode entry point (dtattn_decode_splitkv_noalloc): the partial
// (O, LSE) of every split lives here instead of in a caller-provided workspace.  Each device that
// loads the library holds its own copy until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, once per device with that device current, and is cached per device.
constexpr size_t kScratchBytes = DTATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
struct ScratchTable {
    std::once_flag once[kMaxScratchDevices];
    void* ptr[kMaxScratchDevices] = {};
    hipError_t status[kMaxScratchDevices] = {};
};
ScratchTable& scratch_table() {
    static ScratchTable t;
    return t;
}

// Device address of `scratch` on the device `stream` belongs to (the current device for the null
// stream).
int scratch_address(hipStream_t stream, void** out) {
    int dev = -1;
    hipError_t e = stream == nullptr ? hipGetDevice(&dev) : hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
        return fail(DTATTN_ERR_DEVICE, "decode_noalloc: cannot tell the stream's device (%s)", hipGetErrorString(e));
    ScratchTable& t = scratch_table();
    std::call_once(t.once[dev], [&]() {
        int cur = -1;
        hipError_t r = hipGetDevice(&cur);
        if (r == hipSuccess && cur != dev) r = hipSetDevice(dev);
        void* ptr = nullptr;
        if (r == hipSuccess) r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != dev) {
            const hipError_t back = hipSetDevice(cur);
            if (r == hipSuccess) r = back;
        }
        t.status[dev] = r;
        t.ptr[dev] = r == hipSuccess ? ptr : nullptr;
    });
    if (t.status[dev] != hipSuccess || t.ptr[dev] == nullptr)
        return fail(DTATTN_ERR_DEVICE, "decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(t.status[dev]));
    *out = t.ptr[dev];
    return DTATTN_OK;
}

}  // namespace

// The split-KV decode with its partials in `ws` (at least decode_ws_parts() bytes, 256-byte aligned),
// or in `scratch` when `noalloc`.
static int decode_splitkv_run(const dtattn_decode_args* a, void* ws, size_t ws_bytes, bool noalloc,
                              hipStream_t stream) {
    if (a->B < 0 || a->Hq <= 0 || a->Hkv <= 0 || a->S_max <= 0 || a->D <= 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode: bad sizes");
    if (a->Hq % a->Hkv != 0) return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode: Hq is not a multiple of Hkv");
    if (a->B == 0) return DTATTN_OK;
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16 && a->dtype != DTATTN_FP32)
        return fail(DTATTN_ERR_UNSUPPORTED, "decode: dtype %d not supported (bf16, fp16, fp32)", a->dtype);
    const int64_t esz = a->dtype == DTATTN_FP32 ? 4 : 2;
    const int32_t chunk = a->chunk > 0 ? a->chunk : auto_chunk(a->Hq, a->Hkv, esz);
    if (chunk != 128 && chunk != 256 && chunk != 384 && chunk != 512)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode: chunk %d must be 128, 256, 384 or 512", chunk);
    // chunk rows are addressed with 32-bit byte offsets
    if (a->k_stride[2] * esz * chunk >= ((int64_t)1 << 31) || a->v_stride[2] * esz * chunk >= ((int64_t)1 << 31))
        return fail(DTATTN_ERR_UNSUPPORTED, "decode: cache row pitch too large");
    if (a->q == nullptr || a->k_cache == nullptr || a->v_cache == nullptr || a->lengths == nullptr || a->o == nullptr)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode: null pointer");
    const int64_t s_all[] = {a->q_stride[0], a->q_stride[1], a->k_stride[0], a->k_stride[1], a->k_stride[2],
                             a->v_stride[0], a->v_stride[1], a->v_stride[2]};
    for (int64_t s : s_all)
        if ((s * esz) % 16 != 0) return fail(DTATTN_ERR_UNSUPPORTED, "decode: strides must be multiples of 16 bytes");
    int64_t nsplit = 0;
    const size_t need = decode_ws_parts(a->B, a->Hq, a->S_max, a->D, chunk, &nsplit);
    if (nsplit > 65535 || a->B > 65535) return fail(DTATTN_ERR_UNSUPPORTED, "decode: grid too large");
    if (noalloc) {
        if (need > kScratchBytes)
            return fail(DTATTN_ERR_WORKSPACE,
                        "decode_noalloc: this call needs %zu bytes of scratch (B * Hq * ceil(S_max / %d) partials); "
                        "the allocation-free entry point holds %zu",
                        need, chunk, kScratchBytes);
        const int st = scratch_address(stream, &ws);
        if (st != DTATTN_OK) return st;
        ws_bytes = kScratchBytes;
    }
    if (ws == nullptr || ws_bytes < need)
        return fail(DTATTN_ERR_WORKSPACE, "decode: workspace of %zu bytes required, %zu given", need, ws_bytes);
    if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
        return fail(DTATTN_ERR_WORKSPACE, "decode: workspace must be 256-byte aligned");

    DecodeParams p;
    p.q = a->q;
    p.k = a->k_cache;
    p.v = a->v_cache;
    p.lengths = a->lengths;
    p.o = a->o;
    p.lse = a->lse;
    const size_t o_bytes = (size_t)a->B * a->Hq * nsplit * (decode_kernel_dim(a->D) > 0 ? decode_kernel_dim(a->D) : a->D) * sizeof(float);
    p.part_o = reinterpret_cast<float*>(ws);
    p.part_lse = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + ((o_bytes + 255) & ~(size_t)255));
    p.qs_b = a->q_stride[0], p.qs_h = a->q_stride[1];
    p.ks_b = a->k_stride[0], p.ks_h = a->k_stride[1], p.ks_s = a->k_stride[2];
    p.vs_b = a->v_stride[0], p.vs_h = a->v_stride[1], p.vs_s = a->v_stride[2];
    p.os_b = a->o_stride[0], p.os_h = a->o_stride[1];
    p.lses_b = a->lse ? a->lse_stride[0] : 0;
    p.B = (int32_t)a->B;
    p.Hq = (int32_t)a->Hq;
    p.Hkv = (int32_t)a->Hkv;
    p.S_max = (int32_t)a->S_max;
    p.group = (int32_t)(a->Hq / a->Hkv);
    p.chunk = chunk;
    p.nsplit = (int32_t)nsplit;
    ScalePlan sp;
    const int sst = plan_scale(a->scale, a->D, a->dtype == DTATTN_FP32 ? kSign32 : kSign16, &sp);
    if (sst != DTATTN_OK) return sst;
    p.c = sp.scale * kLog2e;
    p.q_and = sp.q_and;
    p.q_xor = sp.q_xor;
    p.block_table = nullptr;
    p.bt_s = 0;
    p.page_shift = 0;
    p.num_pages = 0;
    p.kspan = p.vspan = 0;
    if (a->dtype == DTATTN_BF16) return dispatch_decode<bf16_t, 0>(p, (int)a->D, stream);
    if (a->dtype == DTATTN_FP32) return dispatch_decode<float, 0>(p, (int)a->D, stream);
    return dispatch_decode<f16_t, 0>(p, (int)a->D, stream);
}

}  // namespace dtattn

extern "C" int dtattn_decode_splitkv(const dtattn_decode_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode: args is NULL");
    return decode_splitkv_run(a, a->workspace, a->workspace_bytes, false, reinterpret_cast<hipStream_t>(stream_));
}

extern "C" int dtattn_decode_splitkv_noalloc(const dtattn_decode_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_noalloc: args is NULL");
    return decode_splitkv_run(a, nullptr, 0, true, reinterpret_cast<hipStream_t>(stream_));
}

extern "C" size_t dtattn_decode_paged_workspace_size(int64_t B, int64_t Hq, int64_t max_pages, int64_t page_size,
                                                     int64_t D, int32_t chunk) {
    if (chunk <= 0) chunk = kDecodeChunk;
    if (B <= 0 || Hq <= 0 || max_pages <= 0 || page_size <= 0 || D <= 0) return 0;
    return decode_ws_parts(B, Hq, max_pages * page_size, D, chunk, nullptr);
}

extern "C" int dtattn_decode_paged(const dtattn_decode_paged_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_paged: args is NULL");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (a->B < 0 || a->Hq <= 0 || a->Hkv <= 0 || a->D <= 0 || a->num_pages <= 0 || a->max_pages <= 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_paged: bad sizes");
    if (a->page_size < 16 || (a->page_size & (a->page_size - 1)) != 0 || a->page_size > (1 << 20))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_paged: page_size %lld must be a power of two >= 16",
                    (long long)a->page_size);
    if (a->Hq % a->Hkv != 0) return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_paged: Hq is not a multiple of Hkv");
    const int64_t S_max = a->max_pages * a->page_size;
    if (S_max > (1 << 29) || a->num_pages > 0x7fffffff)
        return fail(DTATTN_ERR_UNSUPPORTED, "decode_paged: cache too large");
    if (a->B == 0) return DTATTN_OK;
    if (a->dtype != DTATTN_BF16 && a->dtype != DTATTN_FP16 && a->dtype != DTATTN_FP32)
        return fail(DTATTN_ERR_UNSUPPORTED, "decode_paged: dtype %d not supported (bf16, fp16, fp32)", a->dtype);
    const int64_t esz = a->dtype == DTATTN_FP32 ? 4 : 2;
    const int32_t chunk = a->chunk > 0 ? a->chunk : auto_chunk(a->Hq, a->Hkv, esz);
    if (chunk != 128 && chunk != 256 && chunk != 384 && chunk != 512)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_paged: chunk %d must be 128, 256, 384 or 512", chunk);
    if (a->q == nullptr || a->k_pages == nullptr || a->v_pages == nullptr || a->block_table == nullptr ||
        a->lengths == nullptr || a->o == nullptr)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "decode_paged: null pointer");
    const int64_t s_all[] = {a->q_stride[0], a->q_stride[1], a->k_stride[0], a->k_stride[1], a->k_stride[2],
                             a->v_stride[0], a->v_stride[1], a->v_stride[2]};
    for (int64_t s : s_all)
        if ((s * esz) % 16 != 0)
            return fail(DTATTN_ERR_UNSUPPORTED, "decode_paged: strides must be multiples of 16 bytes");
    int64_t nsplit = 0;
    const size_t need = decode_ws_parts(a->B, a->Hq, S_max, a->D, chunk, &nsplit);
    if (a->workspace == nullptr || a->workspace_bytes < need)
        return fail(DTATTN_ERR_WORKSPACE, "decode_paged: workspace of %zu bytes required, %zu given", need,
                    a->workspace_bytes);
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0)
        return fail(DTATTN_ERR_WORKSPACE, "decode_paged: workspace must be 256-byte aligned");
    if (nsplit > 65535 || a->B > 65535) return fail(DTATTN_ERR_UNSUPPORTED, "decode_paged: grid too large");

    DecodeParams p;
    p.q = a->q;
    p.k = a->k_pages;
    p.v = a->v_pages;
    p.lengths = a->lengths;
    p.o = a->o;
    p.lse = a->lse;
    const size_t o_bytes = (size_t)a->B * a->Hq * nsplit * (decode_kernel_dim(a->D) > 0 ? decode_kernel_dim(a->D) : a->D) * sizeof(float);
    p.part_o = reinterpret_cast<float*>(a->workspace);
    p.part_lse = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) + ((o_bytes + 255) & ~(size_t)255));
    p.qs_b = a->q_stride[0], p.qs_h = a->q_stride[1];
    p.ks_b = a->k_stride[0], p.ks_h = a->k_stride[1], p.ks_s = a->k_stride[2];  // page, H, row
    p.vs_b = a->v_stride[0], p.vs_h = a->v_stride[1], p.vs_s = a->v_stride[2];
    p.os_b = a->o_stride[0], p.os_h = a->o_stride[1];
    p.lses_b = a->lse ? a->lse_stride[0] : 0;
    p.B = (int32_t)a->B;
    p.Hq = (int32_t)a->Hq;
    p.Hkv = (int32_t)a->Hkv;
    p.S_max = (int32_t)S_max;
    p.group = (int32_t)(a->Hq / a->Hkv);
    p.chunk = chunk;
    p.nsplit = (int32_t)nsplit;
    ScalePlan sp;
    const int sst = plan_scale(a->scale, a->D, a->dtype == DTATTN_FP32 ? kSign32 : kSign16, &sp);
    if (sst != DTATTN_OK) return sst;
    p.c = sp.scale * kLog2e;
    p.q_and = sp.q_and;
    p.q_xor = sp.q_xor;
    p.block_table = a->block_table;
    p.bt_s = a->block_table_stride;
    p.page_shift = __builtin_ctzll((unsigned long long)a->page_size);
    p.num_pages = (int32_t)a->num_pages;
    // byte span of one kv head's pages, for 32-bit buffer offsets when it fits
    auto span = [&](const int64_t st[3]) -> uint32_t {
        if (st[0] < 0 || st[2] < 0) return 0u;
        const int64_t bytes = ((a->num_pages - 1) * st[0] + (a->page_size - 1) * st[2] + a->D) * esz;
        return bytes < ((int64_t)1 << 32) ? (uint32_t)bytes : 0u;
    };
    p.kspan = span(a->k_stride);
    p.vspan = span(a->v_stride);
    if (p.kspan == 0 || p.vspan == 0) p.kspan = p.vspan = 0;
    if (p.kspan != 0 && a->page_size == 16 && a->dtype != DTATTN_FP32) {
        if (a->dtype == DTATTN_BF16) return dispatch_decode<bf16_t, 3>(p, (int)a->D, stream);
        return dispatch_decode<f16_t, 3>(p, (int)a->D, stream);
    }
    if (p.kspan != 0 && a->page_size == 32 && a->dtype != DTATTN_FP32) {
        if (a->dtype == DTATTN_BF16) return dispatch_decode<bf16_t, 4>(p, (int)a->D, stream);
        return dispatch_decode<f16_t, 4>(p, (int)a->D, stream);
    }
    if (p.kspan != 0 && a->page_size >= 64 && a->dtype != DTATTN_FP32) {
        if (a->dtype == DTATTN_BF16) return dispatch_decode<bf16_t, 5>(p, (int)a->D, stream);
        return dispatch_decode<f16_t, 5>(p, (int)a->D, stream);
    }
    if (p.kspan != 0) {
        if (a->dtype == DTATTN_BF16) return dispatch_decode<bf16_t, 2>(p, (int)a->D, stream);
        if (a->dtype == DTATTN_FP32) return dispatch_decode<float, 2>(p, (int)a->D, stream);
        return dispatch_decode<f16_t, 2>(p, (int)a->D, stream);
    }
    if (a->dtype == DTATTN_BF16) return dispatch_decode<bf16_t, 1>(p, (int)a->D, stream);
    if (a->dtype == DTATTN_FP32) return dispatch_decode<float, 1>(p, (int)a->D, stream);
    return dispatch_decode<f16_t, 1>(p, (int)a->D, stream);
}
