// Attention forward at head dim 512 (bf16 / fp16, non-causal, no mask, no padding), software-pipelined.
//
// The arithmetic of SdpaOp::Compute (dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:
// 107-109) for the calls prefill_wide_kernel would otherwise take at kernel head dim 512 without causal
// masking, attention mask or padded head dims: the VAE mid-block attention of the reference's diffusers
// ports, one head of 512 dimensions (python/dtorch/applications/huggingface/diffusers/models/unets/
// unet_2d_blocks.py:126-140).
//
// Same decomposition as prefill_wide_kernel: a workgroup of 4 waves owns 64 query rows, 2 row groups of 32
// rows times 2 halves of the head dims; the two waves of a row group add their partial scores through LDS.
// At one wave per SIMD the compiler's code ran each 32-key tile as a chain of dependent phases (partial
// scores, exchange, softmax, PV) with nothing overlapping, and a software-pipelined form in C++ did not fit
// its register allocator (Q was parked in accumulation registers and copied back for every MFMA).  Here the
// tile loop is one inline-asm program written out by gen_prefill_wide512.py (the build runs it): the
// partial scores of tile t+1 run on the MFMAs while the VALU finishes tile t (the partner's partial, row
// max, lazy rescale decision, P), the next tiles load one instruction per MFMA, and one barrier closes each
// tile.  O and Q live in accumulation registers.  The arithmetic is prefill_wide_kernel's element for
// element, so the two kernels return identical bits.
#include "dtattn_common.hpp"
#include "prefill_params.hpp"
#include "prefill_wide512_asm.inc"

namespace dtattn {

namespace {

typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

// 16-byte chunk swizzle of an LDS row, as prefill_wide_kernel's: chunk c of row r at c ^ wswz512(r).
__device__ __forceinline__ int wswz512(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// LDS layout (bytes): K tiles at 0 / 32768, V tiles at 65536 / 98304 (32 keys x 512 elements each), the two
// exchange slabs of partial scores at 131072 / 147456 (4 waves x 64 lanes x 16 floats each).
constexpr int kWideLds = 163840;
constexpr uint32_t kVOff = 65536, kSlabOff = 131072;

}  // namespace

template <typename T>
__global__ void __launch_bounds__(256, 1) prefill_wide512_kernel(const PrefillParams p) {
    typedef typename Elem<T>::vec4 V4;
    constexpr int D = 512, BN = 32, DH = 256, DCH = 64;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kWideLds];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave >> 1;  // row group
    const int dh = wave & 1;   // half of the head dims
    const int l32 = lane & 31;
    const int hf = lane >> 5;
    const int d0 = dh * DH;

    const BlockCoord bc = block_coord<false>(p);
    const int b = bc.b, hq = bc.hq, hk = bc.hk;
    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.qs_b + hq * p.qs_h;
    const T* kp = reinterpret_cast<const T*>(p.k) + b * p.ks_b + hk * p.ks_h;
    const T* vp = reinterpret_cast<const T*>(p.v) + b * p.vs_b + hk * p.vs_h;
    const int q0 = bc.qb * 64;
    const int wq0 = q0 + rg * 32;

    // key block of this workgroup (the whole key range unless split): tiles t0 .. nt-1 from key 0
    const int split = blockIdx.y;
    const int kb0 = split * p.kblock;
    const int kend = min(p.Sk, kb0 + p.kblock);
    const int t0 = kb0 / BN;
    const int nt = kend > kb0 ? (kend + BN - 1) / BN : t0;

    const int krow = (int)(p.ks_s * (int64_t)sizeof(T));
    const int vrow = (int)(p.vs_s * (int64_t)sizeof(T));
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;

    // K fragment of S^T k-step ks (A operand): lane (l32, hf) reads key l32, chunk 32 dh + 2 ks + hf; k-steps
    // ks and ks + 8 differ by 16 chunks (the swizzle only touches the low 4 bits)
    u32x8 ak;
#pragma unroll
    for (int q = 0; q < 8; ++q) ak[q] = sbase + (uint32_t)(l32 * 1024 + 16 * (32 * dh + ((2 * q + hf) ^ wswz512(l32))));
    // V^T fragments (ds_read_b64_tr_b16): within each 16-lane block, lane 4j+a addresses key K0+j, d-segment
    // D0+4a; d-tiles dt and dt + 4 differ by 16 chunks, k-steps by 16 keys (same swizzle)
    u32x8 av;
    {
        const int blk = lane >> 4, bl = lane & 15;
        const int tr_key = bl >> 2, tr_d = 16 * (blk & 1) + 4 * (bl & 3), tr_k4 = 4 * (blk >> 1);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k = tr_k4 + tr_key + 8 * h;
                av[2 * q + h] = sbase + kVOff +
                                (uint32_t)(k * 1024 + 16 * (32 * dh + ((4 * q + (tr_d >> 3)) ^ wswz512(k))) + 2 * (tr_d & 7));
            }
    }
    // exchange slab chunks: lane l of wave w at (64 w + l) * 64 bytes, its chunk j at 16 (j ^ ((l >> 2) & 3))
    u32x4 as, ap;
    {
        const int sxs = (lane >> 2) & 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            as[j] = sbase + kSlabOff + (uint32_t)((wave * 64 + lane) * 64 + 16 * (j ^ sxs));
            ap[j] = sbase + kSlabOff + (uint32_t)(((wave ^ 1) * 64 + lane) * 64 + 16 * (j ^ sxs));
        }
    }
    // tile loads: row r0 = 8 wave + i per instruction, lane l takes its chunk l ^ wswz512(r0)
    u32x8 dk, dv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r0 = wave * 8 + i;
        const int c = lane ^ wswz512(r0);
        dk[i] = (uint32_t)(r0 * krow + c * 16);
        dv[i] = (uint32_t)(r0 * vrow + c * 16);
    }
    const uint32_t limlane = (uint32_t)(p.Sk - 1 - 4 * hf);
    const uint32_t m0base = __builtin_amdgcn_readfirstlane(sbase + (uint32_t)(wave * 8 * 1024));

    if (nt > t0) {  // tile t0 -> K buffer 0, V buffer 0
        const int rows = min(BN, kend - t0 * BN);
        const auto krs = make_rsrc(kp + (int64_t)t0 * BN * p.ks_s, (uint32_t)((rows - 1) * krow + D * (int)sizeof(T)));
        const auto vrs = make_rsrc(vp + (int64_t)t0 * BN * p.vs_s, (uint32_t)((rows - 1) * vrow + D * (int)sizeof(T)));
#pragma unroll
        for (int i = 0; i < 8; ++i) buf_ld16_lds_async(krs, smem + (wave * 8 + i) * 1024, dk[i]);
#pragma unroll
        for (int i = 0; i < 8; ++i) buf_ld16_lds_async(vrs, smem + kVOff + (wave * 8 + i) * 1024, dv[i]);
    }
    // Q fragment of k-step ks (B operand): row wq0 + l32 (rows past Sq read row Sq-1, never stored), dims
    // d0 + 16 ks + 8 hf .. + 8, straight into accumulation registers a[128 + 4 ks]
    u32x32 QA, QB;
    {
        const T* qsrc = qp + (int64_t)min(wq0 + l32, p.Sq - 1) * p.qs_s + d0 + 8 * hf;
        asm volatile(
            "global_load_dwordx4 a[128:131], %2, off\n\tglobal_load_dwordx4 a[132:135], %2, off offset:32\n\t"
            "global_load_dwordx4 a[136:139], %2, off offset:64\n\tglobal_load_dwordx4 a[140:143], %2, off offset:96\n\t"
            "global_load_dwordx4 a[144:147], %2, off offset:128\n\tglobal_load_dwordx4 a[148:151], %2, off offset:160\n\t"
            "global_load_dwordx4 a[152:155], %2, off offset:192\n\tglobal_load_dwordx4 a[156:159], %2, off offset:224\n\t"
            "global_load_dwordx4 a[160:163], %2, off offset:256\n\tglobal_load_dwordx4 a[164:167], %2, off offset:288\n\t"
            "global_load_dwordx4 a[168:171], %2, off offset:320\n\tglobal_load_dwordx4 a[172:175], %2, off offset:352\n\t"
            "global_load_dwordx4 a[176:179], %2, off offset:384\n\tglobal_load_dwordx4 a[180:183], %2, off offset:416\n\t"
            "global_load_dwordx4 a[184:187], %2, off offset:448\n\tglobal_load_dwordx4 a[188:191], %2, off offset:480"
            : "={a[128:159]}"(QA), "={a[160:191]}"(QB)
            : "v"(qsrc)
            : "memory");
    }
    f32x32 O0, O1, O2, O3;
#pragma unroll
    for (int i = 0; i < 32; ++i) O0[i] = 0.f, O1[i] = 0.f, O2[i] = 0.f, O3[i] = 0.f;
    float mrow = kNegInf, lrow = 0.f;
    const float c = p.c;
    const uint64_t kb64 = (uint64_t)(uintptr_t)kp, vb64 = (uint64_t)(uintptr_t)vp;
    const uint32_t klo = __builtin_amdgcn_readfirstlane((uint32_t)kb64);
    const uint32_t khi = __builtin_amdgcn_readfirstlane((uint32_t)(kb64 >> 32));
    const uint32_t vlo = __builtin_amdgcn_readfirstlane((uint32_t)vb64);
    const uint32_t vhi = __builtin_amdgcn_readfirstlane((uint32_t)(vb64 >> 32));
    const int t0s = __builtin_amdgcn_readfirstlane(t0), nts = __builtin_amdgcn_readfirstlane(nt);
    const int kends = __builtin_amdgcn_readfirstlane(kend);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): Q and tile t0
    lds_barrier();
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is named as clobbered: the program sets it for its loads
    if (nt > t0) {
#define DTATTN_WIDE512_OPERANDS                                                                                 \
    : "+{a[0:31]}"(O0), "+{a[32:63]}"(O1), "+{a[64:95]}"(O2), "+{a[96:127]}"(O3), [m] "+v"(mrow), [l] "+v"(lrow) \
    : "{a[128:159]}"(QA), "{a[160:191]}"(QB), "{v[160:167]}"(ak), "{v[168:175]}"(av), "{v[176:179]}"(as),        \
      "{v[180:183]}"(ap), "{v[184:191]}"(dk), "{v[192:199]}"(dv), "{v200}"(limlane), [t0] "s"(t0s), [nt] "s"(nts),  \
      [kend] "s"(kends), [c] "s"(c), [kp] "s"(krow), [vp] "s"(vrow), [klo] "s"(klo), [khi] "s"(khi),               \
      [vlo] "s"(vlo), [vhi] "s"(vhi), [m0base] "s"(m0base)
        if constexpr (__is_same(T, f16_t)) asm volatile(DTATTN_WIDE512_PROGRAM_F16 DTATTN_WIDE512_OPERANDS : DTATTN_WIDE512_CLOBBERS);
        else asm volatile(DTATTN_WIDE512_PROGRAM_BF16 DTATTN_WIDE512_OPERANDS : DTATTN_WIDE512_CLOBBERS);
#undef DTATTN_WIDE512_OPERANDS
    }
#pragma clang diagnostic pop

    // Epilogue: row group rg stages its 32 output rows in K buffer rg (row r, 16-byte chunk c at c ^ (r % 16)),
    // each wave its half, then all threads store whole rows.  The program's last barrier has every wave past
    // its last read of the tile buffers.
    T* Os = reinterpret_cast<T*>(smem + rg * 32768);
    {
        const float l = sum_xor32(lrow);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int row = l32;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                V4 o4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 16 * (dt & 1) + 4 * i4 + e;
                    const float ov = dt < 2 ? O0[k] : dt < 4 ? O1[k] : dt < 6 ? O2[k] : O3[k];
                    o4[e] = Elem<T>::from_f32(ov * inv);
                }
                const int cc = (d0 >> 3) + dt * 4 + i4;
                *reinterpret_cast<V4*>(Os + row * D + 8 * (cc ^ (row & 15)) + 4 * hf) = o4;
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
    const T* ostage = reinterpret_cast<const T*>(smem);
#pragma unroll
    for (int it = 0; it < 64 * DCH / 256; ++it) {
        const int id = it * 256 + tid;
        const int row = id / DCH, cc = id % DCH;  // row of the workgroup's 64 (row group = row / 32)
        const int qrow = q0 + row;
        if (qrow < p.Sq) st16(op + (int64_t)qrow * p.os_s + cc * 8, ld16(ostage + row * D + 8 * (cc ^ (row & 15))));
    }
}

// Whether a call can take the pipelined kernel: a positive scale (Q is loaded untransformed), and every tile's
// byte offset from the head's first key row in 32 bits: the program computes it as one 32-bit scalar product
// (32 j) * pitch for tiles j up to two past the last.
bool prefill_wide512_fits(const PrefillParams& p) {
    const int64_t pitch = (p.ks_s > p.vs_s ? p.ks_s : p.vs_s) * 2;
    return p.q_and == 0xffffffffu && p.q_xor == 0u && p.ks_s >= 0 && p.vs_s >= 0 &&
           ((int64_t)p.Sk + 64) * pitch < ((int64_t)1 << 31);
}

template <typename T>
static int launch_wide512(const PrefillParams& prm, hipStream_t stream) {
    PrefillParams p = prm;
    p.n_qblocks = (p.Sq + 63) / 64;
    const int64_t grid = (int64_t)p.n_qblocks * p.B * p.Hq;
    if (grid == 0) return DTATTN_OK;
    if (grid > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "prefill grid too large (%lld blocks)", (long long)grid);
    hipLaunchKernelGGL((prefill_wide512_kernel<T>), dim3((unsigned)grid, (unsigned)p.nsplit), dim3(256), 0, stream, p);
    return check_launch("prefill_wide512_kernel");
}

// Entry from prefill_wide for kernel head dim 512, non-causal, no mask, no padding (prefill_wide512_fits).
int prefill_wide512(const PrefillParams& p, bool f16, hipStream_t stream) {
    return f16 ? launch_wide512<f16_t>(p, stream) : launch_wide512<bf16_t>(p, stream);
}

}  // namespace dtattn
