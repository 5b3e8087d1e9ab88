// Shared device helpers for the gfx950 attention kernels: vector types, bf16/fp16/fp8 conversions,
// MFMA wrappers and the launch-side argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dtattn.h"

namespace dtattn {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef bf16_t bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16_t bf16x4 __attribute__((ext_vector_type(4)));
typedef bf16_t bf16x2 __attribute__((ext_vector_type(2)));
typedef f16_t f16x8 __attribute__((ext_vector_type(8)));
typedef f16_t f16x4 __attribute__((ext_vector_type(4)));
typedef f16_t f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// ---- element traits -------------------------------------------------------------------------

template <typename T>
struct Elem;

template <>
struct Elem<bf16_t> {
    typedef bf16x8 vec8;
    typedef bf16x4 vec4;
    static __device__ __forceinline__ float to_f32(bf16_t x) { return static_cast<float>(x); }
    static __device__ __forceinline__ bf16_t from_f32(float x) { return static_cast<bf16_t>(x); }
    static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                               false);
    }
};

// fp32 elements (decode and append of fp32 caches): conversions only.
template <>
struct Elem<float> {
    static __device__ __forceinline__ float to_f32(float x) { return x; }
    static __device__ __forceinline__ float from_f32(float x) { return x; }
};

template <>
struct Elem<f16_t> {
    typedef f16x8 vec8;
    typedef f16x4 vec4;
    static __device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }
    static __device__ __forceinline__ f16_t from_f32(float x) { return static_cast<f16_t>(x); }
    static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
    }
};

// Unpack a 16-byte chunk of 8 elements into fp32.
template <typename T>
__device__ __forceinline__ void unpack8(u32x4 raw, float* out) {
    typedef typename Elem<T>::vec8 V;
    V v = __builtin_bit_cast(V, raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = Elem<T>::to_f32(v[i]);
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* in) {
    typedef typename Elem<T>::vec8 V;
    V v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elem<T>::from_f32(in[i]);
    return __builtin_bit_cast(u32x4, v);
}

// (low or high 16-bit half e of a) | (same half of b) << 16
__device__ __forceinline__ uint32_t pack_lo_hi(uint32_t a, uint32_t b, int e) {
    return __builtin_amdgcn_perm(b, a, e ? 0x07060302u : 0x05040100u);
}

// Two floats rounded to the element type and packed as an element pair.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    typedef T pair __attribute__((ext_vector_type(2)));
    pair v;
    v[0] = Elem<T>::from_f32(x);
    v[1] = Elem<T>::from_f32(y);
    return __builtin_bit_cast(uint32_t, v);
}

// ---- e4m3fn quantization ----------------------------------------------------------------------

// Per-head absmax scaling: the factor applied before rounding and the descale of a head whose max |x|
// is m (m = 0: both 1).
__device__ __forceinline__ float quant_inv(float m) { return m > 0.f ? 448.f / m : 1.f; }
__device__ __forceinline__ float quant_descale(float m) { return m > 0.f ? m / 448.f : 1.f; }

// Four floats times inv, saturated to +-448 and rounded to nearest even e4m3fn (v_cvt_pk_fp8_f32),
// packed in one word, first value in the low byte.  The quantizer and the attention kernel that
// quantizes its own Q both use this, so their codes are identical.
__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, float inv) {
    int packed = __builtin_amdgcn_cvt_pk_fp8_f32(fminf(fmaxf(a * inv, -448.f), 448.f),
                                                 fminf(fmaxf(b * inv, -448.f), 448.f), 0, false);
    packed = __builtin_amdgcn_cvt_pk_fp8_f32(fminf(fmaxf(c * inv, -448.f), 448.f),
                                             fminf(fmaxf(d * inv, -448.f), 448.f), packed, true);
    return (uint32_t)packed;
}

// ---- raw memory access ------------------------------------------------------------------------

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Same load with the non-temporal hint, for data read exactly once.
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Raw bits of 8 consecutive elements of type T (16 bytes, or 32 for fp32).  Loading chunks and
// unpacking them in separate steps lets a thread put all of its loads in flight before any use.
template <typename T>
struct Chunk {
    u32x4 v[sizeof(T) == 4 ? 2 : 1];
};
template <typename T, bool NT>
__device__ __forceinline__ Chunk<T> load_chunk(const T* p) {
    Chunk<T> c;
    c.v[0] = NT ? ld16_nt(p) : ld16(p);
    if constexpr (sizeof(T) == 4) c.v[1] = NT ? ld16_nt(p + 4) : ld16(p + 4);
    return c;
}
template <typename T>
__device__ __forceinline__ void unpack_chunk(const Chunk<T>& c, float* out) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 a = __builtin_bit_cast(f32x4, c.v[0]);
        const f32x4 b = __builtin_bit_cast(f32x4, c.v[1]);
        out[0] = a.x, out[1] = a.y, out[2] = a.z, out[3] = a.w;
        out[4] = b.x, out[5] = b.y, out[6] = b.z, out[7] = b.w;
    } else {
        unpack8<T>(c.v[0], out);
    }
}

// Buffer resource over `bytes` bytes from `base` (raw, stride 0).  Loads at offsets >= bytes return
// zeros instead of touching memory, which is how tile loads handle ragged tails.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// 16-byte load through a buffer resource (voffset in bytes).
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0));
}

// 16-byte load with the non-temporal hint (cache policy NT): for data streamed exactly once, such as
// a KV cache in decode, so that it does not evict reused lines from L2.
__device__ __forceinline__ u32x4 buf_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 2));
}

// 16 bytes per lane straight into LDS (lane l lands at lds + 16 * l; lds is wave-uniform).  The compiler
// tracks this form in its wait counts, and its scheduler can place the load between MFMAs.
__device__ __forceinline__ void buf_ld16_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
}

// The same load issued from inline assembly, so the compiler's wait-count pass does not track it (it
// cannot always prove that later reads of other LDS buffers do not alias the copy and would drain it with
// vmcnt(0)).  The caller owns completion: an explicit wait_vmem() plus a barrier before any wave reads the
// destination.
// m0 carries the LDS address.  The compiler reserves m0 and warns that it may not honour the clobber
// (-Winline-asm, silenced here).  No kernel holds a value of its own in m0, and none uses both forms (the
// builtin form sets m0 as well).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void buf_ld16_lds_async(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset) {
    // a flat pointer into LDS carries the LDS byte offset in its low 32 bits
    const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_addr), "v"(voffset), "s"(r)
                 : "m0");
}
#pragma clang diagnostic pop

// ---- wave helpers -----------------------------------------------------------------------------

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f(v, m));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
    return v;
}

// DPP lane exchanges within a row of 16 lanes (no LDS round trip, unlike ds_bpermute).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- lane 7-i within each half row
constexpr int kDppRowMirror = 0x140;     // lane i <- lane 15-i within the row

// Cross-row exchanges on gfx950 (VALU, no LDS round trip).  v_permlane32_swap with both operands
// equal to x returns {x[l], x[l^32]} in some order in every lane, and v_permlane16_swap returns
// {x[l], x[l^16]}; combining the pair with a commutative op is the xor-32 / xor-16 butterfly step.
__device__ __forceinline__ void pair32(float x, float& a, float& b) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = __builtin_bit_cast(float, (unsigned)r[0]);
    b = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ void pair16(float x, float& a, float& b) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = __builtin_bit_cast(float, (unsigned)r[0]);
    b = __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float max_xor32(float x) {
    float a, b;
    pair32(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor32(float x) {
    float a, b;
    pair32(x, a, b);
    return a + b;
}
__device__ __forceinline__ float max_xor16(float x) {
    float a, b;
    pair16(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor16(float x) {
    float a, b;
    pair16(x, a, b);
    return a + b;
}

// Sum over aligned groups of N lanes (N = 8, 16 or 32); every lane of the group receives the total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 8 || N == 16 || N == 32, "group of 8, 16 or 32 lanes");
    x += dpp_f<kDppQuadXor1>(x);
    x += dpp_f<kDppQuadXor2>(x);
    x += dpp_f<kDppRowHalfMirror>(x);
    if (N >= 16) x += dpp_f<kDppRowMirror>(x);
    if (N == 32) x = sum_xor16(x);
    return x;
}

// Reductions over the lanes that share lane % N (N = 8, 16 or 32), i.e. across the 64/N lane groups.
template <int N>
__device__ __forceinline__ float sum_across_groups(float x) {
    if (N == 32) return sum_xor32(x);
    if (N == 8) x += dpp_f<0x128>(x);  // row_ror:8 == lane ^ 8 within a row of 16
    return sum_xor32(sum_xor16(x));
}
template <int N>
__device__ __forceinline__ float max_across_groups(float x) {
    if (N == 32) return max_xor32(x);
    if (N == 8) x = fmaxf(x, dpp_f<0x128>(x));
    return max_xor32(max_xor16(x));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// q's 16 bytes after the call's scale plan (see ScalePlan).
__device__ __forceinline__ u32x4 q_bits(u32x4 w, uint32_t q_and, uint32_t q_xor) {
    return u32x4{(w.x & q_and) ^ q_xor, (w.y & q_and) ^ q_xor, (w.z & q_and) ^ q_xor, (w.w & q_and) ^ q_xor};
}

// Workgroup barrier for LDS producer/consumer hand-offs: waits only for this wave's LDS operations
// (lgkmcnt) before s_barrier.  __syncthreads() is a workgroup release fence, which on gfx9 also
// drains every outstanding global load (vmcnt(0)) and so would stall prefetches in flight.  The
// memory clobber keeps the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait until this wave's global loads, including direct global->LDS loads, have completed.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- workgroup placement ------------------------------------------------------------------------

// Workgroup -> (query block, batch, query head, kv head) of the prefill kernels.  Causal launches take
// the longest query blocks first.  Workgroups are dispatched round-robin over the 8 XCDs
// (blockIdx % 8), each with its own L2; with xcd_map the slices (b, kv head) are dealt to XCDs so that
// every workgroup reading a slice's K/V runs on the same XCD and the slice is fetched from HBM once per
// L2 instead of once per XCD.  xcd_map requires B * Hkv to be a multiple of 8.
struct BlockCoord {
    int qb, b, hq, hk;
};

template <bool CAUSAL>
__device__ __forceinline__ BlockCoord block_coord_at(int bid, int B, int Hq, int Hkv, int group, int n_qblocks,
                                                     int xcd_map) {
    BlockCoord r;
    if (xcd_map) {
        const int x = bid & 7, j = bid >> 3;
        const int per_rank = (B * Hkv / 8) * group;  // workgroups per query-block rank per XCD
        const int rank = j / per_rank, rem = j % per_rank;
        const int slice = (rem / group) * 8 + x;
        r.b = slice / Hkv;
        r.hk = slice % Hkv;
        r.hq = r.hk * group + rem % group;
        r.qb = CAUSAL ? (n_qblocks - 1 - rank) : rank;
    } else {
        const int bh = B * Hq;
        const int rest = bid % bh;
        r.qb = CAUSAL ? (n_qblocks - 1 - bid / bh) : (bid / bh);
        r.hq = rest % Hq;
        r.b = rest / Hq;
        r.hk = r.hq / group;
    }
    return r;
}

template <bool CAUSAL>
__device__ __forceinline__ BlockCoord block_coord(int B, int Hq, int Hkv, int group, int n_qblocks, int xcd_map) {
    return block_coord_at<CAUSAL>(blockIdx.x, B, Hq, Hkv, group, n_qblocks, xcd_map);
}

// ---- host-side status plumbing ----------------------------------------------------------------

void set_last_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---- softmax scale -------------------------------------------------------------------------------

// Sign bits of one 32-bit word of q's elements, by element width.
constexpr uint32_t kSign16 = 0x80008000u, kSign32 = 0x80000000u, kSign8 = 0x80808080u;

// The softmax scale of a call (a NaN scale selects 1/sqrt(D)), as the kernels run it: always positive.
// A negative scale runs as |scale| on negated q, zero as scale 1 on zeroed q (every logit is then the
// mask alone, or 0).  Both are exact bit operations on each 32-bit word of q: (w & q_and) ^ q_xor.
struct ScalePlan {
    float scale;
    uint32_t q_and, q_xor;
};
int plan_scale(float scale, int64_t D, uint32_t sign_bits, ScalePlan* out);

}  // namespace dtattn
