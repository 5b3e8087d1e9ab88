// KV-cache append: the write side of the decode loop.
//
// No counterpart in the reference: its Llama port keeps no cache and recomputes attention over the
// whole sequence every step (python/dtorch/test/modules/llama.py:126-156).  Token j of sequence b of
// the new keys/values lands at cache position t = max(lengths[b], 0) + j; positions at or past the
// capacity (S_max, or max_pages * page_size for a paged cache) are not written, and neither are
// paged positions whose block-table entry is not a page of the pool (below 0 or at least num_pages).
// A second launch on the same stream then advances lengths[b] to min(max(lengths[b], 0) + n_new,
// capacity), so the copy kernel can read lengths while the update cannot race with it.
//
// HBM-bound copy: one thread per 16-byte chunk of a token row, 16-byte vector loads and stores.
#include "dtattn_common.hpp"

namespace dtattn {

struct AppendParams {
    const char* k_new;
    const char* v_new;
    char* k_dst;  // contiguous cache base, or page pool base
    char* v_dst;
    const int32_t* block_table;  // paged only
    int32_t* lengths;
    int64_t kn_b, kn_h, kn_s;  // element strides of the new tokens
    int64_t vn_b, vn_h, vn_s;
    int64_t k_b, k_h, k_s;  // cache strides: (batch | page, head, row)
    int64_t v_b, v_h, v_s;
    int64_t bt_s;
    int64_t rows;  // B * Hkv * n_new
    int32_t Hkv, n_new, cpr, esz;  // cpr: 16-byte chunks per token row
    int32_t capacity, page_shift, num_pages;
};

template <bool PAGED>
__global__ void __launch_bounds__(256) kv_append_kernel(const AppendParams p) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gid / p.cpr;
    if (row >= p.rows) return;
    const int c = (int)(gid % p.cpr);
    const int j = (int)(row % p.n_new);
    const int64_t bh = row / p.n_new;
    const int h = (int)(bh % p.Hkv);
    const int64_t b = bh / p.Hkv;
    const int t = max(p.lengths[b], 0) + j;
    if (t >= p.capacity) return;  // past the cache: not written
    const int64_t cb = (int64_t)c * 16;
    const u32x4 kv = ld16(p.k_new + (b * p.kn_b + h * p.kn_h + (int64_t)j * p.kn_s) * p.esz + cb);
    const u32x4 vv = ld16(p.v_new + (b * p.vn_b + h * p.vn_h + (int64_t)j * p.vn_s) * p.esz + cb);
    int64_t kbase, vbase;
    if constexpr (PAGED) {
        // A table entry outside [0, num_pages) names no page of the pool (an unassigned slot, or a corrupt
        // table): the token is dropped.  Clamping it into the pool, as the decode kernel does for its reads
        // (whose rows past the length are masked), would overwrite another sequence's cache.
        const int page = p.block_table[b * p.bt_s + (t >> p.page_shift)];
        if (page < 0 || page >= p.num_pages) return;
        const int r = t & ((1 << p.page_shift) - 1);
        kbase = page * p.k_b + h * p.k_h + (int64_t)r * p.k_s;
        vbase = page * p.v_b + h * p.v_h + (int64_t)r * p.v_s;
    } else {
        kbase = b * p.k_b + h * p.k_h + (int64_t)t * p.k_s;
        vbase = b * p.v_b + h * p.v_h + (int64_t)t * p.v_s;
    }
    st16(p.k_dst + kbase * p.esz + cb, kv);
    st16(p.v_dst + vbase * p.esz + cb, vv);
}

__global__ void __launch_bounds__(256) kv_lengths_kernel(int32_t* lengths, int64_t B, int32_t n_new, int32_t capacity) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b < B) lengths[b] = min(max(lengths[b], 0) + n_new, capacity);
}

static int launch_append(const AppendParams& p, int64_t B, bool paged, hipStream_t stream) {
    const int64_t threads = p.rows * p.cpr;
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "kv_append: grid too large");
    if (blocks > 0) {
        if (paged)
            hipLaunchKernelGGL(kv_append_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(kv_append_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, p);
        const int st = check_launch("kv_append_kernel");
        if (st != DTATTN_OK) return st;
    }
    hipLaunchKernelGGL(kv_lengths_kernel, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, stream, p.lengths, B,
                       p.n_new, p.capacity);
    return check_launch("kv_lengths_kernel");
}

// Shared validation of the new-token tensors and the dtype; fills the common fields of p.
static int common_append(AppendParams& p, const void* k_new, const void* v_new, int32_t* lengths, int64_t B,
                         int64_t Hkv, int64_t n_new, int64_t D, const int64_t kn[3], const int64_t vn[3],
                         const int64_t ks[3], const int64_t vs[3], int32_t dtype, const char* who) {
    if (B < 0 || Hkv <= 0 || n_new < 0 || D <= 0)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "%s: bad sizes", who);
    if (dtype != DTATTN_BF16 && dtype != DTATTN_FP16 && dtype != DTATTN_FP32)
        return fail(DTATTN_ERR_UNSUPPORTED, "%s: dtype %d not supported (bf16, fp16, fp32)", who, dtype);
    const int esz = dtype == DTATTN_FP32 ? 4 : 2;
    if ((D * esz) % 16 != 0)
        return fail(DTATTN_ERR_UNSUPPORTED, "%s: a token row of D=%lld elements is not a multiple of 16 bytes", who,
                    (long long)D);
    if (n_new > 0x3fffffff) return fail(DTATTN_ERR_UNSUPPORTED, "%s: too many new tokens", who);
    if (lengths == nullptr || (B > 0 && n_new > 0 && (k_new == nullptr || v_new == nullptr)))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "%s: null pointer", who);
    const int64_t* all[4] = {kn, vn, ks, vs};
    for (int i = 0; i < 4; ++i)
        for (int s = 0; s < 3; ++s)
            if ((all[i][s] * esz) % 16 != 0)
                return fail(DTATTN_ERR_UNSUPPORTED, "%s: strides must be multiples of 16 bytes", who);
    if ((reinterpret_cast<uintptr_t>(k_new) | reinterpret_cast<uintptr_t>(v_new)) & 15u)
        return fail(DTATTN_ERR_UNSUPPORTED, "%s: new tokens must be 16-byte aligned", who);
    p.k_new = reinterpret_cast<const char*>(k_new);
    p.v_new = reinterpret_cast<const char*>(v_new);
    p.lengths = lengths;
    p.kn_b = kn[0], p.kn_h = kn[1], p.kn_s = kn[2];
    p.vn_b = vn[0], p.vn_h = vn[1], p.vn_s = vn[2];
    p.k_b = ks[0], p.k_h = ks[1], p.k_s = ks[2];
    p.v_b = vs[0], p.v_h = vs[1], p.v_s = vs[2];
    p.rows = B * Hkv * n_new;
    p.Hkv = (int32_t)Hkv;
    p.n_new = (int32_t)n_new;
    p.cpr = (int32_t)(D * esz / 16);
    p.esz = esz;
    return DTATTN_OK;
}

}  // namespace dtattn

using namespace dtattn;

extern "C" int dtattn_kv_append(const dtattn_kv_append_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append: args is NULL");
    AppendParams p = {};
    int st = common_append(p, a->k_new, a->v_new, a->lengths, a->B, a->Hkv, a->n_new, a->D, a->k_new_stride,
                           a->v_new_stride, a->k_stride, a->v_stride, a->dtype, "kv_append");
    if (st != DTATTN_OK) return st;
    if (a->S_max <= 0 || a->S_max > (1 << 29))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append: S_max=%lld out of range", (long long)a->S_max);
    if (a->B == 0) return DTATTN_OK;
    if (a->k_cache == nullptr || a->v_cache == nullptr)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append: null cache pointer");
    if ((reinterpret_cast<uintptr_t>(a->k_cache) | reinterpret_cast<uintptr_t>(a->v_cache)) & 15u)
        return fail(DTATTN_ERR_UNSUPPORTED, "kv_append: caches must be 16-byte aligned");
    p.k_dst = reinterpret_cast<char*>(a->k_cache);
    p.v_dst = reinterpret_cast<char*>(a->v_cache);
    p.capacity = (int32_t)a->S_max;
    return launch_append(p, a->B, false, reinterpret_cast<hipStream_t>(stream_));
}

extern "C" int dtattn_kv_append_paged(const dtattn_kv_append_paged_args* a, void* stream_) {
    if (a == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append_paged: args is NULL");
    AppendParams p = {};
    int st = common_append(p, a->k_new, a->v_new, a->lengths, a->B, a->Hkv, a->n_new, a->D, a->k_new_stride,
                           a->v_new_stride, a->k_stride, a->v_stride, a->dtype, "kv_append_paged");
    if (st != DTATTN_OK) return st;
    if (a->page_size < 16 || (a->page_size & (a->page_size - 1)) != 0 || a->page_size > (1 << 20))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append_paged: page_size %lld must be a power of two >= 16",
                    (long long)a->page_size);
    if (a->num_pages <= 0 || a->max_pages <= 0 || a->num_pages > 0x7fffffff ||
        a->max_pages * a->page_size > (1 << 29))
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append_paged: bad page counts");
    if (a->B == 0) return DTATTN_OK;
    if (a->k_pages == nullptr || a->v_pages == nullptr || a->block_table == nullptr)
        return fail(DTATTN_ERR_INVALID_ARGUMENT, "kv_append_paged: null pointer");
    if ((reinterpret_cast<uintptr_t>(a->k_pages) | reinterpret_cast<uintptr_t>(a->v_pages)) & 15u)
        return fail(DTATTN_ERR_UNSUPPORTED, "kv_append_paged: page pools must be 16-byte aligned");
    p.k_dst = reinterpret_cast<char*>(a->k_pages);
    p.v_dst = reinterpret_cast<char*>(a->v_pages);
    p.block_table = a->block_table;
    p.bt_s = a->block_table_stride;
    p.capacity = (int32_t)(a->max_pages * a->page_size);
    p.page_shift = __builtin_ctzll((unsigned long long)a->page_size);
    p.num_pages = (int32_t)a->num_pages;
    return launch_append(p, a->B, true, reinterpret_cast<hipStream_t>(stream_));
}
