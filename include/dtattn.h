/*
 * dtattn — C ABI of the MI355X (gfx950) attention kernels behind DTorch's SdpaOp.
 *
 * Every entry point takes device pointers, element strides and a HIP stream passed as `void*`
 * (a hipStream_t; NULL is the null stream).  Nothing here allocates device memory, creates or
 * switches streams, or synchronises: work is enqueued on `stream` and the call returns.  The
 * functions are reentrant; the only global state is a per-device property cache and the
 * allocation-free decode's per-device scratch table, each filled once under std::call_once.  On failure they return a non-zero dtattn_status and dtattn_last_error() gives
 * a thread-local message (the C++ host op turns it into std::invalid_argument, the exception
 * SdpaOp's callers already handle: dtorch/core/kernel/kernel.cc:140-148).
 *
 * Layout is the reference's HND, [B, H, S, D], with arbitrary strides in elements for B, H and S
 * and a unit stride for D (scaled_dot_product_attention_op.cc:16-32 takes [..., H, S, E]).
 */
#ifndef DTATTN_H_
#define DTATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DTATTN_ABI_VERSION 10

/* Softmax scale fields (ABI version 8): NaN selects 1/sqrt(D) (computed in double and rounded once to
 * float, as libtorch computes its default, from ABI version 10); any finite value is used as given,
 * zero and negative included, as torch::scaled_dot_product_attention takes SdpaParam's scale
 * (scaled_dot_product_attention_op.cc:107-109); +-inf is rejected.  Up to version 7 a scale <= 0
 * selected 1/sqrt(D). */

typedef enum {
    DTATTN_OK = 0,
    DTATTN_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad shape/stride, head counts that do not divide */
    DTATTN_ERR_UNSUPPORTED = 2,      /* valid request the kernels do not implement (dtype, head dim) */
    DTATTN_ERR_WORKSPACE = 3,        /* workspace missing or smaller than dtattn_*_workspace_size() */
    DTATTN_ERR_LAUNCH = 4,           /* the HIP launch itself failed */
    DTATTN_ERR_DEVICE = 5            /* HIP device query failed */
} dtattn_status;

typedef enum {
    DTATTN_BF16 = 0,
    DTATTN_FP16 = 1,
    DTATTN_FP8_E4M3FN = 2, /* OCP e4m3fn, max 448, per-head descales */
    DTATTN_FP32 = 3
} dtattn_dtype;

/* Prefill / per-block attention: O = softmax(scale * Q K^T [causal]) V, plus the per-row LSE.
 *
 * Replaces the arithmetic of SdpaOp::Compute, i.e. the libtorch call at
 * dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109
 * (torch::scaled_dot_product_attention(q, k, v, mask, 0.0, isCausal, scale, enableGqa)), for
 * mask == nullopt or an additive mask (below).  GQA: query head h reads kv head h / (Hq / Hkv) (the op's enableGqa and the
 * Llama port's repeat_kv, python/dtorch/test/modules/llama.py:80-85).  Causal rule: key j is
 * visible to query i iff j + k_offset <= i + q_offset; (0, 0) is torch's top-left alignment, a ring
 * block uses the chunks' global offsets.  Rows that see no key get O = 0 and LSE = -inf.
 *
 * dtype: BF16 or FP16 (inputs and output, fp32 softmax and accumulation); FP32 (inputs and output,
 * every step in fp32: the fp32 matrix cores, no 16-bit rounding of P; ABI version 5); or FP8_E4M3FN
 * codes with descales and a BF16 or FP16 (ABI version 7) output.
 * Head dims: BF16/FP16 take any D and Dv that are multiples of 8 up to 512, independently (the output
 * takes v's last axis, as scaled_dot_product_attention_op.cc:26-29 does); the kernels run at 64, 128,
 * 256 or 512 and read the columns past the real dims as zeros (ABI version 6).  FP32 takes any D and
 * Dv that are multiples of 4 up to 512, independently, the same way at 64, 128, 256 or 512 (up to 128
 * from ABI version 9, up to 512 from version 10).  FP8 takes D == Dv in {64, 128}.
 */
typedef struct {
    const void* q; /* [B, Hq, Sq, D] */
    const void* k; /* [B, Hkv, Sk, D] */
    const void* v; /* [B, Hkv, Sk, Dv] */
    void* o;       /* [B, Hq, Sq, Dv], dtype `o_dtype` */
    float* lse;    /* [B, Hq, Sq] natural-log LSE, fp32; may be NULL */
    int64_t B, Hq, Hkv, Sq, Sk, D, Dv;
    int64_t q_stride[3]; /* element strides of B, H, S (D stride is 1) */
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int64_t lse_stride[2]; /* B, H (S stride is 1) */
    int32_t dtype;   /* dtattn_dtype of q, k, v */
    int32_t o_dtype; /* dtattn_dtype of o: equal to dtype, or BF16 / FP16 when dtype is FP8_E4M3FN */
    float scale;     /* softmax scale; NaN means 1/sqrt(D) (ABI version 8) */
    int32_t causal;
    int64_t q_offset, k_offset;
    const float* q_descale; /* FP8 only: [B, Hq] fp32, real = code * descale */
    const float* k_descale; /* FP8 only: [B, Hkv] */
    const float* v_descale; /* FP8 only: [B, Hkv] */
    /* Optional additive attention mask (BF16/FP16/FP32 inputs; NULL: none), the attn_mask of
     * scaled_dot_product_attention_op.cc:107-109 in float form: logits = scale * q.k + m, applied together
     * with the causal rule.  Element (b, h, i, j) is mask[b*mask_stride[0] + h*mask_stride[1] +
     * i*mask_stride[2] + j] (key stride 1; a stride of 0 broadcasts); strides are multiples of 4 and the
     * pointer is 16-byte aligned.  -inf, or any value whose m / scale overflows fp32 (the dtype-minimum
     * fill of additive masks), hides the key; a boolean mask is passed as 0 / -inf. */
    const float* mask;
    int64_t mask_stride[3];
    /* Optional workspace (ABI version 7; NULL / 0: none).  Wide heads (a kernel head dim of 256 or 512)
     * whose grid would leave CUs idle run the keys as several blocks in one launch and merge them by
     * LSE; the blocks' partial outputs live here.  Non-causal FP8 calls whose grid ends in a partly
     * empty round over the GPU's workgroup slots run that round's query blocks as key pieces, merged by
     * a second launch; their partials live here.  Non-causal BF16/FP16 calls at D = Dv = 128 whose
     * 256-row work items (groups not multiples of 4) would leave CUs idle run as equal shares of key
     * tiles per CU, the items the shares cut merged by a second launch from records kept here.
     * dtattn_prefill_workspace_size() says
     * how much a call can use; with less, the call runs unsplit (same results up to the rounding of the
     * partials). */
    void* workspace;
    size_t workspace_bytes;
} dtattn_prefill_args;

int dtattn_prefill_fwd(const dtattn_prefill_args* args, void* stream);
/* Workspace bytes dtattn_prefill_fwd can use for `args` on the current device (0 when it would not
 * split the keys); 256-byte aligned pointers expected. */
size_t dtattn_prefill_workspace_size(const dtattn_prefill_args* args);

/* Native fp8 attention from bf16/fp16 inputs (ABI version 7): the path SdpaOption
 * sageAttentionType "native_fp8" selects, superseding the quantized branch of SdpaOp::Compute that hands
 * q/k/v to the third-party SageAttention package (dtorch/external/sage_attn/sage_attn_adapter.cc:28-158,
 * which takes fp16 and bf16).  q, k and v are quantized per (b, head) to e4m3fn as
 * dtattn_fp8_quantize_per_head does (absmax scaling, round to nearest even), the attention runs on fp8
 * MFMA with fp32 accumulation, and the output has the inputs' dtype.  args: dtype BF16 or FP16, o_dtype
 * equal to it, D == Dv in {64, 128}, no mask; `workspace` of dtattn_prefill_fp8_workspace_size() bytes
 * (on the current device), 256-byte aligned: K/V codes, scales, partial maxima, then the tail split's
 * partials as for FP8 codes in dtattn_prefill_fwd (optional: a workspace that ends before them runs
 * unsplit).  Three launches: the per-head maxima of q, k and v; the K/V codes and every scale; the
 * attention, which rounds its own Q rows to e4m3 in registers (and a fourth, merging the split's pieces,
 * when the split runs). */
size_t dtattn_prefill_fp8_workspace_size(const dtattn_prefill_args* args);
int dtattn_prefill_fp8(const dtattn_prefill_args* args, void* stream);

/* Split-KV single-token decode against a padded per-sequence KV cache.
 *
 * No counterpart in the reference (it has no KV cache, python/dtorch/test/modules/llama.py:126-156);
 * defined as SdpaOp::Compute's arithmetic (scaled_dot_product_attention_op.cc:107-109) with Lq = 1,
 * is_causal = False and GQA, over keys [0, lengths[b]).  Cache rows at or past lengths[b] are never
 * read.  Each (b, kv head, chunk of `chunk` tokens) is one work item writing a partial (O, LSE)
 * into the workspace; a second kernel merges the partials by LSE.  Head dims: any multiple of 16 bytes
 * of elements up to 128 (8 for BF16/FP16, 4 for FP32; ABI version 6; the kernels run at 64 or 128).
 */
typedef struct {
    const void* q;         /* [B, Hq, 1, D] */
    const void* k_cache;   /* [B, Hkv, S_max, D] */
    const void* v_cache;   /* [B, Hkv, S_max, D] */
    const int32_t* lengths;/* [B] device int32; clamped to [0, S_max]; 0 gives O = 0, LSE = -inf */
    void* o;               /* [B, Hq, 1, D], same dtype as q */
    float* lse;            /* [B, Hq] fp32; may be NULL */
    int64_t B, Hq, Hkv, S_max, D;
    int64_t q_stride[2];   /* B, H */
    int64_t k_stride[3];   /* B, H, S */
    int64_t v_stride[3];
    int64_t o_stride[2];   /* B, H */
    int64_t lse_stride[1]; /* B (H stride is 1) */
    int32_t dtype;         /* BF16, FP16 or FP32 (FP32 from ABI version 5) */
    float scale;           /* NaN means 1/sqrt(D) (ABI version 8) */
    int32_t chunk;         /* tokens per split: 128, 256, 384 or 512; 0 picks 128 when Hq / Hkv is a
                              multiple of 8 and Hkv is not, else 384 for bf16/fp16 and 256 for
                              fp32; workspace sizes for chunk 0 cover every choice */
    void* workspace;       /* >= dtattn_decode_workspace_size(...) bytes, 256-byte aligned */
    size_t workspace_bytes;
} dtattn_decode_args;

size_t dtattn_decode_workspace_size(int64_t B, int64_t Hq, int64_t S_max, int64_t D, int32_t chunk);
int dtattn_decode_splitkv(const dtattn_decode_args* args, void* stream);

/* Allocation-free variant of dtattn_decode_splitkv.
 *
 * No counterpart in the reference.  For callers that cannot allocate device memory at call time: code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.  Same arguments,
 * kernels and results (bit-identical) as dtattn_decode_splitkv, except that `workspace` and
 * `workspace_bytes` are ignored: the split partials live in a device array of
 * DTATTN_NOALLOC_SCRATCH_BYTES that the library holds on each device it runs on until the process
 * ends (its address is looked up once per device, on the first call there).  A call whose partials
 * need more than that (dtattn_decode_workspace_size() with the call's chunk) returns
 * DTATTN_ERR_WORKSPACE.  Nothing is allocated and nothing needs clearing between calls; every call on
 * one device shares the array, so calls that overlap in time on one device (two streams, or two host
 * threads) race and must be ordered by the caller.  The first call on a device may itself be recorded
 * under HIP graph capture: the address lookup it makes is not a stream operation.
 */
#define DTATTN_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int dtattn_decode_splitkv_noalloc(const dtattn_decode_args* args, void* stream);

/* Split-KV single-token decode against a paged KV cache.
 *
 * No counterpart in the reference, whose Llama attention (python/dtorch/test/modules/llama.py:126-156)
 * keeps no KV cache and attends over the whole sequence on every call: a paged KV cache feeding the
 * decode operator.  Same arithmetic as
 * dtattn_decode_splitkv; token t of sequence b lives in page block_table[b][t / page_size] at row
 * t % page_size.  Page ids are clamped to [0, num_pages), so a corrupt block table reads wrong rows
 * but never leaves the pool.  Rows at or past lengths[b] never enter the result; with bf16/fp16 rows
 * (and a pool whose kv-head span fits 4 GB) the last chunk of a sequence may read them, and the table
 * entries past its last page, from within the pool and the table.
 */
typedef struct {
    const void* q;             /* [B, Hq, 1, D] */
    const void* k_pages;       /* page pool, e.g. [num_pages, Hkv, page_size, D] (any strides below) */
    const void* v_pages;
    const int32_t* block_table;/* [B, max_pages] device int32 */
    const int32_t* lengths;    /* [B] device int32; clamped to [0, max_pages * page_size] */
    void* o;                   /* [B, Hq, 1, D], same dtype as q */
    float* lse;                /* [B, Hq] fp32; may be NULL */
    int64_t B, Hq, Hkv, D;
    int64_t num_pages, page_size, max_pages;  /* page_size: a power of two >= 16 */
    int64_t q_stride[2];       /* B, H */
    int64_t k_stride[3];       /* page, H, row within the page */
    int64_t v_stride[3];
    int64_t o_stride[2];       /* B, H */
    int64_t lse_stride[1];     /* B (H stride is 1) */
    int64_t block_table_stride;/* elements between rows of block_table */
    int32_t dtype;             /* BF16, FP16 or FP32 (FP32 from ABI version 5) */
    float scale;               /* NaN means 1/sqrt(D) (ABI version 8) */
    int32_t chunk;             /* tokens per split: 128, 256, 384 or 512; 0 picks as dtattn_decode_args does */
    void* workspace;           /* >= dtattn_decode_paged_workspace_size(...) bytes, 256-byte aligned */
    size_t workspace_bytes;
} dtattn_decode_paged_args;

size_t dtattn_decode_paged_workspace_size(int64_t B, int64_t Hq, int64_t max_pages, int64_t page_size, int64_t D,
                                          int32_t chunk);
int dtattn_decode_paged(const dtattn_decode_paged_args* args, void* stream);

/* KV-cache append: writes the new tokens' keys and values into the cache that the decode entry points
 * read.
 *
 * No counterpart in the reference (its Llama port keeps no cache and recomputes attention over the whole
 * sequence each step, python/dtorch/test/modules/llama.py:126-156); the write side of the decode loop
 * listed as the next step for decode.  Token j (0 <= j < n_new) of sequence b goes to cache position
 * t = max(lengths[b], 0) + j; positions at or past the capacity are not written.  Afterwards, in stream
 * order, lengths[b] = min(max(lengths[b], 0) + n_new, capacity): callers that must not drop tokens check
 * the capacity on the host.  dtype BF16, FP16 or FP32 (ABI version 5) for new tokens and cache alike; a
 * token row of D elements a multiple of 16 bytes.
 */
typedef struct {
    const void* k_new;     /* [B, Hkv, n_new, D] (any strides, D stride 1) */
    const void* v_new;
    void* k_cache;         /* [B, Hkv, S_max, D]; capacity S_max */
    void* v_cache;
    int32_t* lengths;      /* [B] device int32, read and then advanced */
    int64_t B, Hkv, n_new, S_max, D;
    int64_t k_new_stride[3]; /* B, H, token */
    int64_t v_new_stride[3];
    int64_t k_stride[3];     /* B, H, S */
    int64_t v_stride[3];
    int32_t dtype;
} dtattn_kv_append_args;

int dtattn_kv_append(const dtattn_kv_append_args* args, void* stream);

/* The same for a paged cache laid out as dtattn_decode_paged reads it: position t of sequence b is row
 * t % page_size of page block_table[b][t / page_size]; capacity max_pages * page_size.  The caller assigns
 * the pages of the positions being written beforehand.  A token whose table entry is not a page of the pool
 * (below 0, e.g. an unassigned -1 slot, or at least num_pages) is dropped: nothing is written for it (the
 * decode reads clamp such ids into the pool instead, since their rows past the length are masked; a write
 * through a clamped id would land in another sequence's page), and the length advances as for a written
 * token (ABI version 9). */
typedef struct {
    const void* k_new;         /* [B, Hkv, n_new, D] (any strides, D stride 1) */
    const void* v_new;
    void* k_pages;             /* page pool, e.g. [num_pages, Hkv, page_size, D] (any strides below) */
    void* v_pages;
    const int32_t* block_table;/* [B, max_pages] device int32 */
    int32_t* lengths;          /* [B] device int32, read and then advanced */
    int64_t B, Hkv, n_new, D;
    int64_t num_pages, page_size, max_pages;  /* page_size: a power of two >= 16 */
    int64_t k_new_stride[3];
    int64_t v_new_stride[3];
    int64_t k_stride[3];       /* page, H, row within the page */
    int64_t v_stride[3];
    int64_t block_table_stride;
    int32_t dtype;
} dtattn_kv_append_paged_args;

int dtattn_kv_append_paged(const dtattn_kv_append_paged_args* args, void* stream);

/* LSE merge of n partial attention blocks over the same queries.
 *
 * No counterpart in the reference: its ring context parallelism all-gathers K/V and runs one SDPA
 * (python/dtorch/nn/scaled_dot_product_attention_with_cp.py:87-101); this is the combine step of
 * the blockwise ring.  With m = max_b LSE_b: LSE = m + log sum_b exp(LSE_b - m) and
 * O = sum_b exp(LSE_b - LSE) O_b.  Blocks with LSE = -inf contribute nothing.
 * All blocks share one shape [B, H, S, D] and one set of strides; D is a multiple of 8 (ABI version 6).
 */
#define DTATTN_MAX_MERGE_BLOCKS 16
typedef struct {
    int32_t n_blocks;                            /* 1 .. DTATTN_MAX_MERGE_BLOCKS */
    const void* o_blocks[DTATTN_MAX_MERGE_BLOCKS];   /* each [B, H, S, D] */
    const float* lse_blocks[DTATTN_MAX_MERGE_BLOCKS];/* each [B, H, S] fp32 */
    int64_t B, H, S, D;
    int64_t block_o_stride[3];  /* B, H, S */
    int64_t block_lse_stride[2];/* B, H */
    int32_t block_dtype;        /* BF16, FP16 or FP32 */
    void* o;                    /* [B, H, S, D] */
    float* lse;                 /* [B, H, S]; may be NULL */
    int64_t o_stride[3];
    int64_t lse_stride[2];
    int32_t o_dtype;            /* BF16, FP16 or FP32 */
} dtattn_merge_args;

int dtattn_lse_merge(const dtattn_merge_args* args, void* stream);

/* Per-head absmax quantization to fp8 e4m3fn (the pre-pass of the fp8 prefill).
 *
 * Supersedes the reference's SageAttention branch, which quantizes inside a third-party Python
 * package (dtorch/external/sage_attn/sage_attn_adapter.cc:28-158).  For each (b, h):
 * amax = max |x|; inv = 448 / amax; code = e4m3fn_rne(x * inv) (saturating); descale = amax / 448;
 * amax == 0 gives inv = descale = 1.  x: [B, H, S, D] BF16/FP16/FP32 with strides; x8: contiguous
 * [B, H, S, D] bytes; descale: [B, H] fp32.
 */
size_t dtattn_fp8_quantize_workspace_size(int64_t B, int64_t H, int64_t S, int64_t D);
int dtattn_fp8_quantize_per_head(const void* x, int32_t x_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                 const int64_t x_stride[3], void* x8, float* descale, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Peak table of the device (analog of dtorch/external/device/device_peak_performance.cc:125-200):
 * CU count and max engine clock from hipGetDeviceProperties times the CDNA4 per-CU dense rates
 * (bf16/fp16 4096, fp8 8192 FLOP/clk/CU), HBM3E bandwidth 8.0e12 B/s. */
typedef struct {
    int32_t cu_count;
    double clock_hz;
    double bf16_flops;
    double fp8_flops;
    double hbm_bytes_per_s;
    char arch[64];
} dtattn_device_peaks;

int dtattn_get_device_peaks(int32_t device, dtattn_device_peaks* out);

const char* dtattn_last_error(void);
int dtattn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DTATTN_H_ */
