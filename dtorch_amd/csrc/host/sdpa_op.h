// Host-side operators of the MI355X attention path, mirroring DTorch's operator contract.
//
// The reference's SdpaOp (dtorch/core/operators/standard/scaled_dot_product_attention_op.h:14-52)
// exposes InferOutputMetaInfo / GetPlacementSignature / GetOperatorCost / Compute, with
// Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) pushing freshly allocated
// outputs.  The classes here keep those names, argument meanings and error behaviour
// (std::invalid_argument on bad input, as Kernel::Run expects: dtorch/core/kernel/kernel.cc:140-148),
// and route the arithmetic through the dtattn C ABI on the thread's current HIP stream.
//
// New operators (no reference counterpart; registered the same way an operator is added to DTorch):
//   SdpaWithLseOp  -> {O, LSE}, with explicit causal offsets for ring blocks
//   SdpaDecodeOp   -> {O, LSE} for one query token per sequence against a padded KV cache
//   SdpaDecodePagedOp -> the same against a paged KV cache (page pool + block table)
//   LseMergeOp     -> {O, LSE} from n (O_b, LSE_b) pairs
//   Fp8QuantizeOp  -> {codes, descale}, per-head absmax e4m3fn
#pragma once

#include <torch/torch.h>

#include <optional>
#include <string>
#include <vector>

#include "param_archive.h"

namespace dtorch_amd {
namespace core {

// dtorch/external/torch/torch_util.h:107-108
using TorchTensorOptArray = std::vector<std::optional<::torch::Tensor>>;
using TorchTensorArray = std::vector<::torch::Tensor>;

// dtorch/api/cpp/functional/functional_option.h:19-30, plus the native fp8 selector.
// sageAttentionType: "" (native bf16/fp16), "native_fp8" (per-head e4m3fn on fp8 MFMA), or one of the
// reference's third-party SageAttention values ("auto", "qk_int8_pv_fp8", "qk_int8_pv_fp16"), which
// this build does not ship and rejects.
struct SdpaOption {
    std::string sageAttentionType;
    SdpaOption() : sageAttentionType("") {}
    explicit SdpaOption(std::string t) : sageAttentionType(std::move(t)) {}

    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar & sageAttentionType;
    }
};

// Operator params.  Each is default-constructible and serialises its fields in declaration order
// through a boost-style `serialize` member, as the reference's params do
// (dtorch/core/operators/operator_param.h:19-69 registers the types, operator_serialization_pack.h:91-140
// dispatches them).  In a DTorch tree each derives from OpParam and serialises
// `BaseObject<OpParam>(*this)` first; the fields after that are exactly the ones below.

// dtorch/core/operators/standard/scaled_dot_product_attention_op.h:14-36 (same fields, same defaults,
// same serialisation order).
struct SdpaParam {
    bool isCausal = false;
    std::optional<double> scale = std::nullopt;
    bool enableGqa = false;
    std::optional<SdpaOption> option = std::nullopt;

    SdpaParam() = default;
    SdpaParam(bool isCausal_, std::optional<double> scale_, bool enableGqa_, std::optional<SdpaOption> option_)
        : isCausal(isCausal_), scale(scale_), enableGqa(enableGqa_), option(std::move(option_)) {}

    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar & isCausal;
        ar & scale;
        ar & enableGqa;
        ar & option;
    }
};

// SdpaWithLse: the SdpaParam fields, then the causal offsets of a ring block (key j is visible to
// query i iff j + kOffset <= i + qOffset).  New operator type; no reference counterpart.
struct SdpaWithLseParam : SdpaParam {
    int64_t qOffset = 0;
    int64_t kOffset = 0;

    SdpaWithLseParam() = default;
    SdpaWithLseParam(SdpaParam base, int64_t qOffset_, int64_t kOffset_)
        : SdpaParam(std::move(base)), qOffset(qOffset_), kOffset(kOffset_) {}

    template <class Archive>
    void serialize(Archive& ar, const unsigned int version) {
        SdpaParam::serialize(ar, version);
        ar & qOffset;
        ar & kOffset;
    }
};

// SdpaDecode / SdpaDecodePaged: softmax scale (none: 1/sqrt(D)) and tokens per split (0: automatic).
struct SdpaDecodeParam {
    std::optional<double> scale = std::nullopt;
    int32_t chunk = 0;

    SdpaDecodeParam() = default;
    SdpaDecodeParam(std::optional<double> scale_, int32_t chunk_) : scale(scale_), chunk(chunk_) {}

    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar & scale;
        ar & chunk;
    }
};
struct SdpaDecodePagedParam : SdpaDecodeParam {
    using SdpaDecodeParam::SdpaDecodeParam;
    SdpaDecodePagedParam() = default;
};

// LseMerge: output element type as a dtattn_dtype code (BF16 0, FP16 1, FP32 3); none keeps the
// blocks' type.
struct LseMergeParam {
    std::optional<int32_t> outKind = std::nullopt;

    LseMergeParam() = default;
    explicit LseMergeParam(std::optional<int32_t> outKind_) : outKind(outKind_) {}

    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar & outKind;
    }
};

// Operators without knobs still get a param type, as every DTorch operator does.
struct KvCacheAppendParam {
    template <class Archive>
    void serialize(Archive&, const unsigned int) {}
};
struct KvCacheAppendPagedParam : KvCacheAppendParam {};
struct Fp8QuantizeParam : KvCacheAppendParam {};

// One allowed input->output placement assignment for one mesh dimension.  Placements are written
// "S(i)" (shard on tensor dim i), "R" (replicate); an empty string in `inputs` marks an optional input.
struct PlacementRule {
    std::vector<std::string> inputs;
    std::vector<std::string> outputs;
    std::vector<bool> optional;
};
using PlacementSignature = std::vector<PlacementRule>;

using Shape = std::vector<int64_t>;

class SdpaOp {
public:
    explicit SdpaOp(SdpaParam param) : mParam(std::move(param)) {}
    virtual ~SdpaOp() = default;

    const SdpaParam& Param() const { return mParam; }

    // scaled_dot_product_attention_op.cc:16-32: q's shape with the last axis replaced by v's.
    Shape InferOutputMetaInfo(const Shape& q, const Shape& k, const Shape& v) const;
    // scaled_dot_product_attention_op.cc:34-66 plus the all-Replicate rule of
    // placement_signature.cc:65-88.
    PlacementSignature GetPlacementSignature(size_t numAxis) const;
    // Output placements for one mesh dimension, or an exception when no rule matches.  `inputs`
    // holds q, k, v, mask placements ("" for an absent mask).
    std::vector<std::string> MatchPlacements(size_t numAxis, const std::vector<std::string>& inputs) const;
    // scaled_dot_product_attention_op.cc:68-95: 2 * batch * qHeads * seqQ * seqKv * (headDim + Ev).
    int64_t GetOperatorCost(const Shape& q, const Shape& k, const Shape& v) const;
    // Useful FLOPs (causal counts only visible pairs, diagonal included); used for roofline figures.
    int64_t GetAlgorithmicFlops(const Shape& q, const Shape& k, const Shape& v) const;

    // inputs = {q, k, v, attn_mask?}; pushes O.
    virtual void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;

protected:
    SdpaParam mParam;
};

// {q, k, v, attn_mask?} -> {O, LSE[B, Hq, Sq] fp32}; key j visible to query i iff
// j + kOffset <= i + qOffset when causal.
class SdpaWithLseOp : public SdpaOp {
public:
    explicit SdpaWithLseOp(SdpaWithLseParam param) : SdpaOp(param), mLseParam(std::move(param)) {}
    SdpaWithLseOp(SdpaParam param, int64_t qOffset, int64_t kOffset)
        : SdpaWithLseOp(SdpaWithLseParam(std::move(param), qOffset, kOffset)) {}
    const SdpaWithLseParam& LseParam() const { return mLseParam; }
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const override;

private:
    SdpaWithLseParam mLseParam;
};

// {q[B,Hq,1,D], k_cache[B,Hkv,S,D], v_cache[B,Hkv,S,D], lengths[B] int32} -> {O[B,Hq,1,D], LSE[B,Hq]}
class SdpaDecodeOp {
public:
    explicit SdpaDecodeOp(SdpaDecodeParam param) : mParam(std::move(param)) {}
    SdpaDecodeOp(std::optional<double> scale, int32_t chunk) : mParam(scale, chunk) {}
    const SdpaDecodeParam& Param() const { return mParam; }
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;

private:
    SdpaDecodeParam mParam;
};

// {q[B,Hq,1,D], k_pages[P,Hkv,page,D], v_pages[P,Hkv,page,D], block_table[B,max_pages] int32,
//  lengths[B] int32} -> {O[B,Hq,1,D], LSE[B,Hq]}.  The page pools may be any 4-D view whose axes are
// (page, kv head, row within the page, D) with a unit D stride (e.g. a permuted [P,page,Hkv,D] pool).
class SdpaDecodePagedOp {
public:
    explicit SdpaDecodePagedOp(SdpaDecodePagedParam param) : mParam(std::move(param)) {}
    SdpaDecodePagedOp(std::optional<double> scale, int32_t chunk) : mParam(scale, chunk) {}
    const SdpaDecodePagedParam& Param() const { return mParam; }
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;

private:
    SdpaDecodePagedParam mParam;
};

// KV-cache append (no counterpart in the reference: its Llama port keeps no cache,
// python/dtorch/test/modules/llama.py:126-156).  {k_cache, v_cache, lengths, k_new, v_new} ->
// {k_cache, v_cache, lengths}, all three updated in place: token j of sequence b lands at position
// lengths[b] + j (dropped at or past S_max), then lengths[b] += n_new, saturating at S_max.
class KvCacheAppendOp {
public:
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;
};

// The same for the paged cache of SdpaDecodePagedOp: {k_pages, v_pages, block_table, lengths, k_new,
// v_new} -> {k_pages, v_pages, lengths}; the block table must already name the pages being written.
class KvCacheAppendPagedOp {
public:
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;
};

// {O_0, LSE_0, O_1, LSE_1, ...} -> {O, LSE}; O in `outDtype` (default: the blocks' dtype).
class LseMergeOp {
public:
    explicit LseMergeOp(LseMergeParam param = LseMergeParam()) : mParam(std::move(param)) {}
    // Convenience: the output type as a torch dtype (bf16, fp16 or fp32).
    static LseMergeParam ParamFor(std::optional<c10::ScalarType> outDtype);
    const LseMergeParam& Param() const { return mParam; }
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;

private:
    LseMergeParam mParam;
};

// {x[B,H,S,D]} -> {codes[B,H,S,D] float8_e4m3fn, descale[B,H] fp32}
class Fp8QuantizeOp {
public:
    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const;
};

// How the host operators hand a tensor to the kernels: leading axes folded into one batch axis,
// element strides of (batch, H, S) and whether a layout copy was needed first.  Exposed for tests.
struct FoldedView {
    int64_t B, H, S, D;
    int64_t sb, sh, ss;
    bool copied;
};
FoldedView FoldedStrides(const at::Tensor& t);

// MI355X peak table of the current device (native analog of DevicePeakPerformance).
struct DevicePeaks {
    int cuCount;
    double clockHz, bf16Flops, fp8Flops, hbmBytesPerS;
    std::string arch;
};
DevicePeaks GetDevicePeaks(int device);

}  // namespace core
}  // namespace dtorch_amd
