/*
Attention operators of the MI355X backend beside SdpaOp: per-block attention with its log-sum-exp (the
building block of a blockwise ring), single-token decode against a KV cache, and the LSE merge of
partial blocks.  Registered as OperatorType kSdpaWithLse, kSdpaDecode and kLseMerge; each param serialises
BaseObject<OpParam> first and then its fields in declaration order, as every DTorch param does.
*/

#pragma once

#include <optional>

#include "../operator.h"

namespace dtorch {
namespace core {

// Inputs {query, key, value, attnMask?}; outputs {O, LSE}.  SdpaParam's fields in SdpaParam's order, then
// the causal offsets of a ring block: key j is visible to query i iff j + kOffset <= i + qOffset.
struct SdpaWithLseParam : public OpParam {
    bool isCausal;
    std::optional<double> scale;
    bool enableGqa;
    std::optional<SdpaOption> option;
    int64_t qOffset;
    int64_t kOffset;

public:
    SdpaWithLseParam()
        : OpParam(OperatorType::kSdpaWithLse),
          isCausal(false),
          scale(std::nullopt),
          enableGqa(false),
          option(std::nullopt),
          qOffset(0),
          kOffset(0) {}

    SdpaWithLseParam(bool isCausal, std::optional<double> scale, bool enableGqa, std::optional<SdpaOption> option,
                     int64_t qOffset, int64_t kOffset)
        : OpParam(OperatorType::kSdpaWithLse),
          isCausal(isCausal),
          scale(scale),
          enableGqa(enableGqa),
          option(option),
          qOffset(qOffset),
          kOffset(kOffset) {}

    friend Serialization;
    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar& BaseObject<OpParam>(*this);
        ar & isCausal;
        ar & scale;
        ar & enableGqa;
        ar & option;
        ar & qOffset;
        ar & kOffset;
    }
};

class SdpaWithLseOp : public Operator {
public:
    SdpaWithLseOp(std::shared_ptr<OpParam> opParamPtr) : Operator(opParamPtr) {}

    bool IsRequireInputSameDataKind() const override { return false; }

    size_t InferOutputSize() const override { return 2; }

    void InferOutputMetaInfo() const override;

    PlacementSignature GetPlacementSignature() const override;

    OperatorCost GetOperatorCost() const override;

    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const override;
};

// Inputs {query [B, Hq, 1, D], kCache [B, Hkv, S_max, D], vCache, lengths [B] int32}; outputs {O, LSE [B, Hq]}.
struct SdpaDecodeParam : public OpParam {
    std::optional<double> scale;
    int64_t chunk;  // tokens per split (0: automatic)

public:
    SdpaDecodeParam() : OpParam(OperatorType::kSdpaDecode), scale(std::nullopt), chunk(0) {}

    SdpaDecodeParam(std::optional<double> scale, int64_t chunk)
        : OpParam(OperatorType::kSdpaDecode), scale(scale), chunk(chunk) {}

    friend Serialization;
    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar& BaseObject<OpParam>(*this);
        ar & scale;
        ar & chunk;
    }
};

class SdpaDecodeOp : public Operator {
public:
    SdpaDecodeOp(std::shared_ptr<OpParam> opParamPtr) : Operator(opParamPtr) {}

    bool IsRequireInputSameDataKind() const override { return false; }

    size_t InferOutputSize() const override { return 2; }

    void InferOutputMetaInfo() const override;

    PlacementSignature GetPlacementSignature() const override;

    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const override;
};

// Inputs {O_0, LSE_0, O_1, LSE_1, ...} over the same queries; outputs {O, LSE}.
struct LseMergeParam : public OpParam {
    std::optional<DataKind> outDataKind;  // none: the blocks' data kind

public:
    LseMergeParam() : OpParam(OperatorType::kLseMerge), outDataKind(std::nullopt) {}

    explicit LseMergeParam(std::optional<DataKind> outDataKind)
        : OpParam(OperatorType::kLseMerge), outDataKind(outDataKind) {}

    friend Serialization;
    template <class Archive>
    void serialize(Archive& ar, const unsigned int /*version*/) {
        ar& BaseObject<OpParam>(*this);
        ar & outDataKind;
    }
};

class LseMergeOp : public Operator {
public:
    LseMergeOp(std::shared_ptr<OpParam> opParamPtr) : Operator(opParamPtr) {}

    bool IsRequireInputSameDataKind() const override { return false; }

    size_t InferOutputSize() const override { return 2; }

    void InferOutputMetaInfo() const override;

    PlacementSignature GetPlacementSignature() const override;

    void Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const override;
};

}  // namespace core
}  // namespace dtorch
