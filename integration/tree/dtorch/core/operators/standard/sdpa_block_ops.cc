/*
Shapes, placements, cost and compute of the MI355X attention operators (sdpa_block_ops.h).
*/

#include "sdpa_block_ops.h"

#include <stdexcept>

#include "dtorch/common/config.h"
#include "dtorch/core/operand.h"

#if DTORCH_WITH_DTATTN
#include "dtorch/external/dtattn/dtattn_adapter.h"
#endif

namespace dtorch {
namespace core {

namespace {

[[noreturn]] void NeedsBackend(const char* op) {
    throw std::invalid_argument(std::string(op) +
                                " runs on the MI355X attention kernels: build with DTORCH_WITH_DTATTN and pass "
                                "tensors on an MI355X device mesh");
}

// q's shape without its last axis: the per-row LSE of an attention output.
Shape RowShape(const Shape& q) {
    Shape s;
    for (size_t i = 0; i + 1 < q.NumAxis(); ++i) s.PushBack(q[i]);
    return s;
}

}  // namespace

//------------------------------------------------- SdpaWithLse -------------------------------------------------------

void SdpaWithLseOp::InferOutputMetaInfo() const {
    DDebugAssert(GetInputSize() == 4);
    DDebugAssert(GetOutputSize() == 2);
    const Shape& qShape = OperandA()->GetShape();
    const Shape& vShape = OperandC()->GetShape();
    DDebugAssert(qShape.NumAxis() >= 4);
    Shape outShape = qShape;
    outShape[-1] = vShape[-1];
    OperandY()->MetaDataSameAs(OperandA());
    OperandY()->SetShapeAndStride(outShape);

    Operand* lse = GetOutputOperand(1);
    lse->MetaDataSameAs(OperandA());
    lse->SetDataKind(DataKind::kFloat32);
    lse->SetShapeAndStride(RowShape(qShape));
}

// SdpaOp's rules: batch (all inputs S(0)), heads (q, k, v S(i), mask R) and the ring's query shard (q S(2), k,
// v, mask R).  The LSE drops the last axis, so it is sharded on the same axis index as O.
PlacementSignature SdpaWithLseOp::GetPlacementSignature() const {
    DDebugAssert(GetInputSize() == 4);
    const size_t numAxis = OperandA()->GetShape().NumAxis();
    PlacementSignature::Builder builder(GetInputSize(), GetOutputSize());
    builder.AddInput(Shard(0))
        .AddInput(Shard(0))
        .AddInput(Shard(0))
        .AddOptionalInput(Shard(0))
        .AddOutput(Shard(0))
        .AddOutput(Shard(0))
        .Build();
    for (size_t i = 1; i < numAxis - 2; i++) {
        builder.AddInput(Shard(i))
            .AddInput(Shard(i))
            .AddInput(Shard(i))
            .AddOptionalInput("R")
            .AddOutput(Shard(i))
            .AddOutput(Shard(i))
            .Build();
    }
    builder.AddInput(Shard(numAxis - 2))
        .AddInput("R")
        .AddInput("R")
        .AddOptionalInput("R")
        .AddOutput(Shard(numAxis - 2))
        .AddOutput(Shard(numAxis - 2))
        .Build();
    return builder.Finish();
}

// The SdpaOp formula, 2 * batch * qHeads * seqQ * seqKv * (headDim + Ev) (scaled_dot_product_attention_op.cc).
OperatorCost SdpaWithLseOp::GetOperatorCost() const {
    const Shape& qShape = OperandA()->GetShape();
    const Shape& kShape = OperandB()->GetShape();
    const Shape& vShape = OperandC()->GetShape();
    const int64_t batch = static_cast<int64_t>(qShape.Prod(0, static_cast<int>(qShape.NumAxis()) - 4));
    return OperatorCost::Compute(2 * batch * qShape[-3] * qShape[-2] * kShape[-2] * (qShape[-1] + vShape[-1]));
}

void SdpaWithLseOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    const auto& param = GetOpParam<SdpaWithLseParam>();
    DDebugAssert(inputs.size() == 4);
#if DTORCH_WITH_DTATTN
    if (external::dtattn::IsSupportedDevice(inputs[0].value())) {
        auto [o, lse] = external::dtattn::SdpaWithLse(inputs[0].value(), inputs[1].value(), inputs[2].value(),
                                                      inputs[3], param.isCausal, param.scale, param.enableGqa,
                                                      param.qOffset, param.kOffset);
        outputs.push_back(o);
        outputs.push_back(lse);
        return;
    }
#endif
    IgnoreUnused(param, outputs);
    NeedsBackend("SdpaWithLse");
}

//------------------------------------------------- SdpaDecode --------------------------------------------------------

void SdpaDecodeOp::InferOutputMetaInfo() const {
    DDebugAssert(GetInputSize() == 4);
    DDebugAssert(GetOutputSize() == 2);
    const Shape& qShape = OperandA()->GetShape();
    DDebugAssert(qShape.NumAxis() == 4);
    OperandY()->MetaDataSameAs(OperandA());
    OperandY()->SetShapeAndStride(qShape);

    Operand* lse = GetOutputOperand(1);
    lse->MetaDataSameAs(OperandA());
    lse->SetDataKind(DataKind::kFloat32);
    lse->SetShapeAndStride(Shape{qShape[0], qShape[1]});
}

// Sequences are independent (all four inputs S(0)); heads split with the lengths replicated.
PlacementSignature SdpaDecodeOp::GetPlacementSignature() const {
    PlacementSignature::Builder builder(GetInputSize(), GetOutputSize());
    builder.AddInput(Shard(0))
        .AddInput(Shard(0))
        .AddInput(Shard(0))
        .AddInput(Shard(0))
        .AddOutput(Shard(0))
        .AddOutput(Shard(0))
        .Build();
    builder.AddInput(Shard(1))
        .AddInput(Shard(1))
        .AddInput(Shard(1))
        .AddInput("R")
        .AddOutput(Shard(1))
        .AddOutput(Shard(1))
        .Build();
    return builder.Finish();
}

void SdpaDecodeOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    const auto& param = GetOpParam<SdpaDecodeParam>();
    DDebugAssert(inputs.size() == 4);
#if DTORCH_WITH_DTATTN
    if (external::dtattn::IsSupportedDevice(inputs[0].value())) {
        auto [o, lse] = external::dtattn::Decode(inputs[0].value(), inputs[1].value(), inputs[2].value(),
                                                 inputs[3].value(), param.scale, param.chunk);
        outputs.push_back(o);
        outputs.push_back(lse);
        return;
    }
#endif
    IgnoreUnused(param, outputs);
    NeedsBackend("SdpaDecode");
}

//-------------------------------------------------- LseMerge ---------------------------------------------------------

void LseMergeOp::InferOutputMetaInfo() const {
    DDebugAssert(GetInputSize() >= 2 && GetInputSize() % 2 == 0);
    DDebugAssert(GetOutputSize() == 2);
    const auto& param = GetOpParam<LseMergeParam>();
    const Shape& oShape = OperandA()->GetShape();
    OperandY()->MetaDataSameAs(OperandA());
    if (param.outDataKind.has_value()) OperandY()->SetDataKind(param.outDataKind.value());
    OperandY()->SetShapeAndStride(oShape);

    Operand* lse = GetOutputOperand(1);
    lse->MetaDataSameAs(OperandB());
    lse->SetDataKind(DataKind::kFloat32);
    lse->SetShapeAndStride(RowShape(oShape));
}

// Rows are independent: every block and the result split alike on batch, heads or query rows.
PlacementSignature LseMergeOp::GetPlacementSignature() const {
    const size_t numAxis = OperandA()->GetShape().NumAxis();
    PlacementSignature::Builder builder(GetInputSize(), GetOutputSize());
    for (size_t axis = 0; axis + 1 < numAxis; ++axis) {
        for (size_t i = 0; i < GetInputSize(); ++i) builder.AddInput(Shard(axis));
        builder.AddOutput(Shard(axis)).AddOutput(Shard(axis)).Build();
    }
    return builder.Finish();
}

void LseMergeOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    const auto& param = GetOpParam<LseMergeParam>();
    DDebugAssert(inputs.size() >= 2 && inputs.size() % 2 == 0);
#if DTORCH_WITH_DTATTN
    if (external::dtattn::IsSupportedDevice(inputs[0].value())) {
        std::vector<::torch::Tensor> outs, lses;
        for (size_t i = 0; i < inputs.size(); i += 2) {
            outs.push_back(inputs[i].value());
            lses.push_back(inputs[i + 1].value());
        }
        std::optional<::torch::ScalarType> outType = std::nullopt;
        if (param.outDataKind.has_value()) outType = external::torch::TorchUtil::ToScalarType(param.outDataKind.value());
        auto [o, lse] = external::dtattn::LseMerge(outs, lses, outType);
        outputs.push_back(o);
        outputs.push_back(lse);
        return;
    }
#endif
    IgnoreUnused(param, outputs);
    NeedsBackend("LseMerge");
}

}  // namespace core
}  // namespace dtorch
