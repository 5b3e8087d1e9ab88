// Python bindings of the host operators (the counterpart of the reference's nanobind layer,
// dtorch/api/python/, for this path).  Exposes the operator objects with their Compute contract and
// the metadata functions, so that the Python front end and the tests drive exactly the code a
// DTorch Kernel would call.
#include <torch/extension.h>

#include "dtattn.h"
#include "sdpa_op.h"

namespace py = pybind11;
using namespace dtorch_amd::core;

namespace {

// Compute runs with the GIL released, so several Python threads (each with its own current stream,
// like the reference's per-device KernelStream threads) drive the host operators concurrently.  The
// arguments are converted before the release and the result after the re-acquire.
TorchTensorArray RunCompute(const std::function<void(const TorchTensorOptArray&, TorchTensorArray&)>& f,
                            const std::vector<std::optional<at::Tensor>>& inputs) {
    TorchTensorOptArray in(inputs.begin(), inputs.end());
    TorchTensorArray out;
    {
        py::gil_scoped_release nogil;
        f(in, out);
    }
    return out;
}

// to_bytes / from_bytes and pickle support through the param's field-order serialisation.
template <typename P, typename C>
void BindSerialisation(C& cls) {
    cls.def("to_bytes", [](const P& p) { return py::bytes(ToBytes(p)); })
        .def_static("from_bytes", [](const py::bytes& b) { return FromBytes<P>(std::string(b)); })
        .def(py::pickle([](const P& p) { return py::make_tuple(py::bytes(ToBytes(p))); },
                        [](py::tuple t) { return FromBytes<P>(t[0].cast<std::string>()); }));
}

}  // namespace

PYBIND11_MODULE(_dtattn_host, m) {
    m.doc() = "MI355X attention host operators (SdpaOp contract over the dtattn C ABI)";

    m.def("abi_version", []() { return dtattn_abi_version(); });

    auto opt = py::class_<SdpaOption>(m, "SdpaOption")
                   .def(py::init<>())
                   .def(py::init<std::string>(), py::arg("sage_attention_type"))
                   .def_readwrite("sage_attention_type", &SdpaOption::sageAttentionType);
    BindSerialisation<SdpaOption>(opt);

    // Serialised field order follows SdpaParam::serialize (scaled_dot_product_attention_op.h:27-35).
    auto sp = py::class_<SdpaParam>(m, "SdpaParam")
                  .def(py::init<>())
                  .def(py::init<bool, std::optional<double>, bool, std::optional<SdpaOption>>(),
                       py::arg("is_causal"), py::arg("scale"), py::arg("enable_gqa"), py::arg("option"))
                  .def_readwrite("is_causal", &SdpaParam::isCausal)
                  .def_readwrite("scale", &SdpaParam::scale)
                  .def_readwrite("enable_gqa", &SdpaParam::enableGqa)
                  .def_readwrite("option", &SdpaParam::option);
    BindSerialisation<SdpaParam>(sp);

    auto lp = py::class_<SdpaWithLseParam, SdpaParam>(m, "SdpaWithLseParam")
                  .def(py::init<>())
                  .def(py::init<SdpaParam, int64_t, int64_t>(), py::arg("base"), py::arg("q_offset") = 0,
                       py::arg("k_offset") = 0)
                  .def_readwrite("q_offset", &SdpaWithLseParam::qOffset)
                  .def_readwrite("k_offset", &SdpaWithLseParam::kOffset);
    BindSerialisation<SdpaWithLseParam>(lp);

    auto dp = py::class_<SdpaDecodeParam>(m, "SdpaDecodeParam")
                  .def(py::init<>())
                  .def(py::init<std::optional<double>, int32_t>(), py::arg("scale") = std::nullopt,
                       py::arg("chunk") = 0)
                  .def_readwrite("scale", &SdpaDecodeParam::scale)
                  .def_readwrite("chunk", &SdpaDecodeParam::chunk);
    BindSerialisation<SdpaDecodeParam>(dp);

    auto dpp = py::class_<SdpaDecodePagedParam, SdpaDecodeParam>(m, "SdpaDecodePagedParam")
                   .def(py::init<>())
                   .def(py::init<std::optional<double>, int32_t>(), py::arg("scale") = std::nullopt,
                        py::arg("chunk") = 0);
    BindSerialisation<SdpaDecodePagedParam>(dpp);

    auto mp = py::class_<LseMergeParam>(m, "LseMergeParam")
                  .def(py::init<>())
                  .def(py::init<std::optional<int32_t>>(), py::arg("out_kind"))
                  .def_readwrite("out_kind", &LseMergeParam::outKind);
    BindSerialisation<LseMergeParam>(mp);

    auto ap = py::class_<KvCacheAppendParam>(m, "KvCacheAppendParam").def(py::init<>());
    BindSerialisation<KvCacheAppendParam>(ap);
    auto app = py::class_<KvCacheAppendPagedParam>(m, "KvCacheAppendPagedParam").def(py::init<>());
    BindSerialisation<KvCacheAppendPagedParam>(app);
    auto qp = py::class_<Fp8QuantizeParam>(m, "Fp8QuantizeParam").def(py::init<>());
    BindSerialisation<Fp8QuantizeParam>(qp);

    py::class_<FoldedView>(m, "FoldedView")
        .def_readonly("B", &FoldedView::B)
        .def_readonly("H", &FoldedView::H)
        .def_readonly("S", &FoldedView::S)
        .def_readonly("D", &FoldedView::D)
        .def_readonly("sb", &FoldedView::sb)
        .def_readonly("sh", &FoldedView::sh)
        .def_readonly("ss", &FoldedView::ss)
        .def_readonly("copied", &FoldedView::copied);
    // The [B, H, S, D] view (folded batch, element strides) the operators pass to the kernels.
    m.def("folded_strides", &FoldedStrides, py::arg("tensor"));

    py::class_<PlacementRule>(m, "PlacementRule")
        .def_readonly("inputs", &PlacementRule::inputs)
        .def_readonly("outputs", &PlacementRule::outputs)
        .def_readonly("optional", &PlacementRule::optional);

    py::class_<SdpaOp>(m, "SdpaOp")
        .def(py::init<SdpaParam>())
        .def_property_readonly("param", &SdpaOp::Param)
        .def("infer_output_meta_info", &SdpaOp::InferOutputMetaInfo)
        .def("get_placement_signature", &SdpaOp::GetPlacementSignature)
        .def("match_placements", &SdpaOp::MatchPlacements)
        .def("get_operator_cost", &SdpaOp::GetOperatorCost)
        .def("get_algorithmic_flops", &SdpaOp::GetAlgorithmicFlops)
        .def("compute", [](const SdpaOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<SdpaWithLseOp, SdpaOp>(m, "SdpaWithLseOp")
        .def(py::init<SdpaWithLseParam>(), py::arg("param"))
        .def(py::init<SdpaParam, int64_t, int64_t>(), py::arg("param"), py::arg("q_offset") = 0,
             py::arg("k_offset") = 0)
        .def_property_readonly("lse_param", &SdpaWithLseOp::LseParam)
        .def("compute", [](const SdpaWithLseOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<SdpaDecodeOp>(m, "SdpaDecodeOp")
        .def(py::init<SdpaDecodeParam>(), py::arg("param"))
        .def(py::init<std::optional<double>, int32_t>(), py::arg("scale") = std::nullopt, py::arg("chunk") = 0)
        .def_property_readonly("param", &SdpaDecodeOp::Param)
        .def("compute", [](const SdpaDecodeOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<SdpaDecodePagedOp>(m, "SdpaDecodePagedOp")
        .def(py::init<SdpaDecodePagedParam>(), py::arg("param"))
        .def(py::init<std::optional<double>, int32_t>(), py::arg("scale") = std::nullopt, py::arg("chunk") = 0)
        .def_property_readonly("param", &SdpaDecodePagedOp::Param)
        .def("compute", [](const SdpaDecodePagedOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<KvCacheAppendOp>(m, "KvCacheAppendOp")
        .def(py::init<>())
        .def("compute", [](const KvCacheAppendOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<KvCacheAppendPagedOp>(m, "KvCacheAppendPagedOp")
        .def(py::init<>())
        .def("compute", [](const KvCacheAppendPagedOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<LseMergeOp>(m, "LseMergeOp")
        .def(py::init<LseMergeParam>(), py::arg("param"))
        .def(py::init([](std::optional<c10::ScalarType> dt) { return LseMergeOp(LseMergeOp::ParamFor(dt)); }),
             py::arg("out_dtype") = std::nullopt)
        .def_property_readonly("param", &LseMergeOp::Param)
        .def("compute", [](const LseMergeOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<Fp8QuantizeOp>(m, "Fp8QuantizeOp")
        .def(py::init<>())
        .def("compute", [](const Fp8QuantizeOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<DevicePeaks>(m, "DevicePeaks")
        .def_readonly("cu_count", &DevicePeaks::cuCount)
        .def_readonly("clock_hz", &DevicePeaks::clockHz)
        .def_readonly("bf16_flops", &DevicePeaks::bf16Flops)
        .def_readonly("fp8_flops", &DevicePeaks::fp8Flops)
        .def_readonly("hbm_bytes_per_s", &DevicePeaks::hbmBytesPerS)
        .def_readonly("arch", &DevicePeaks::arch);
    m.def("get_device_peaks", &GetDevicePeaks, py::arg("device") = 0);
}
