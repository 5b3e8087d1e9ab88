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

TorchTensorArray RunCompute(const std::function<void(const TorchTensorOptArray&, TorchTensorArray&)>& f,
                            const std::vector<std::optional<at::Tensor>>& inputs) {
    TorchTensorOptArray in(inputs.begin(), inputs.end());
    TorchTensorArray out;
    f(in, out);
    return out;
}

}  // namespace

PYBIND11_MODULE(_dtattn_host, m) {
    m.doc() = "MI355X attention host operators (SdpaOp contract over the dtattn C ABI)";

    m.def("abi_version", []() { return dtattn_abi_version(); });

    py::class_<SdpaOption>(m, "SdpaOption")
        .def(py::init<>())
        .def(py::init<std::string>(), py::arg("sage_attention_type"))
        .def_readwrite("sage_attention_type", &SdpaOption::sageAttentionType)
        .def(py::pickle([](const SdpaOption& o) { return py::make_tuple(o.sageAttentionType); },
                        [](py::tuple t) { return SdpaOption(t[0].cast<std::string>()); }));

    py::class_<SdpaParam>(m, "SdpaParam")
        .def(py::init<>())
        .def(py::init<bool, std::optional<double>, bool, std::optional<SdpaOption>>(), py::arg("is_causal"),
             py::arg("scale"), py::arg("enable_gqa"), py::arg("option"))
        .def_readwrite("is_causal", &SdpaParam::isCausal)
        .def_readwrite("scale", &SdpaParam::scale)
        .def_readwrite("enable_gqa", &SdpaParam::enableGqa)
        .def_readwrite("option", &SdpaParam::option)
        // Serialised field order follows SdpaParam::serialize (scaled_dot_product_attention_op.h:27-35).
        .def(py::pickle(
            [](const SdpaParam& p) { return py::make_tuple(p.isCausal, p.scale, p.enableGqa, p.option); },
            [](py::tuple t) {
                return SdpaParam(t[0].cast<bool>(), t[1].cast<std::optional<double>>(), t[2].cast<bool>(),
                                 t[3].cast<std::optional<SdpaOption>>());
            }));

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
        .def(py::init<SdpaParam, int64_t, int64_t>(), py::arg("param"), py::arg("q_offset") = 0,
             py::arg("k_offset") = 0)
        .def("compute", [](const SdpaWithLseOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<SdpaDecodeOp>(m, "SdpaDecodeOp")
        .def(py::init<std::optional<double>, int32_t>(), py::arg("scale") = std::nullopt, py::arg("chunk") = 0)
        .def("compute", [](const SdpaDecodeOp& op, const std::vector<std::optional<at::Tensor>>& in) {
            return RunCompute([&](const TorchTensorOptArray& i, TorchTensorArray& o) { op.Compute(i, o); }, in);
        });

    py::class_<SdpaDecodePagedOp>(m, "SdpaDecodePagedOp")
        .def(py::init<std::optional<double>, int32_t>(), py::arg("scale") = std::nullopt, py::arg("chunk") = 0)
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
        .def(py::init<std::optional<c10::ScalarType>>(), py::arg("out_dtype") = std::nullopt)
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
