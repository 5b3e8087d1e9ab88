// Test module over the DTorch integration adapter (integration/tree/dtorch/external/dtattn/dtattn_adapter.cc):
// exposes its four entry points to Python so the GPU tests can hold the adapter's argument fills against
// the product path and the oracle.  Built in-tree by dtorch_amd/build.py (build_adapter_check).
#include <torch/extension.h>

#include "dtorch/external/dtattn/dtattn_adapter.h"

namespace A = dtorch::external::dtattn;

PYBIND11_MODULE(_adapter_check, m) {
    m.def("sdpa", &A::Sdpa, "SdpaOp::Compute's MI355X branch", pybind11::arg("q"), pybind11::arg("k"),
          pybind11::arg("v"), pybind11::arg("attn_mask") = std::nullopt, pybind11::arg("is_causal") = false,
          pybind11::arg("scale") = std::nullopt, pybind11::arg("enable_gqa") = false,
          pybind11::arg("sage_attention_type") = "", pybind11::call_guard<pybind11::gil_scoped_release>());
    m.def("sdpa_with_lse", &A::SdpaWithLse, pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"),
          pybind11::arg("attn_mask") = std::nullopt, pybind11::arg("is_causal") = false,
          pybind11::arg("scale") = std::nullopt, pybind11::arg("enable_gqa") = false, pybind11::arg("q_offset") = 0,
          pybind11::arg("k_offset") = 0, pybind11::call_guard<pybind11::gil_scoped_release>());
    m.def("decode", &A::Decode, pybind11::arg("q"), pybind11::arg("k_cache"), pybind11::arg("v_cache"),
          pybind11::arg("lengths"), pybind11::arg("scale") = std::nullopt, pybind11::arg("chunk") = 0,
          pybind11::call_guard<pybind11::gil_scoped_release>());
    m.def("lse_merge", &A::LseMerge, pybind11::arg("outs"), pybind11::arg("lses"),
          pybind11::arg("out_dtype") = std::nullopt, pybind11::call_guard<pybind11::gil_scoped_release>());
    m.def("is_supported_device", &A::IsSupportedDevice);
}
