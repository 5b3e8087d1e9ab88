#!/usr/bin/env python3
"""Regenerate integration/dtorch_mi355x.patch: the changes that put the MI355X attention kernels behind
DTorch's SdpaOp and register the block, decode and merge operators.

The script copies a DTorch source tree (default /root/reference) to a scratch directory, adds the new files
kept under integration/tree/, applies the in-place edits listed in EDITS below (each anchored on one line of
the original file, and checked to match exactly once), and writes `git diff` of the result with one line of
context.  Apply the patch from the root of a DTorch checkout with `git apply dtorch_mi355x.patch`, then
configure with -DDTORCH_WITH_DTATTN=ON -DDTATTN_ROOT=<this repository, built>.

Usage: python integration/make_patch.py [--src DTORCH_TREE] [--out PATCH]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
TREE = os.path.join(HERE, "tree")
DEFAULT_OUT = os.path.join(HERE, "dtorch_mi355x.patch")

# (file, anchor line, replacement text): the anchor must occur exactly once; the replacement keeps it.
EDITS = [
    # X-macro: the next free values after Sync (49); the serialisation pack and OpTypeToString follow it.
    ("dtorch/core/operators/operator_param.h",
     "    Func(Sync                           , 49)\n",
     "    Func(Sync                           , 49)           \\\n"
     "    Func(SdpaWithLse                    , 50)           \\\n"
     "    Func(SdpaDecode                     , 51)           \\\n"
     "    Func(LseMerge                       , 52)\n"),
    ("dtorch/core/operators/operator_factory.cc",
     '#include "standard/scaled_dot_product_attention_op.h"\n',
     '#include "standard/scaled_dot_product_attention_op.h"\n#include "standard/sdpa_block_ops.h"\n'),
    ("dtorch/core/operators/operator_factory.cc",
     "    RegisterOpConstructor<SdpaOp>(OperatorType::kSdpa);\n",
     "    RegisterOpConstructor<SdpaOp>(OperatorType::kSdpa);\n"
     "    RegisterOpConstructor<SdpaWithLseOp>(OperatorType::kSdpaWithLse);\n"
     "    RegisterOpConstructor<SdpaDecodeOp>(OperatorType::kSdpaDecode);\n"
     "    RegisterOpConstructor<LseMergeOp>(OperatorType::kLseMerge);\n"),
    ("dtorch/core/operators/operator_serialization_pack.h",
     '#include "standard/scaled_dot_product_attention_op.h"\n',
     '#include "standard/scaled_dot_product_attention_op.h"\n#include "standard/sdpa_block_ops.h"\n'),
    # SdpaOp::Compute: the MI355X kernels for device tensors, libtorch everywhere else (CPU meshes unchanged).
    ("dtorch/core/operators/standard/scaled_dot_product_attention_op.cc",
     '#include "dtorch/external/sage_attn/sage_attn_adapter.h"\n',
     '#include "dtorch/common/config.h"\n'
     '#include "dtorch/external/sage_attn/sage_attn_adapter.h"\n'
     "#if DTORCH_WITH_DTATTN\n"
     '#include "dtorch/external/dtattn/dtattn_adapter.h"\n'
     "#endif\n"),
    ("dtorch/core/operators/standard/scaled_dot_product_attention_op.cc",
     '    if (sageAttentionType == "") {\n',
     "#if DTORCH_WITH_DTATTN\n"
     "    // MI355X: every device call runs the gfx950 kernels, natively in fp8 for \"native_fp8\"; the third-party\n"
     "    // SageAttention types keep their adapter below.\n"
     "    if (external::dtattn::IsSupportedDevice(inputs[0].value()) &&\n"
     '        (sageAttentionType == "" || sageAttentionType == "native_fp8")) {\n'
     "        outputs.push_back(external::dtattn::Sdpa(inputs[0].value(), inputs[1].value(), inputs[2].value(),\n"
     "                                                 inputs[3], param.isCausal, param.scale, param.enableGqa,\n"
     "                                                 sageAttentionType));\n"
     "        return;\n"
     "    }\n"
     "#endif\n"
     '    if (sageAttentionType == "") {\n'),
    ("dtorch/api/cpp/functional/functional_option.h",
     '    // candidate: "", "auto", "qk_int8_pv_fp8", "qk_int8_pv_fp16"\n',
     '    // candidate: "", "auto", "qk_int8_pv_fp8", "qk_int8_pv_fp16", and "native_fp8" (the MI355X fp8\n'
     "    // kernels: per-head e4m3fn quantization, fp8 MFMA, output in the inputs' dtype)\n"),
    # Builders; the Python bindings are generated from these declarations.
    ("dtorch/api/cpp/functional/neural_network.h",
     "                                  bool enableGqa = false, std::optional<SdpaOption> sdpa_option = std::nullopt);\n",
     "                                  bool enableGqa = false, std::optional<SdpaOption> sdpa_option = std::nullopt);\n"
     "\n"
     "// Attention with its per-row log-sum-exp and the causal offsets of a ring block (key j visible to query i\n"
     "// iff j + kOffset <= i + qOffset): returns {O, LSE}.\n"
     "TensorArray _ScaledDotProductAttentionWithLse(const Tensor& query, const Tensor& key, const Tensor& value,\n"
     "                                              const std::optional<Tensor>& attnMask = std::nullopt,\n"
     "                                              bool isCausal = false, std::optional<double> scale = std::nullopt,\n"
     "                                              bool enableGqa = false, int64_t qOffset = 0, int64_t kOffset = 0);\n"
     "\n"
     "// Single-token decode against a padded KV cache with per-sequence lengths: returns {O, LSE}.\n"
     "TensorArray _DecodeAttention(const Tensor& query, const Tensor& kCache, const Tensor& vCache, const Tensor& lengths,\n"
     "                             std::optional<double> scale = std::nullopt, int64_t chunk = 0);\n"
     "\n"
     "// LSE merge of partial attention blocks over the same queries: returns {O, LSE}.\n"
     "TensorArray _LseMerge(const TensorArray& outs, const TensorArray& lses);\n"),
    ("dtorch/api/cpp/functional/neural_network.cc",
     '#include "dtorch/core/operators/standard/scaled_dot_product_attention_op.h"\n',
     '#include "dtorch/core/operators/standard/scaled_dot_product_attention_op.h"\n'
     '#include "dtorch/core/operators/standard/sdpa_block_ops.h"\n'),
    ("dtorch/api/cpp/functional/neural_network.cc",
     "Tensor Interpolate(const Tensor& input, const std::optional<Shape>& size,\n"
     "                   const std::optional<std::vector<double>>& scaleFactor, const std::string& mode,\n",
     "TensorArray _ScaledDotProductAttentionWithLse(const Tensor& query, const Tensor& key, const Tensor& value,\n"
     "                                              const std::optional<Tensor>& attnMask, bool isCausal,\n"
     "                                              std::optional<double> scale, bool enableGqa, int64_t qOffset,\n"
     "                                              int64_t kOffset) {\n"
     "    std::unique_ptr<core::OpParam> param(\n"
     "        new core::SdpaWithLseParam(isCausal, scale, enableGqa, std::nullopt, qOffset, kOffset));\n"
     "    TensorArray inputs = {query, key, value};\n"
     "    TensorArrayPushOptional(inputs, attnMask);\n"
     "    return core::GraphConstructor::AddOperator(std::move(param), inputs, true);\n"
     "}\n"
     "\n"
     "TensorArray _DecodeAttention(const Tensor& query, const Tensor& kCache, const Tensor& vCache, const Tensor& lengths,\n"
     "                             std::optional<double> scale, int64_t chunk) {\n"
     "    std::unique_ptr<core::OpParam> param(new core::SdpaDecodeParam(scale, chunk));\n"
     "    return core::GraphConstructor::AddOperator(std::move(param), {query, kCache, vCache, lengths}, true);\n"
     "}\n"
     "\n"
     "TensorArray _LseMerge(const TensorArray& outs, const TensorArray& lses) {\n"
     "    DAlwaysAssert(!outs.empty() && outs.size() == lses.size());\n"
     "    std::unique_ptr<core::OpParam> param(new core::LseMergeParam());\n"
     "    TensorArray inputs;\n"
     "    for (size_t i = 0; i < outs.size(); ++i) {\n"
     "        inputs.push_back(outs[i]);\n"
     "        inputs.push_back(lses[i]);\n"
     "    }\n"
     "    return core::GraphConstructor::AddOperator(std::move(param), inputs, true);\n"
     "}\n"
     "\n"
     "Tensor Interpolate(const Tensor& input, const std::optional<Shape>& size,\n"
     "                   const std::optional<std::vector<double>>& scaleFactor, const std::string& mode,\n"),
    # Build switch: off by default; on, the adapter links the library built from this repository.
    ("CMakeLists.txt",
     "option(DTORCH_WITH_BOOST                    \"Build DTorch with Boost\"                           ON)\n",
     "option(DTORCH_WITH_BOOST                    \"Build DTorch with Boost\"                           ON)\n"
     "option(DTORCH_WITH_DTATTN                   \"Build DTorch with the MI355X attention kernels\"    OFF)\n"
     "set(DTATTN_ROOT \"\" CACHE PATH \"Built MI355X attention library tree (include/dtattn.h, dtorch_amd/libdtattn.so)\")\n"),
    ("CMakeLists.txt",
     "message(STATUS \"DTORCH_WITH_BOOST:                             ${DTORCH_WITH_BOOST}\")\n",
     "message(STATUS \"DTORCH_WITH_BOOST:                             ${DTORCH_WITH_BOOST}\")\n"
     "message(STATUS \"DTORCH_WITH_DTATTN:                            ${DTORCH_WITH_DTATTN}\")\n"),
    ("dtorch/common/config.h.in",
     "#cmakedefine01  DTORCH_WITH_BOOST\n",
     "#cmakedefine01  DTORCH_WITH_BOOST\n#cmakedefine01  DTORCH_WITH_DTATTN\n"),
    ("dtorch/CMakeLists.txt",
     "#----------------------------------------------------------------------------------------\n"
     "# Set DTORCH_INCLUDE_DIRS DTORCH_LINK_LIBRARIES\n",
     "if(DTORCH_WITH_DTATTN)\n"
     "    if(NOT EXISTS \"${DTATTN_ROOT}/include/dtattn.h\" OR NOT EXISTS \"${DTATTN_ROOT}/dtorch_amd/libdtattn.so\")\n"
     "        message(FATAL_ERROR \"DTORCH_WITH_DTATTN needs DTATTN_ROOT at a built MI355X attention tree\")\n"
     "    endif()\n"
     "    list(APPEND DTORCH_INCLUDE_DIRS ${DTATTN_ROOT}/include)\n"
     "    list(APPEND DTORCH_LINK_LIBRARIES ${DTATTN_ROOT}/dtorch_amd/libdtattn.so)\n"
     "else()\n"
     "    file(GLOB_RECURSE tmp ${CMAKE_CURRENT_SOURCE_DIR}/external/dtattn/*)\n"
     "    list(REMOVE_ITEM DTORCH_LIB_CXX_SRCS ${tmp})\n"
     "endif()\n"
     "\n"
     "#----------------------------------------------------------------------------------------\n"
     "# Set DTORCH_INCLUDE_DIRS DTORCH_LINK_LIBRARIES\n"),
    # Python front end: native_fp8 is a valid option and needs no third-party package.
    ("python/dtorch/nn/functional.py",
     '            "qk_int8_pv_fp16",\n',
     '            "qk_int8_pv_fp16",\n            "native_fp8",\n'),
    ("python/dtorch/nn/functional.py",
     "    if sdpa_option.sage_attn_type:\n",
     '    if sdpa_option.sage_attn_type and sdpa_option.sage_attn_type != "native_fp8":\n'),
]


def apply_edits(root: str) -> None:
    for rel, anchor, repl in EDITS:
        path = os.path.join(root, rel)
        with open(path) as f:
            text = f.read()
        n = text.count(anchor)
        if n != 1:
            raise SystemExit(f"make_patch: anchor found {n} times in {rel}: {anchor!r}")
        with open(path, "w") as f:
            f.write(text.replace(anchor, repl))
    for dirpath, _, files in os.walk(TREE):
        for name in files:
            src = os.path.join(dirpath, name)
            dst = os.path.join(root, os.path.relpath(src, TREE))
            os.makedirs(os.path.dirname(dst), exist_ok=True)
            shutil.copyfile(src, dst)


def git(root: str, *args: str) -> str:
    env = dict(os.environ, GIT_AUTHOR_NAME="x", GIT_AUTHOR_EMAIL="x@x", GIT_COMMITTER_NAME="x",
               GIT_COMMITTER_EMAIL="x@x")
    r = subprocess.run(["git", "-c", "core.autocrlf=false", *args], cwd=root, env=env, capture_output=True, text=True)
    if r.returncode != 0:
        raise SystemExit(f"make_patch: git {' '.join(args)} failed: {r.stderr}")
    return r.stdout


def make_patch(src: str) -> str:
    with tempfile.TemporaryDirectory() as tmp:
        root = os.path.join(tmp, "dtorch")
        shutil.copytree(src, root, symlinks=True)
        for dirpath, dirnames, files in os.walk(root):  # the source tree may be read-only: make it writable
            for n in dirnames:
                os.chmod(os.path.join(dirpath, n), 0o755)
            for n in files:
                path = os.path.join(dirpath, n)
                if not os.path.islink(path):
                    os.chmod(path, 0o755 if os.stat(path).st_mode & 0o111 else 0o644)
        git(root, "init", "-q")
        git(root, "add", "-A")
        git(root, "commit", "-q", "-m", "base")
        apply_edits(root)
        git(root, "add", "-A")
        return git(root, "diff", "--cached", "--unified=1", "--no-color")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--src", default="/root/reference", help="DTorch source tree the patch is made against")
    ap.add_argument("--out", default=DEFAULT_OUT)
    args = ap.parse_args()
    patch = make_patch(args.src)
    with open(args.out, "w") as f:
        f.write(patch)
    print(f"wrote {args.out} ({patch.count(chr(10))} lines)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
