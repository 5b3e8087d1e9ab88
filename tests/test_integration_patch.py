"""The DTorch integration patch (integration/dtorch_mi355x.patch), on the CPU.

- It applies with `git apply --check` to a scratch copy of a DTorch source tree (skipped where no tree is
  present, which includes every GPU box).
- It is what integration/make_patch.py produces from integration/tree/ and the edit list, so the committed
  patch cannot drift from the files the GPU tests compile.
- The X-macro gains the next free operator values after Sync (49), contiguous, so OperatorType::kCount and
  OpTypeToString's static_assert stay consistent.
- The adapter it adds compiles here against libtorch and include/dtattn.h.
"""
import os
import re
import shutil
import subprocess
import sys
import sysconfig

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATCH = os.path.join(ROOT, "integration", "dtorch_mi355x.patch")
SRC = os.environ.get("DTORCH_REFERENCE_TREE", "/root/reference")
ADAPTER = os.path.join(ROOT, "integration", "tree", "dtorch", "external", "dtattn", "dtattn_adapter.cc")

needs_tree = pytest.mark.skipif(not os.path.isfile(os.path.join(SRC, "dtorch", "core", "operators", "operator_param.h")),
                                reason="no DTorch source tree to check the patch against")


@needs_tree
def test_patch_applies_to_a_scratch_copy(tmp_path):
    dst = tmp_path / "dtorch"
    shutil.copytree(SRC, dst, symlinks=True)
    for dirpath, dirnames, files in os.walk(dst):
        for n in dirnames + files:
            p = os.path.join(dirpath, n)
            if not os.path.islink(p):
                os.chmod(p, os.stat(p).st_mode | 0o200)
    r = subprocess.run(["git", "apply", "--check", "-v", PATCH], cwd=dst, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run(["git", "apply", PATCH], cwd=dst, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    op = (dst / "dtorch" / "core" / "operators" / "operator_param.h").read_text()
    values = [int(v) for v in re.findall(r"Func\(\s*\w+\s*,\s*(\d+)\)", op)]
    assert values == list(range(len(values))) and values[-3:] == [50, 51, 52]
    for name in ("SdpaWithLse", "SdpaDecode", "LseMerge"):
        assert re.search(rf"Func\({name}\s*,", op)
    fac = (dst / "dtorch" / "core" / "operators" / "operator_factory.cc").read_text()
    for op_name, kind in (("SdpaWithLseOp", "kSdpaWithLse"), ("SdpaDecodeOp", "kSdpaDecode"), ("LseMergeOp", "kLseMerge")):
        assert f"RegisterOpConstructor<{op_name}>(OperatorType::{kind});" in fac
    sdpa = (dst / "dtorch" / "core" / "operators" / "standard" / "scaled_dot_product_attention_op.cc").read_text()
    assert "external::dtattn::Sdpa(" in sdpa


@needs_tree
def test_committed_patch_is_what_the_generator_makes():
    sys.path.insert(0, os.path.join(ROOT, "integration"))
    try:
        import make_patch
    finally:
        sys.path.pop(0)
    with open(PATCH) as f:
        assert make_patch.make_patch(SRC) == f.read(), "run python integration/make_patch.py"


def test_adapter_compiles_against_libtorch_and_the_abi():
    import torch
    import torch.utils.cpp_extension as ce
    incs = ce.include_paths() + [sysconfig.get_paths()["include"], os.path.join(ROOT, "include"),
                                 os.path.join(ROOT, "integration", "tree"), "/opt/rocm/include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-fsyntax-only", "-std=c++17", "-Wall", "-Werror", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", *[f"-I{i}" for i in incs], ADAPTER]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]


def test_block_op_params_serialise_their_base_first():
    # Every new param derives from OpParam and serialises BaseObject<OpParam>(*this) before its own fields,
    # in declaration order (operator_serialization_pack.h dispatches Name##Param for each X-macro entry).
    hdr = open(os.path.join(ROOT, "integration", "tree", "dtorch", "core", "operators", "standard",
                            "sdpa_block_ops.h")).read()
    for name in ("SdpaWithLseParam", "SdpaDecodeParam", "LseMergeParam"):
        body = hdr[hdr.index(f"struct {name} : public OpParam"):]
        body = body[:body.index("};")]
        fields = re.findall(r"^\s{4}(?:std::optional<[\w:]+>|bool|int64_t)\s+(\w+);", body, re.M)
        ser = re.findall(r"ar\s*&\s*(\w+);", body)
        assert "ar& BaseObject<OpParam>(*this);" in body, name
        assert ser == fields and fields, (name, fields, ser)
