"""In-tree build of the MI355X attention library and its host operator extension.

Outputs (next to this file, git-ignored, shipped with the tree):
  libdtattn.so                         HIP kernels for gfx950 + the dtattn C ABI (include/dtattn.h)
  _dtattn_host.<ext-suffix>.so         C++ host operators (SdpaOp contract) + Python bindings,
                                       linked against libtorch and libdtattn.so (RPATH $ORIGIN)

Run ``python -m dtorch_amd.build`` (or call :func:`build`).  Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_SOURCES = ["prefill_fwd.hip", "prefill_rows64.hip", "prefill_f32.hip", "prefill_wide.hip", "prefill_wide512.hip", "prefill_fp8.hip", "decode_splitkv.hip", "lse_merge.hip", "fp8_quant.hip", "kv_append.hip",
               "dtattn_abi.cpp"]
HOST_SOURCES = ["host/sdpa_op.cc", "host/bindings.cc"]

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
    # packed-fp32 VALU forms are disabled for every HIP translation unit
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{CSRC}", f"-I{BUILD}",
]

# Per-file flags.  The D = 512 wide-head kernel runs one wave per SIMD with 256 VGPRs and AGPRs beside them;
# left to its heuristics the compiler keeps O's 128 accumulators in AGPRs and copies all of them to VGPRs
# and back around every tile's PV MFMAs (256 moves per 32-key tile), and parks the LDS read addresses in
# AGPRs.  MFMAs in their VGPR-accumulator form remove the copies: 980 -> 924 us on a 16384-token VAE
# attention, bit-identical output; the D = 256 instantiations compile to the same code.
EXTRA_FLAGS = {"prefill_wide.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form=1"]}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _hipcc():
    p = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; the MI355X kernels need ROCm's hipcc")
    return p


def generate_sources() -> None:
    """Sources written by generators: the tile-loop programs of prefill_rows64.hip and prefill_wide512.hip."""
    os.makedirs(BUILD, exist_ok=True)
    _run([sys.executable, os.path.join(CSRC, "gen_prefill_rows64.py"), os.path.join(BUILD, "prefill_rows64_asm.inc")])
    _run([sys.executable, os.path.join(CSRC, "gen_prefill_wide512.py"), os.path.join(BUILD, "prefill_wide512_asm.inc")])


def build_library(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    generate_sources()
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, cmds):
            if out.strip():
                print(out)
    lib = os.path.join(PKG, "libdtattn.so")
    tmp = lib + ".tmp"
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp, "-Wl,-soname,libdtattn.so"])
    os.replace(tmp, lib)
    return lib


def build_host_extension() -> str:
    import torch  # noqa: F401  (only for include/library paths)
    import torch.utils.cpp_extension as ce

    os.makedirs(BUILD, exist_ok=True)
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "_dtattn_host" + suffix)
    incs = ce.include_paths() + [sysconfig.get_paths()["include"], INCLUDE, os.path.join(CSRC, "host"),
                                 os.path.join(ROCM, "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-variable", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
              "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_dtattn_host",
              "-DTORCH_API_INCLUDE_EXTENSION_H"] + [f"-I{i}" for i in incs]
    objs, cmds = [], []
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append(["g++", *cflags, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(_run, cmds))
    libdirs = ce.library_paths()
    tmp = out + ".tmp"
    _run(["g++", "-shared", "-fPIC", *objs, "-o", tmp, f"-L{PKG}", "-ldtattn", *[f"-L{d}" for d in libdirs],
          "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_c_client(src: str, out: str) -> str:
    """A plain C program against include/dtattn.h and libdtattn.so (no torch): gcc with the HIP runtime's C
    API, RPATH to the package directory and ROCm's libraries."""
    rel = os.path.relpath(PKG, os.path.dirname(out))
    _run(["gcc", "-O2", "-std=c11", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", f"-I{os.path.join(ROCM, 'include')}",
          src, "-o", out + ".tmp", f"-L{PKG}", "-ldtattn", f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64", "-lm",
          f"-Wl,-rpath,$ORIGIN/{rel}", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"])
    os.replace(out + ".tmp", out)
    return out


def build_adapter_check() -> str:
    """The test module over the DTorch integration adapter (integration/tree/.../dtattn_adapter.cc, the file the
    integration patch adds to a DTorch tree): the adapter and its pybind wrapper, compiled as the host
    extension is, in-tree under tests/integration_adapter/."""
    import torch  # noqa: F401
    import torch.utils.cpp_extension as ce

    tree = os.path.join(ROOT, "integration", "tree")
    outdir = os.path.join(ROOT, "tests", "integration_adapter")
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(outdir, "_adapter_check" + suffix)
    incs = ce.include_paths() + [sysconfig.get_paths()["include"], INCLUDE, tree, os.path.join(ROCM, "include")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1",
              "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_adapter_check", "-DTORCH_API_INCLUDE_EXTENSION_H"]
    cflags += [f"-I{i}" for i in incs]
    srcs = [os.path.join(tree, "dtorch", "external", "dtattn", "dtattn_adapter.cc"), os.path.join(outdir, "bindings.cc")]
    objs, cmds = [], []
    for src in srcs:
        obj = os.path.join(BUILD, "adapter_" + os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append(["g++", *cflags, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(_run, cmds))
    rel = os.path.relpath(PKG, outdir)
    tmp = out + ".tmp"
    _run(["g++", "-shared", "-fPIC", *objs, "-o", tmp, f"-L{PKG}", "-ldtattn",
          *[f"-L{d}" for d in ce.library_paths()], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
          "-ltorch_python", f"-Wl,-rpath,$ORIGIN/{rel}"])
    os.replace(tmp, out)
    return out


def build() -> None:
    build_library()
    build_host_extension()
    build_adapter_check()


if __name__ == "__main__":
    build()
    print("built", os.path.join(PKG, "libdtattn.so"), file=sys.stderr)
