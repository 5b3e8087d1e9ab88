"""The C ABI from a plain C program (tests/c_abi/abi_client.c: gcc, the HIP runtime's C API, no torch and
no Python): inputs written here, the program calls dtattn_prefill_fwd / dtattn_decode_splitkv /
dtattn_decode_splitkv_noalloc on hipMalloc'd buffers, and its outputs are checked against the oracle.
This is the boundary a DTorch maintainer's SdpaOp::Compute branch would call
(scaled_dot_product_attention_op.cc:107-109), exercised without the host extension."""
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import sdpa as orc
from tests.attn_cases import LSE_TOL, O_TOL_BF16, lse_rel, max_abs, randn

pytestmark = pytest.mark.gpu

CLIENT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "abi_client")


def _bf16_bits(x: np.ndarray) -> bytes:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().tobytes()


def _bf16_values(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).double().numpy()


def _read_bf16(path: str, shape) -> np.ndarray:
    bits = np.fromfile(path, dtype=np.int16).reshape(shape)
    return torch.from_numpy(bits).view(torch.bfloat16).double().numpy()


def _run(mode: str, d: str) -> None:
    assert os.path.exists(CLIENT), f"{CLIENT} is missing: run __graft_entry__.build() first"
    print(f"abi_client {mode} {open(os.path.join(d, 'meta')).read().strip()}", flush=True)
    r = subprocess.run([CLIENT, mode, d], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", [
    (1, 4, 2, 200, 200, 128, True),     # causal GQA
    (2, 2, 2, 130, 257, 96, False),     # a padded head dim, ragged
    (1, 2, 1, 256, 2048, 512, False),   # a wide head whose keys run as blocks in the C caller's workspace
])
def test_c_client_prefill(tmp_path, B, Hq, Hkv, Sq, Sk, D, causal):
    rng = np.random.default_rng(Sq + D)
    q, k, v = randn(rng, (B, Hq, Sq, D)), randn(rng, (B, Hkv, Sk, D)), randn(rng, (B, Hkv, Sk, D))
    d = str(tmp_path)
    with open(os.path.join(d, "meta"), "w") as f:
        f.write(f"{B} {Hq} {Hkv} {Sq} {Sk} {D} {int(causal)}\n")
    for name, x in (("q", q), ("k", k), ("v", v)):
        with open(os.path.join(d, name + ".bin"), "wb") as f:
            f.write(_bf16_bits(x))
    _run("prefill", d)
    o = _read_bf16(os.path.join(d, "o.bin"), (B, Hq, Sq, D))
    lse = np.fromfile(os.path.join(d, "lse.bin"), dtype=np.float32).reshape(B, Hq, Sq)
    ro, rl = orc.sdpa_fwd(_bf16_values(q), _bf16_values(k), _bf16_values(v), is_causal=causal, enable_gqa=True)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl) <= LSE_TOL


def test_c_client_decode_and_noalloc(tmp_path):
    rng = np.random.default_rng(5)
    B, Hq, Hkv, Smax, D = 3, 8, 2, 1024, 128
    lengths = np.array([0, 300, 1000], dtype=np.int32)
    q = randn(rng, (B, Hq, 1, D))
    kc, vc = randn(rng, (B, Hkv, Smax, D)), randn(rng, (B, Hkv, Smax, D))
    d = str(tmp_path)
    with open(os.path.join(d, "meta"), "w") as f:
        f.write(f"{B} {Hq} {Hkv} {Smax} {D}\n")
    for name, x in (("q", q), ("k", kc), ("v", vc)):
        with open(os.path.join(d, name + ".bin"), "wb") as f:
            f.write(_bf16_bits(x))
    lengths.tofile(os.path.join(d, "lengths.bin"))
    _run("decode", d)
    o = _read_bf16(os.path.join(d, "o.bin"), (B, Hq, 1, D))
    lse = np.fromfile(os.path.join(d, "lse.bin"), dtype=np.float32).reshape(B, Hq)
    ro, rl = orc.decode(_bf16_values(q), _bf16_values(kc), _bf16_values(vc), lengths)
    assert max_abs(o, ro) <= O_TOL_BF16
    assert lse_rel(lse, rl[..., 0]) <= LSE_TOL
    # the allocation-free entry point returns the same bits as the workspace one
    assert open(os.path.join(d, "o.bin"), "rb").read() == open(os.path.join(d, "o_noalloc.bin"), "rb").read()
    assert open(os.path.join(d, "lse.bin"), "rb").read() == open(os.path.join(d, "lse_noalloc.bin"), "rb").read()
