"""Writes tests/golden/sdpa_golden.npz: small seeded cases run through libtorch's CPU SDPA.

libtorch's ``scaled_dot_product_attention`` is the arithmetic SdpaOp::Compute executes
(dtorch/core/operators/standard/scaled_dot_product_attention_op.cc:107-109); the LSE comes from
libtorch's CPU flash-attention op.  The fp8 case records torch's float8_e4m3fn cast of the per-head
scaled inputs.  Regenerate with ``python tests/golden/make_golden.py`` (needs only torch + numpy).
"""
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sdpa_golden.npz")


def rnd(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


def sdpa_case(rng, B, Hq, Hkv, L, S, D, causal, scale=None):
    q, k, v = rnd(rng, B, Hq, L, D), rnd(rng, B, Hkv, S, D), rnd(rng, B, Hkv, S, D)
    tq, tk, tv = map(torch.from_numpy, (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, None, 0.0, causal, scale=scale,
                                                         enable_gqa=Hq != Hkv).numpy()
    g = Hq // Hkv
    _, lse = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu(
        tq, tk.repeat_interleave(g, 1), tv.repeat_interleave(g, 1), 0.0, causal, scale=scale)
    return dict(q=q, k=k, v=v, o=o, lse=lse.numpy(), causal=np.int32(causal),
                scale=np.float64(np.nan if scale is None else scale))


def main():
    rng = np.random.default_rng(0)
    cases = {
        "c1_small": sdpa_case(rng, 1, 2, 2, 64, 64, 64, True),
        "gqa_full": sdpa_case(rng, 2, 4, 2, 40, 72, 32, False),
        "causal_rect": sdpa_case(rng, 1, 2, 1, 24, 56, 64, True),
        "scaled": sdpa_case(rng, 1, 3, 3, 33, 47, 16, False, scale=0.3),
    }
    # decode: per-sequence loop over the true lengths, GQA, non-causal
    B, Hq, Hkv, Smax, D = 3, 4, 2, 96, 64
    q, kc, vc = rnd(rng, B, Hq, 1, D), rnd(rng, B, Hkv, Smax, D), rnd(rng, B, Hkv, Smax, D)
    lengths = np.array([5, 96, 41], dtype=np.int32)
    outs = []
    for b in range(B):
        L = int(lengths[b])
        outs.append(torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[b:b + 1]), torch.from_numpy(kc[b:b + 1, :, :L]), torch.from_numpy(vc[b:b + 1, :, :L]),
            enable_gqa=True).numpy())
    cases["decode"] = dict(q=q, k=kc, v=vc, lengths=lengths, o=np.concatenate(outs, 0))
    # fp8 per-head quantization via torch's float8_e4m3fn cast
    x = rnd(rng, 1, 3, 16, 32) * np.float32(3.0)
    x[0, 2] = 0.0  # an all-zero head
    amax = np.abs(x).max(axis=(-2, -1)).astype(np.float32)
    inv = np.where(amax > 0, np.float32(448.0) / np.where(amax > 0, amax, 1), 1).astype(np.float32)
    y = torch.from_numpy((x * inv[..., None, None]).astype(np.float32)).clamp(-448, 448)
    codes = y.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    descale = np.where(amax > 0, amax / np.float32(448.0), 1).astype(np.float32)
    cases["fp8"] = dict(x=x, codes=codes, descale=descale)

    flat = {}
    for name, d in cases.items():
        for k, v in d.items():
            flat[f"{name}/{k}"] = v
    np.savez_compressed(OUT, **flat)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
