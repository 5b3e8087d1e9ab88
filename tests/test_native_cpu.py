"""CPU-only checks of the native library and host operators (no kernel is launched).

* libdtattn.so loads and exports every function include/dtattn.h declares;
* the C ABI rejects bad arguments before touching a device, with the documented status codes and a
  readable dtattn_last_error();
* the SdpaOp mirror reproduces the reference's shape inference, placement signature and cost
  (scaled_dot_product_attention_op.cc:16-95, dtorch/tests/test_operator_cost.cc:171-183);
* errors surface as the reference's exception type (std::invalid_argument -> ValueError).
"""
import ctypes
import os
import pickle
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dtattn.h")

from dtorch_amd import _lib  # noqa: E402

lib = _lib.cabi()
host = _lib.load()


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\**\s+\**(dtattn_[a-z_0-9]+)\s*\(", text, re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    for n in ["dtattn_prefill_fwd", "dtattn_decode_splitkv", "dtattn_decode_workspace_size", "dtattn_decode_paged",
              "dtattn_decode_paged_workspace_size", "dtattn_kv_append", "dtattn_kv_append_paged", "dtattn_lse_merge",
              "dtattn_fp8_quantize_per_head", "dtattn_fp8_quantize_workspace_size", "dtattn_get_device_peaks",
              "dtattn_last_error", "dtattn_abi_version"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_matches_header():
    ver = int(re.search(r"#define DTATTN_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    lib.dtattn_abi_version.restype = ctypes.c_int
    assert lib.dtattn_abi_version() == ver == host.abi_version()


PrefillArgs = _lib.PrefillArgs  # ctypes mirror of dtattn_prefill_args (only used for validation paths)


def _args(**kw):
    a = PrefillArgs()
    fake = 0x10000  # never dereferenced: every case below fails validation first
    a.q = a.k = a.v = a.o = fake
    a.B, a.Hq, a.Hkv, a.Sq, a.Sk, a.D, a.Dv = 1, 8, 8, 64, 64, 128, 128
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[0], s[1], s[2] = 8 * 64 * 128, 64 * 128, 128
    a.dtype = a.o_dtype = 0
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _last_error():
    lib.dtattn_last_error.restype = ctypes.c_char_p
    return lib.dtattn_last_error().decode()


@pytest.mark.parametrize("kw,code,text", [
    (dict(Hq=6, Hkv=4), 1, "multiple"),
    (dict(D=100, Dv=100), 2, "multiples of 8"),                      # bf16 head dims: multiples of 8
    (dict(D=520, Dv=520), 2, "exceeds 512"),
    (dict(Dv=64, dtype=2, o_dtype=0, q_descale=0x10000, k_descale=0x10000, v_descale=0x10000), 2,
     "bf16/fp16/fp32 only"),                                         # D != Dv: not for fp8 codes
    (dict(D=520, Dv=520, dtype=3, o_dtype=3), 2, "fp32 head dims"),  # fp32: up to 512
    (dict(D=96, Dv=66, dtype=3, o_dtype=3), 2, "multiples of 4"),    # fp32: multiples of 4
    (dict(D=96, Dv=96, dtype=2, o_dtype=0, q_descale=0x10000, k_descale=0x10000, v_descale=0x10000), 2,
     "head dim"),                                                    # fp8: 64 or 128
    (dict(dtype=5, o_dtype=5), 2, "dtype"),
    (dict(dtype=3, o_dtype=0), 2, "output dtype"),                   # fp32 inputs need an fp32 output
    (dict(dtype=3, o_dtype=3, q_stride=(ctypes.c_int64 * 3)(8 * 64 * 128, 64 * 128, 130)), 2, "16 bytes"),
    (dict(dtype=2, o_dtype=0), 1, "descale"),
    (dict(q=0), 1, "null"),
    (dict(Sq=-1), 1, "bad sizes"),
    (dict(scale=float("inf")), 1, "finite"),                         # NaN selects 1/sqrt(D); any finite scale runs
    (dict(scale=float("-inf")), 1, "finite"),
])
def test_prefill_validation(kw, code, text):
    lib.dtattn_prefill_fwd.restype = ctypes.c_int
    a = _args(**kw)
    assert lib.dtattn_prefill_fwd(ctypes.byref(a), None) == code
    assert text in _last_error()


def test_prefill_mask_validation():
    # every case fails validation before any launch (the pointers are never dereferenced)
    lib.dtattn_prefill_fwd.restype = ctypes.c_int
    a = _args(mask=0x20000)
    a.mask_stride[0], a.mask_stride[1], a.mask_stride[2] = 0, 0, 6  # key-row pitch not a multiple of 4
    assert lib.dtattn_prefill_fwd(ctypes.byref(a), None) == 2 and "mask stride" in _last_error()
    a.mask_stride[2] = 64
    a.mask = 0x20004  # not 16-byte aligned
    assert lib.dtattn_prefill_fwd(ctypes.byref(a), None) == 2 and "aligned" in _last_error()
    a.mask, a.dtype = 0x20000, 2
    assert lib.dtattn_prefill_fwd(ctypes.byref(a), None) == 2 and "fp8" in _last_error()


def test_prefill_null_args():
    assert lib.dtattn_prefill_fwd(None, None) == 1
    assert "NULL" in _last_error()


def test_empty_problem_is_a_no_op():
    assert lib.dtattn_prefill_fwd(ctypes.byref(_args(B=0)), None) == 0


def test_workspace_sizes():
    lib.dtattn_decode_workspace_size.restype = ctypes.c_size_t
    lib.dtattn_decode_workspace_size.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int32]
    n = lib.dtattn_decode_workspace_size(64, 32, 8192, 128, 128)
    nsplit = 8192 // 128
    o_bytes = 64 * 32 * nsplit * 128 * 4
    lse_bytes = 64 * 32 * nsplit * 4
    up = lambda x: (x + 255) // 256 * 256
    assert n == up(o_bytes) + up(lse_bytes)
    assert lib.dtattn_decode_workspace_size(64, 32, 8192, 128, 0) == n  # sized for the smallest split, 128
    ns384 = -(-8192 // 384)  # 22 splits of 384 tokens
    assert lib.dtattn_decode_workspace_size(64, 32, 8192, 128, 384) == up(64 * 32 * ns384 * 128 * 4) + up(
        64 * 32 * ns384 * 4)
    lib.dtattn_fp8_quantize_workspace_size.restype = ctypes.c_size_t
    lib.dtattn_fp8_quantize_workspace_size.argtypes = [ctypes.c_int64] * 4
    assert lib.dtattn_fp8_quantize_workspace_size(1, 24, 4608, 128) == ((24 * 72 * 4 + 255) // 256) * 256  # 64-row slices


def test_decode_paged_validation():
    class PagedArgs(ctypes.Structure):
        _fields_ = [("q", ctypes.c_void_p), ("k_pages", ctypes.c_void_p), ("v_pages", ctypes.c_void_p),
                    ("block_table", ctypes.c_void_p), ("lengths", ctypes.c_void_p), ("o", ctypes.c_void_p),
                    ("lse", ctypes.c_void_p), ("B", ctypes.c_int64), ("Hq", ctypes.c_int64),
                    ("Hkv", ctypes.c_int64), ("D", ctypes.c_int64), ("num_pages", ctypes.c_int64),
                    ("page_size", ctypes.c_int64), ("max_pages", ctypes.c_int64), ("q_stride", ctypes.c_int64 * 2),
                    ("k_stride", ctypes.c_int64 * 3), ("v_stride", ctypes.c_int64 * 3),
                    ("o_stride", ctypes.c_int64 * 2), ("lse_stride", ctypes.c_int64 * 1),
                    ("block_table_stride", ctypes.c_int64), ("dtype", ctypes.c_int32), ("scale", ctypes.c_float),
                    ("chunk", ctypes.c_int32), ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t)]
    lib.dtattn_decode_paged.restype = ctypes.c_int
    a = PagedArgs()
    a.B, a.Hq, a.Hkv, a.D, a.num_pages, a.max_pages = 2, 8, 2, 128, 10, 4
    a.page_size = 48  # not a power of two
    assert lib.dtattn_decode_paged(ctypes.byref(a), None) == 1 and "page_size" in _last_error()
    a.page_size = 16
    a.Hq = 5  # not a multiple of Hkv
    assert lib.dtattn_decode_paged(ctypes.byref(a), None) == 1 and "multiple" in _last_error()
    a.Hq = 8
    assert lib.dtattn_decode_paged(ctypes.byref(a), None) == 1 and "null" in _last_error()
    a.chunk = 640  # split lengths are 128, 256, 384 or 512
    assert lib.dtattn_decode_paged(ctypes.byref(a), None) == 1 and "chunk" in _last_error()
    a.chunk = 384  # accepted: validation goes on to the pointers
    assert lib.dtattn_decode_paged(ctypes.byref(a), None) == 1 and "null" in _last_error()
    lib.dtattn_decode_paged_workspace_size.restype = ctypes.c_size_t
    lib.dtattn_decode_paged_workspace_size.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int32]
    lib.dtattn_decode_workspace_size.restype = ctypes.c_size_t
    lib.dtattn_decode_workspace_size.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int32]
    # the paged workspace is the padded one for S_max = max_pages * page_size
    assert lib.dtattn_decode_paged_workspace_size(64, 32, 512, 16, 128, 0) == \
        lib.dtattn_decode_workspace_size(64, 32, 8192, 128, 0)


class AppendArgs(ctypes.Structure):
    _fields_ = [("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p), ("k_cache", ctypes.c_void_p),
                ("v_cache", ctypes.c_void_p), ("lengths", ctypes.c_void_p), ("B", ctypes.c_int64),
                ("Hkv", ctypes.c_int64), ("n_new", ctypes.c_int64), ("S_max", ctypes.c_int64), ("D", ctypes.c_int64),
                ("k_new_stride", ctypes.c_int64 * 3), ("v_new_stride", ctypes.c_int64 * 3),
                ("k_stride", ctypes.c_int64 * 3), ("v_stride", ctypes.c_int64 * 3), ("dtype", ctypes.c_int32)]


class AppendPagedArgs(ctypes.Structure):
    _fields_ = [("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p), ("k_pages", ctypes.c_void_p),
                ("v_pages", ctypes.c_void_p), ("block_table", ctypes.c_void_p), ("lengths", ctypes.c_void_p),
                ("B", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("n_new", ctypes.c_int64), ("D", ctypes.c_int64),
                ("num_pages", ctypes.c_int64), ("page_size", ctypes.c_int64), ("max_pages", ctypes.c_int64),
                ("k_new_stride", ctypes.c_int64 * 3), ("v_new_stride", ctypes.c_int64 * 3),
                ("k_stride", ctypes.c_int64 * 3), ("v_stride", ctypes.c_int64 * 3),
                ("block_table_stride", ctypes.c_int64), ("dtype", ctypes.c_int32)]


def test_kv_append_validation():
    # every case fails validation before any launch (no pointer here is dereferenced)
    lib.dtattn_kv_append.restype = ctypes.c_int
    lib.dtattn_kv_append_paged.restype = ctypes.c_int
    assert lib.dtattn_kv_append(None, None) == 1
    a = AppendArgs()
    a.B, a.Hkv, a.n_new, a.S_max, a.D = 2, 2, 1, 64, 128
    a.dtype = 2  # fp8 is not a cache dtype
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 2 and "dtype" in _last_error()
    a.dtype, a.D = 0, 12
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 2 and "multiple of 16 bytes" in _last_error()
    a.dtype, a.D = 3, 6  # fp32 rows of 6 elements: 24 bytes
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 2 and "multiple of 16 bytes" in _last_error()
    a.dtype = 0
    a.D = 128
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 1 and "null" in _last_error()
    a.k_new = a.v_new = a.lengths = 4096  # never dereferenced: the stride check fails first
    for arr in (a.k_new_stride, a.v_new_stride, a.k_stride, a.v_stride):
        arr[0], arr[1], arr[2] = 2 * 64 * 128, 64 * 128, 128
    a.k_stride[2] = 100
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 2 and "16 bytes" in _last_error()
    a.k_stride[2] = 128
    a.k_new = 4104  # not 16-byte aligned
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 2 and "aligned" in _last_error()
    a.k_new, a.S_max = 4096, 0
    assert lib.dtattn_kv_append(ctypes.byref(a), None) == 1 and "S_max" in _last_error()
    p = AppendPagedArgs()
    p.B, p.Hkv, p.n_new, p.D, p.num_pages, p.max_pages, p.page_size = 2, 2, 1, 128, 8, 4, 24
    p.k_new = p.v_new = p.lengths = 4096
    for arr in (p.k_new_stride, p.v_new_stride, p.k_stride, p.v_stride):
        arr[0], arr[1], arr[2] = 2 * 64 * 128, 64 * 128, 128
    assert lib.dtattn_kv_append_paged(ctypes.byref(p), None) == 1 and "page_size" in _last_error()
    p.page_size, p.num_pages = 16, 0
    assert lib.dtattn_kv_append_paged(ctypes.byref(p), None) == 1 and "page counts" in _last_error()


def test_merge_validation():
    class MergeArgs(ctypes.Structure):
        _fields_ = [("n_blocks", ctypes.c_int32), ("o_blocks", ctypes.c_void_p * 16),
                    ("lse_blocks", ctypes.c_void_p * 16), ("B", ctypes.c_int64), ("H", ctypes.c_int64),
                    ("S", ctypes.c_int64), ("D", ctypes.c_int64), ("block_o_stride", ctypes.c_int64 * 3),
                    ("block_lse_stride", ctypes.c_int64 * 2), ("block_dtype", ctypes.c_int32),
                    ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p), ("o_stride", ctypes.c_int64 * 3),
                    ("lse_stride", ctypes.c_int64 * 2), ("o_dtype", ctypes.c_int32)]
    a = MergeArgs()
    a.n_blocks = 17
    assert lib.dtattn_lse_merge(ctypes.byref(a), None) == 1 and "n_blocks" in _last_error()
    a.n_blocks, a.B, a.H, a.S, a.D = 2, 1, 1, 4, 128
    a.o = 0x10000
    for s in (a.block_o_stride, a.o_stride):
        s[0], s[1], s[2] = 512, 512, 128
    a.o_blocks[0] = 0x10000
    assert lib.dtattn_lse_merge(ctypes.byref(a), None) == 1 and "null" in _last_error()


# --------------------------------------------------------------------------- host operator metadata

def test_infer_output_meta_info():
    op = host.SdpaOp(host.SdpaParam())
    assert op.infer_output_meta_info([1, 8, 512, 64], [1, 8, 512, 64], [1, 8, 512, 32]) == [1, 8, 512, 32]
    assert op.infer_output_meta_info([2, 3, 4, 32, 7, 16], [2, 3, 4, 32, 9, 16], [2, 3, 4, 32, 9, 16]) == \
        [2, 3, 4, 32, 7, 16]
    with pytest.raises(ValueError):
        op.infer_output_meta_info([8, 512, 64], [8, 512, 64], [8, 512, 64])


def test_operator_cost_matches_reference_test():
    op = host.SdpaOp(host.SdpaParam())
    assert op.get_operator_cost([2, 8, 16, 64], [2, 8, 20, 64], [2, 8, 20, 64]) == 2 * 2 * 8 * 16 * 20 * (64 + 64)
    # rank 5: batch = Prod(0, NumAxis - 4) over an inclusive range
    assert op.get_operator_cost([3, 2, 8, 16, 64], [3, 2, 8, 20, 64], [3, 2, 8, 20, 64]) == \
        2 * 6 * 8 * 16 * 20 * 128
    causal = host.SdpaOp(host.SdpaParam(True, None, False, None))
    assert causal.get_algorithmic_flops([4, 32, 2048, 128], [4, 8, 2048, 128], [4, 8, 2048, 128]) == 137506062336
    assert causal.get_operator_cost([4, 32, 2048, 128], [4, 8, 2048, 128], [4, 8, 2048, 128]) == 274877906944


def test_placement_signature_matches_reference():
    # scaled_dot_product_attention_op.cc:34-66 plus placement_signature.cc:65-88 (all-Replicate)
    op = host.SdpaOp(host.SdpaParam())
    rules = [(r.inputs, r.outputs) for r in op.get_placement_signature(4)]
    assert rules == [
        (["S(0)", "S(0)", "S(0)", "S(0)"], ["S(0)"]),
        (["S(1)", "S(1)", "S(1)", "R"], ["S(1)"]),
        (["S(2)", "R", "R", "R"], ["S(2)"]),
        (["R", "R", "R", "R"], ["R"]),
    ]
    assert len(op.get_placement_signature(5)) == 5  # heads axes 1 and 2 for rank 5
    assert op.match_placements(4, ["S(1)", "S(1)", "S(1)", ""]) == ["S(1)"]
    assert op.match_placements(4, ["S(2)", "R", "R", ""]) == ["S(2)"]
    with pytest.raises(ValueError):
        op.match_placements(4, ["S(2)", "S(2)", "S(2)", ""])  # ring needs K/V replicated


def test_param_serialisation_round_trip():
    p = host.SdpaParam(True, 0.125, True, host.SdpaOption("native_fp8"))
    q = pickle.loads(pickle.dumps(p))
    assert (q.is_causal, q.scale, q.enable_gqa, q.option.sage_attention_type) == (True, 0.125, True, "native_fp8")
    d = pickle.loads(pickle.dumps(host.SdpaParam()))
    assert (d.is_causal, d.scale, d.enable_gqa, d.option) == (False, None, False, None)


def test_cpu_tensors_are_rejected_not_computed():
    import dtorch_amd.nn.functional as F
    x = torch.randn(1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device tensors"):
        F.scaled_dot_product_attention(x, x, x)
    with pytest.raises(ValueError, match="device tensors"):
        F.lse_merge([x], [torch.zeros(1, 2, 8)])


def test_front_end_option_validation():
    import dtorch_amd.nn.functional as F
    assert F.SdpaOption().check_valid()
    assert F.SdpaOption(sage_attn_type="native_fp8").check_valid()
    assert not F.SdpaOption(sage_attn_type="int4").check_valid()
    x = torch.randn(1, 2, 8, 64)
    with pytest.raises(AssertionError):
        F.scaled_dot_product_attention(x, x, x, sdpa_option=F.SdpaOption(sage_attn_type="int4"))
    with pytest.raises(RuntimeError, match="sageattention"):
        F.scaled_dot_product_attention(x, x, x, sdpa_option=F.SdpaOption(sage_attn_type="auto"))
    with pytest.raises(NotImplementedError):
        F.scaled_dot_product_attention(x, x, x, sdpa_option=F.SdpaOption(ring_cp_dim=2))


def test_every_param_type_round_trips_in_field_order():
    import struct
    base = host.SdpaParam(True, 0.125, False, host.SdpaOption("native_fp8"))
    # SdpaParam: isCausal, scale, enableGqa, option (scaled_dot_product_attention_op.h:27-35); an optional
    # is a presence byte plus the value, a string a u64 length plus its bytes.
    want = (struct.pack("<?", True) + struct.pack("<B", 1) + struct.pack("<d", 0.125) + struct.pack("<?", False) +
            struct.pack("<B", 1) + struct.pack("<Q", 10) + b"native_fp8")
    assert base.to_bytes() == want
    assert host.SdpaParam().to_bytes() == b"\x00\x00\x00\x00"
    lp = host.SdpaWithLseParam(base, 4096, -7)
    assert lp.to_bytes() == want + struct.pack("<qq", 4096, -7)
    cases = [
        (host.SdpaParam, base, lambda p: (p.is_causal, p.scale, p.enable_gqa, p.option.sage_attention_type)),
        (host.SdpaWithLseParam, lp, lambda p: (p.is_causal, p.scale, p.q_offset, p.k_offset)),
        (host.SdpaDecodeParam, host.SdpaDecodeParam(0.09, 384), lambda p: (p.scale, p.chunk)),
        (host.SdpaDecodeParam, host.SdpaDecodeParam(), lambda p: (p.scale, p.chunk)),
        (host.SdpaDecodePagedParam, host.SdpaDecodePagedParam(None, 256), lambda p: (p.scale, p.chunk)),
        (host.LseMergeParam, host.LseMergeParam(3), lambda p: p.out_kind),
        (host.LseMergeParam, host.LseMergeParam(), lambda p: p.out_kind),
        (host.KvCacheAppendParam, host.KvCacheAppendParam(), lambda p: type(p).__name__),
        (host.KvCacheAppendPagedParam, host.KvCacheAppendPagedParam(), lambda p: type(p).__name__),
        (host.Fp8QuantizeParam, host.Fp8QuantizeParam(), lambda p: type(p).__name__),
    ]
    for cls, p, key in cases:
        q = cls.from_bytes(p.to_bytes())
        assert key(q) == key(p), cls
        r = pickle.loads(pickle.dumps(p))
        assert type(r) is cls and key(r) == key(p), cls
        assert cls().to_bytes() == cls.from_bytes(cls().to_bytes()).to_bytes()  # default-constructible
    assert host.SdpaDecodeParam(0.09, 384).to_bytes() == struct.pack("<Bd", 1, 0.09) + struct.pack("<i", 384)
    assert host.LseMergeParam(3).to_bytes() == struct.pack("<Bi", 1, 3)
    # a layout mismatch fails loudly instead of leaving fields unset
    with pytest.raises(ValueError, match="trailing"):
        host.SdpaParam.from_bytes(lp.to_bytes())
    with pytest.raises(ValueError, match="truncated"):
        host.SdpaWithLseParam.from_bytes(base.to_bytes())
    # a bool byte other than 0 or 1 (isCausal, then enableGqa) is rejected rather than copied into a bool
    for pos in (0, 1 + 1 + 8):
        bad = bytearray(want)
        bad[pos] = 2
        with pytest.raises(ValueError, match="corrupt bool"):
            host.SdpaParam.from_bytes(bytes(bad))
    # the operators keep their params
    assert host.SdpaWithLseOp(lp).lse_param.q_offset == 4096
    assert host.SdpaDecodeOp(host.SdpaDecodeParam(None, 128)).param.chunk == 128
    assert host.LseMergeOp(torch.float32).param.out_kind == 3
    assert host.LseMergeOp().param.out_kind is None


def _element_offset(t, idx):
    return sum(i * s for i, s in zip(idx, t.stride()))


def _check_folded(t):
    """Every element (b..., h, s, d) of t sits at b*sb + h*sh + s*ss + d of the view the kernels get."""
    import itertools
    f = host.folded_strides(t)
    src = t.contiguous() if f.copied else t
    batch = t.shape[:-3]
    assert f.B == int(torch.tensor(batch).prod()) if batch else f.B == 1
    assert (f.H, f.S, f.D) == tuple(t.shape[-3:])
    for bi, bidx in enumerate(itertools.product(*[range(n) for n in batch])):
        for h in {0, t.shape[-3] - 1}:
            for s in {0, t.shape[-2] - 1}:
                want = _element_offset(src, (*bidx, h, s, 0))
                assert bi * f.sb + h * f.sh + s * f.ss == want, (tuple(t.shape), t.stride(), bidx, h, s)
    for st, n in ((f.sb, f.B), (f.sh, f.H), (f.ss, f.S)):
        assert (st * t.element_size()) % 16 == 0 or n == 1


def test_folded_strides_of_rank5_views():
    # x.transpose(1, 2).unsqueeze(1): a size-1 axis right before H with a real batch axis before it
    x = torch.zeros(2, 96, 4, 128, dtype=torch.bfloat16)
    t = x.transpose(1, 2).unsqueeze(1)
    f = host.folded_strides(t)
    assert (f.B, f.sb, f.sh, f.ss, f.copied) == (2, 49152, 128, 512, False)
    _check_folded(t)
    # a head slice of a [A, 1, 2H, S, D] tensor
    y = torch.zeros(2, 1, 8, 16, 64, dtype=torch.bfloat16)[:, :, :4]
    f = host.folded_strides(y)
    assert (f.B, f.sb, f.copied) == (2, 8192, False)
    _check_folded(y)
    for shape in ((1, 3, 4, 16, 64), (3, 1, 1, 4, 16, 64), (1, 1, 4, 16, 64), (2, 3, 4, 16, 64)):
        _check_folded(torch.zeros(shape, dtype=torch.bfloat16))


def test_folded_strides_property_over_random_views():
    g = torch.Generator().manual_seed(0)
    for trial in range(200):
        nd = int(torch.randint(4, 7, (1,), generator=g))
        shape = [int(torch.randint(1, 4, (1,), generator=g)) for _ in range(nd - 3)] + [3, 5, 64]
        base = torch.zeros([n * 2 for n in shape[:-1]] + [64], dtype=torch.bfloat16)
        t = base[tuple(slice(0, n) for n in shape)]                       # strided slice
        if trial % 3 == 0 and nd >= 5:
            t = t.transpose(0, 1)                                        # permuted batch axes
        if trial % 4 == 1:
            t = t.transpose(-3, -2).contiguous().transpose(-3, -2)        # [.., S, H, D] memory
        if trial % 5 == 2:
            t = t.unsqueeze(int(torch.randint(0, t.dim() - 2, (1,), generator=g)))
        _check_folded(t)


def test_last_error_is_per_thread():
    # Each thread sees only the message of its own last failing call (validation runs before any device
    # work, so this needs no GPU).
    import threading
    lib.dtattn_last_error.restype = ctypes.c_char_p
    lib.dtattn_prefill_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.dtattn_lse_merge.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.dtattn_decode_splitkv.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    calls = {"prefill": (lib.dtattn_prefill_fwd, b"prefill: args is NULL"),
             "merge": (lib.dtattn_lse_merge, b"merge"),
             "decode": (lib.dtattn_decode_splitkv, b"decode: args is NULL")}
    bad, start = [], threading.Barrier(len(calls) + 1)

    def worker(name):
        fn, want = calls[name]
        start.wait()
        for _ in range(2000):
            if fn(None, None) == 0:
                bad.append((name, "accepted NULL"))
                return
            msg = lib.dtattn_last_error()
            if want not in msg or any(w in msg for n, (_, w) in calls.items() if n != name):
                bad.append((name, msg))
                return

    def quiet():  # never fails a call: its message stays empty throughout
        start.wait()
        for _ in range(2000):
            lib.dtattn_abi_version()
            if lib.dtattn_last_error() != b"":
                bad.append(("quiet", lib.dtattn_last_error()))
                return

    threads = [threading.Thread(target=worker, args=(n,)) for n in calls] + [threading.Thread(target=quiet)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not bad, bad
