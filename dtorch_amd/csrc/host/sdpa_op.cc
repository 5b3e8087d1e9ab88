// Host operators of the MI355X attention path (see sdpa_op.h).  All arithmetic goes through the
// dtattn C ABI; this file only validates, allocates outputs/workspace from the c10 caching
// allocator on the current device, and launches on the thread's current HIP stream (the stream the
// reference's KernelStream thread sets once: dtorch/core/kernel_stream/cuda_kernel_stream.cc:25-43).
// It never creates or switches streams and never synchronises.
#include "sdpa_op.h"

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <sstream>
#include <stdexcept>

#include "dtattn.h"

namespace dtorch_amd {
namespace core {

namespace {

[[noreturn]] void Throw(const std::string& msg) { throw std::invalid_argument("dtorch_amd: " + msg); }

void Check(int status, const char* what) {
    if (status == DTATTN_OK) return;
    std::ostringstream os;
    os << what << " failed (status " << status << "): " << dtattn_last_error();
    if (status == DTATTN_ERR_LAUNCH || status == DTATTN_ERR_DEVICE) throw std::runtime_error("dtorch_amd: " + os.str());
    Throw(os.str());
}

void* CurrentStream(const at::Tensor& t) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

int32_t DtypeCode(c10::ScalarType st) {
    switch (st) {
        case c10::ScalarType::BFloat16: return DTATTN_BF16;
        case c10::ScalarType::Half: return DTATTN_FP16;
        case c10::ScalarType::Float8_e4m3fn: return DTATTN_FP8_E4M3FN;
        case c10::ScalarType::Float: return DTATTN_FP32;
        default: return -1;
    }
}

// A tensor viewed as [B, H, S, D] (leading axes folded into B), last-axis stride 1, 16-byte aligned
// strides and base pointer.  Anything else is made contiguous first (a layout copy, not compute).
struct View4 {
    at::Tensor t;
    int64_t B, H, S, D;
    int64_t sb, sh, ss;
};

// The leading (batch) axes 0 .. nd-4 fold into one axis of stride `sb` iff the axes of size > 1 form
// one arithmetic progression: for consecutive such axes i < j, stride(i) == stride(j) * size(j).
// Size-1 axes carry no stride information and are skipped; `sb` is then the stride of the innermost
// batch axis of size > 1 (any value works when the folded batch is 1, since it is never multiplied
// by a non-zero index).
bool FoldBatch(const at::Tensor& t, int64_t& sb) {
    const int64_t nd = t.dim();
    int64_t prev = -1;
    sb = 0;
    for (int64_t i = 0; i < nd - 3; ++i) {
        if (t.size(i) == 1) continue;
        if (prev >= 0 && t.stride(prev) != t.stride(i) * t.size(i)) return false;
        prev = i;
        sb = t.stride(i);
    }
    return true;
}

View4 MakeView4(const at::Tensor& in, const char* name) {
    if (in.dim() < 4) Throw(std::string(name) + " must have at least 4 dimensions [..., H, S, D]");
    at::Tensor t = in;
    const int64_t esz = t.element_size();
    int64_t sb = 0;
    auto ok = [&](const at::Tensor& x) {
        if (x.stride(-1) != 1 || !FoldBatch(x, sb)) return false;
        if ((reinterpret_cast<uintptr_t>(x.data_ptr()) & 15u) != 0) return false;
        for (int64_t i = 0; i < x.dim() - 1; ++i)
            if (x.size(i) > 1 && (x.stride(i) * esz) % 16 != 0) return false;
        return true;
    };
    if (!ok(t)) {
        t = t.contiguous();
        FoldBatch(t, sb);  // always foldable once contiguous
    }
    View4 v;
    v.t = t;
    const int64_t nd = t.dim();
    v.B = 1;
    for (int64_t i = 0; i < nd - 3; ++i) v.B *= t.size(i);
    v.H = t.size(nd - 3);
    v.S = t.size(nd - 2);
    v.D = t.size(nd - 1);
    // Size-1 axes are never indexed past 0, so their strides are free: give them the contiguous
    // values, which keeps every stride the kernels see a multiple of 16 bytes.
    v.ss = v.S > 1 ? t.stride(nd - 2) : v.D;
    v.sh = v.H > 1 ? t.stride(nd - 3) : v.S * v.ss;
    // A folded batch of 1 is never indexed past 0: give it the extent of one (H, S, D) slab.
    v.sb = v.B > 1 ? sb : v.H * v.sh;
    return v;
}

}  // namespace

FoldedView FoldedStrides(const at::Tensor& t) {
    const View4 v = MakeView4(t, "tensor");
    return {v.B, v.H, v.S, v.D, v.sb, v.sh, v.ss, !v.t.is_same(t)};
}

namespace {

void CheckDevice(const std::vector<const at::Tensor*>& ts) {
    const at::Device dev = ts[0]->device();
    if (!dev.is_cuda())
        Throw("the MI355X attention kernels take device tensors; CPU meshes keep DTorch's libtorch path");
    for (const at::Tensor* t : ts)
        if (t->device() != dev) Throw("all tensors must be on the same device");
}

struct PrefillResult {
    at::Tensor o, lse;
};

// attn_mask -> the additive fp32 form the kernels read: [B, Hq, Sq, Sk] with broadcast axes at stride 0,
// key stride 1, other strides multiples of 4 and a 16-byte aligned base.  A boolean mask keeps True
// entries (0) and hides False ones (-inf), as torch::scaled_dot_product_attention does.  Only the
// mask's own (unbroadcast) extent is ever copied: to fp32, and to a row pitch padded to 4 when needed.
at::Tensor PrepareMask(const at::Tensor& m, const at::Tensor& q, const at::Tensor& k, int64_t B, int64_t Hq,
                       int64_t Sq, int64_t Sk) {
    if (m.device() != q.device()) Throw("attn_mask must be on the query's device");
    if (m.scalar_type() != at::kBool && !at::isFloatingType(m.scalar_type()))
        Throw("attn_mask must be boolean or floating point");
    if (m.dim() < 1) Throw("attn_mask must have at least one dimension");
    at::Tensor mf = m.scalar_type() == at::kBool
                        ? at::where(m, at::zeros({}, q.options().dtype(at::kFloat)),
                                    at::full({}, -std::numeric_limits<float>::infinity(), q.options().dtype(at::kFloat)))
                        : m.to(at::kFloat);
    if (mf.size(-1) == 1 && Sk > 1) {  // broadcast along the keys: spell it out (the kernel reads key stride 1)
        std::vector<int64_t> sz = mf.sizes().vec();
        sz.back() = Sk;
        mf = mf.expand(sz);
    }
    bool ok = mf.stride(-1) == 1 && (reinterpret_cast<uintptr_t>(mf.data_ptr()) & 15u) == 0;
    for (int64_t i = 0; i + 1 < mf.dim(); ++i)
        if (mf.size(i) > 1 && mf.stride(i) % 4 != 0) ok = false;
    if (!ok) {  // padded row pitch, contiguous otherwise
        std::vector<int64_t> sz = mf.sizes().vec();
        const int64_t n = sz.back();
        sz.back() = (n + 3) / 4 * 4;
        at::Tensor pad = at::zeros(sz, mf.options());
        pad.narrow(-1, 0, n).copy_(mf);
        mf = pad.narrow(-1, 0, n);
    }
    std::vector<int64_t> full = q.sizes().vec();
    full.back() = k.size(-2);
    at::Tensor e;
    try {
        e = mf.expand(full);
    } catch (const c10::Error&) {
        Throw("attn_mask is not broadcastable to [..., Hq, L, S]");
    }
    if (e.dim() > 4) e = e.reshape({B, Hq, Sq, Sk});  // a view when the batch axes fold, else a copy
    if (e.stride(3) != 1 && Sk > 1) Throw("internal: mask key stride");
    for (int i = 0; i < 3; ++i)
        if (e.size(i) > 1 && e.stride(i) % 4 != 0) e = e.contiguous();  // only after a reshape copy of odd pitch
    return e;
}

PrefillResult RunPrefill(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_, const SdpaParam& prm,
                         int64_t qOffset, int64_t kOffset, bool wantLse, const at::Tensor* mask = nullptr) {
    CheckDevice({&q_, &k_, &v_});
    c10::DeviceGuard guard(q_.device());
    if (q_.dim() != k_.dim() || q_.dim() != v_.dim()) Throw("query, key and value must have the same rank");
    for (int64_t i = 0; i < q_.dim() - 3; ++i)
        if (q_.size(i) != k_.size(i) || q_.size(i) != v_.size(i))
            Throw("query, key and value batch dimensions differ");
    if (q_.size(-1) != k_.size(-1)) Throw("query and key head dims differ");
    if (k_.size(-2) != v_.size(-2) || k_.size(-3) != v_.size(-3)) Throw("key and value shapes differ");
    const int64_t hq = q_.size(-3), hkv = k_.size(-3);
    if (hkv == 0 && hq > 0) Throw("key and value must have at least one head");
    if (hq != hkv) {
        if (!prm.enableGqa) Throw("query and key/value head counts differ; set enable_gqa=True");
        if (hq % hkv != 0) Throw("number of query heads must be a multiple of key/value heads");
    }
    if (prm.scale.has_value() && !std::isfinite(prm.scale.value())) Throw("scale must be finite");

    std::string quant;
    if (prm.option.has_value()) quant = prm.option->sageAttentionType;
    const bool fp8 = quant == "native_fp8";
    if (!quant.empty() && !fp8)
        Throw("sage_attn_type '" + quant +
              "' selects the third-party SageAttention package, which this build does not ship; use '' or "
              "'native_fp8'");

    const c10::ScalarType st = q_.scalar_type();
    if (k_.scalar_type() != st || v_.scalar_type() != st) Throw("query, key and value dtypes differ");
    if (st != c10::ScalarType::BFloat16 && st != c10::ScalarType::Half && st != c10::ScalarType::Float)
        Throw(std::string("dtype ") + c10::toString(st) + " is not supported by the MI355X kernels (bf16, fp16, fp32)");
    if (fp8 && st != c10::ScalarType::BFloat16 && st != c10::ScalarType::Half)
        Throw("native_fp8 takes bf16 or fp16 inputs");

    // Head dims the kernels do not take directly (16-bit: not a multiple of 8; fp32: not a multiple of 4), as
    // libtorch takes any (scaled_dot_product_attention_op.cc:107-109 forwards them): q and k are zero-padded
    // on D and v on Dv to the next multiple, the call runs on the padded tensors with the scale of the real D
    // (1/sqrt(D) when none is given), and the output is cut back to Dv.  Zero columns add nothing to any score,
    // and the padded output columns are dropped, so the result is the call on the real dims.
    {
        const int64_t step = st == c10::ScalarType::Float ? 4 : 8;
        const int64_t d = q_.size(-1), dv = v_.size(-1);
        const int64_t dp = (d + step - 1) / step * step, dvp = (dv + step - 1) / step * step;
        if ((dp != d || dvp != dv) && d > 0 && dv > 0) {
            SdpaParam padded = prm;
            if (!padded.scale.has_value()) padded.scale = 1.0 / std::sqrt((double)d);
            const at::Tensor qp = dp != d ? at::constant_pad_nd(q_, {0, dp - d}) : q_;
            const at::Tensor kp = dp != d ? at::constant_pad_nd(k_, {0, dp - d}) : k_;
            const at::Tensor vp = dvp != dv ? at::constant_pad_nd(v_, {0, dvp - dv}) : v_;
            PrefillResult r = RunPrefill(qp, kp, vp, padded, qOffset, kOffset, wantLse, mask);
            if (dvp != dv) r.o = r.o.narrow(-1, 0, dv).contiguous();
            return r;
        }
    }

    std::vector<int64_t> oshape = q_.sizes().vec();
    oshape.back() = v_.size(-1);
    at::Tensor o = at::empty(oshape, q_.options());
    std::vector<int64_t> lshape(q_.sizes().begin(), q_.sizes().end() - 1);
    at::Tensor lse = wantLse ? at::empty(lshape, q_.options().dtype(at::kFloat)) : at::Tensor();
    if (o.numel() == 0) return {o, lse};

    View4 q = MakeView4(q_, "query"), k = MakeView4(k_, "key"), v = MakeView4(v_, "value");
    View4 ov = MakeView4(o, "output");
    void* stream = CurrentStream(q_);

    dtattn_prefill_args a;
    std::memset(&a, 0, sizeof(a));
    a.B = q.B, a.Hq = q.H, a.Hkv = k.H, a.Sq = q.S, a.Sk = k.S, a.D = q.D, a.Dv = v.D;
    a.o = ov.t.data_ptr();
    a.o_stride[0] = ov.sb, a.o_stride[1] = ov.sh, a.o_stride[2] = ov.ss;
    if (wantLse) {
        a.lse = lse.data_ptr<float>();
        a.lse_stride[0] = q.H * q.S, a.lse_stride[1] = q.S;
    }
    a.scale = prm.scale.has_value() ? (float)prm.scale.value() : std::nanf("");  // NaN: 1/sqrt(D)
    a.causal = prm.isCausal ? 1 : 0;
    a.q_offset = qOffset, a.k_offset = kOffset;
    at::Tensor maskf;
    if (mask != nullptr) {
        if (fp8) Throw("attn_mask is not supported with sage_attn_type 'native_fp8'");
        maskf = PrepareMask(*mask, q_, k_, q.B, q.H, q.S, k.S);
        a.mask = maskf.data_ptr<float>();
        for (int i = 0; i < 3; ++i) a.mask_stride[i] = maskf.size(i) > 1 ? maskf.stride(i) : 0;
    }

    a.q = q.t.data_ptr(), a.k = k.t.data_ptr(), a.v = v.t.data_ptr();
    a.q_stride[0] = q.sb, a.q_stride[1] = q.sh, a.q_stride[2] = q.ss;
    a.k_stride[0] = k.sb, a.k_stride[1] = k.sh, a.k_stride[2] = k.ss;
    a.v_stride[0] = v.sb, a.v_stride[1] = v.sh, a.v_stride[2] = v.ss;
    a.dtype = DtypeCode(st);
    a.o_dtype = a.dtype;
    if (fp8) {
        // per-head e4m3fn quantization and fp8 attention in one call; the K/V codes live in its workspace.
        // Head dims below 64 or 128 (multiples of 8, D == Dv) are zero-padded to the next of the two and the
        // output cut back, the rule of the SageAttention package the quantized branch calls
        // (sage_attn_adapter.cc:28-40 hands it q/k/v as they are): zero columns change no score, no per-head
        // maximum and no code, and the default scale stays 1/sqrt(real D).
        const int64_t d = q.D;
        const int64_t dk = d <= 64 ? 64 : 128;
        at::Tensor qp, kp, vp, op;
        if (d == v.D && d % 8 == 0 && d < dk) {
            qp = at::constant_pad_nd(q.t, {0, dk - d}).reshape({q.B, q.H, q.S, dk});  // contiguous: a view
            kp = at::constant_pad_nd(k.t, {0, dk - d}).reshape({k.B, k.H, k.S, dk});
            vp = at::constant_pad_nd(v.t, {0, dk - d}).reshape({v.B, v.H, v.S, dk});
            op = at::empty({q.B, q.H, q.S, dk}, q_.options());
            const at::Tensor* src[3] = {&qp, &kp, &vp};
            int64_t* dst[3] = {a.q_stride, a.k_stride, a.v_stride};
            for (int i = 0; i < 3; ++i)
                for (int j = 0; j < 3; ++j) dst[i][j] = src[i]->stride(j);
            a.q = qp.data_ptr(), a.k = kp.data_ptr(), a.v = vp.data_ptr();
            a.o = op.data_ptr();
            for (int j = 0; j < 3; ++j) a.o_stride[j] = op.stride(j);
            a.D = a.Dv = dk;
            if (!prm.scale.has_value()) a.scale = (float)(1.0 / std::sqrt((double)d));
        }
        const size_t ws = dtattn_prefill_fp8_workspace_size(&a);
        at::Tensor wst = at::empty({(int64_t)std::max<size_t>(ws, 1)}, q_.options().dtype(at::kByte));
        a.workspace = wst.data_ptr();
        a.workspace_bytes = ws;
        Check(dtattn_prefill_fp8(&a, stream), "dtattn_prefill_fp8");
        if (op.defined()) {
            o.view({q.B, q.H, q.S, d}).copy_(op.narrow(3, 0, d));  // o is freshly allocated, contiguous
            return {o, lse};
        }
        if (!ov.t.is_same(o)) o.copy_(ov.t);
        return {o, lse};
    }
    // Workspace for the key blocks of small wide-head grids (zero bytes for every other call).
    at::Tensor wst;
    const size_t ws = dtattn_prefill_workspace_size(&a);
    if (ws > 0) {
        wst = at::empty({(int64_t)ws}, q_.options().dtype(at::kByte));
        a.workspace = wst.data_ptr();
        a.workspace_bytes = ws;
    }
    Check(dtattn_prefill_fwd(&a, stream), "dtattn_prefill_fwd");
    if (!ov.t.is_same(o)) o.copy_(ov.t);
    return {o, lse};
}

}  // namespace

Shape SdpaOp::InferOutputMetaInfo(const Shape& q, const Shape& k, const Shape& v) const {
    if (q.size() < 4 || k.size() < 4 || v.size() < 4) Throw("q, k and v must have at least 4 axes");
    Shape out = q;
    out.back() = v.back();
    return out;
}

PlacementSignature SdpaOp::GetPlacementSignature(size_t numAxis) const {
    if (numAxis < 4) Throw("placement signature needs at least 4 axes");
    PlacementSignature sig;
    const std::vector<bool> opt = {false, false, false, true};
    sig.push_back({{"S(0)", "S(0)", "S(0)", "S(0)"}, {"S(0)"}, opt});
    for (size_t i = 1; i < numAxis - 2; ++i) {
        const std::string s = "S(" + std::to_string(i) + ")";
        sig.push_back({{s, s, s, "R"}, {s}, opt});
    }
    sig.push_back({{"S(2)", "R", "R", "R"}, {"S(2)"}, opt});
    sig.push_back({{"R", "R", "R", "R"}, {"R"}, opt});
    return sig;
}

std::vector<std::string> SdpaOp::MatchPlacements(size_t numAxis, const std::vector<std::string>& inputs) const {
    const PlacementSignature sig = GetPlacementSignature(numAxis);
    for (const PlacementRule& r : sig) {
        if (inputs.size() != r.inputs.size()) continue;
        bool match = true;
        for (size_t i = 0; i < inputs.size() && match; ++i) {
            if (inputs[i].empty() && r.optional[i]) continue;
            match = inputs[i] == r.inputs[i];
        }
        if (match) return r.outputs;
    }
    std::ostringstream os;
    os << "no placement rule for inputs (";
    for (size_t i = 0; i < inputs.size(); ++i) os << (i ? ", " : "") << (inputs[i].empty() ? "-" : inputs[i]);
    os << ")";
    Throw(os.str());
}

int64_t SdpaOp::GetOperatorCost(const Shape& q, const Shape& k, const Shape& v) const {
    if (q.size() < 4) Throw("cost needs at least 4 axes");
    // batch = Shape::Prod(0, NumAxis - 4), an inclusive range (dtorch/api/cpp/shape.cc:65-75).
    int64_t batch = 1;
    for (size_t i = 0; i + 4 <= q.size(); ++i) batch *= q[i];
    const int64_t qHeads = q[q.size() - 3], seqQ = q[q.size() - 2], headDim = q.back();
    const int64_t seqKv = k[k.size() - 2], eV = v.back();
    return 2 * batch * qHeads * seqQ * seqKv * (headDim + eV);
}

int64_t SdpaOp::GetAlgorithmicFlops(const Shape& q, const Shape& k, const Shape& v) const {
    int64_t batch = 1;
    for (size_t i = 0; i + 3 < q.size(); ++i) batch *= q[i];
    const int64_t qHeads = q[q.size() - 3], L = q[q.size() - 2], D = q.back();
    const int64_t S = k[k.size() - 2], eV = v.back();
    int64_t pairs = L * S;
    if (mParam.isCausal) {
        pairs = 0;
        for (int64_t i = 0; i < L; ++i) pairs += std::min<int64_t>(std::max<int64_t>(i + 1, 0), S);
    }
    return 2 * (D + eV) * batch * qHeads * pairs;
}

void SdpaOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 4) Throw("SdpaOp expects 4 inputs {query, key, value, attn_mask}");
    if (!inputs[0].has_value() || !inputs[1].has_value() || !inputs[2].has_value())
        Throw("query, key and value are required");
    const at::Tensor* mask = inputs[3].has_value() && inputs[3]->defined() ? &*inputs[3] : nullptr;
    outputs.push_back(RunPrefill(*inputs[0], *inputs[1], *inputs[2], mParam, 0, 0, false, mask).o);
}

void SdpaWithLseOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 4) Throw("SdpaWithLseOp expects 4 inputs {query, key, value, attn_mask}");
    if (!inputs[0].has_value() || !inputs[1].has_value() || !inputs[2].has_value())
        Throw("query, key and value are required");
    const at::Tensor* mask = inputs[3].has_value() && inputs[3]->defined() ? &*inputs[3] : nullptr;
    PrefillResult r = RunPrefill(*inputs[0], *inputs[1], *inputs[2], mParam, mLseParam.qOffset, mLseParam.kOffset, true, mask);
    outputs.push_back(r.o);
    outputs.push_back(r.lse);
}

void SdpaDecodeOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 4 || !inputs[0] || !inputs[1] || !inputs[2] || !inputs[3])
        Throw("SdpaDecodeOp expects 4 inputs {query, k_cache, v_cache, lengths}");
    const at::Tensor &q = *inputs[0], &kc = *inputs[1], &vc = *inputs[2], &len = *inputs[3];
    CheckDevice({&q, &kc, &vc, &len});
    c10::DeviceGuard guard(q.device());
    if (q.dim() != 4 || kc.dim() != 4 || vc.dim() != 4) Throw("decode tensors must be 4-D [B, H, S, D]");
    if (q.size(2) != 1) Throw("decode query must have one token per sequence ([B, Hq, 1, D])");
    if (kc.sizes() != vc.sizes()) Throw("k_cache and v_cache shapes differ");
    if (q.size(0) != kc.size(0) || q.size(3) != kc.size(3)) Throw("query and cache shapes do not match");
    if (kc.size(1) <= 0 || q.size(1) % kc.size(1) != 0) Throw("number of query heads must be a multiple of kv heads");
    if (len.scalar_type() != at::kInt || len.dim() != 1 || len.size(0) != q.size(0))
        Throw("lengths must be an int32 tensor of shape [B]");
    const c10::ScalarType st = q.scalar_type();
    if (kc.scalar_type() != st || vc.scalar_type() != st) Throw("query and cache dtypes differ");
    if (st != at::kBFloat16 && st != at::kHalf && st != at::kFloat) Throw("decode supports bf16, fp16 and fp32");
    if (mParam.scale.has_value() && !std::isfinite(mParam.scale.value())) Throw("scale must be finite");

    at::Tensor o = at::empty(q.sizes(), q.options());
    at::Tensor lse = at::empty({q.size(0), q.size(1)}, q.options().dtype(at::kFloat));
    if (q.size(0) == 0) {
        outputs.push_back(o);
        outputs.push_back(lse);
        return;
    }
    View4 qv = MakeView4(q, "query"), kv = MakeView4(kc, "k_cache"), vv = MakeView4(vc, "v_cache");
    at::Tensor lc = len.contiguous();
    dtattn_decode_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = qv.t.data_ptr(), a.k_cache = kv.t.data_ptr(), a.v_cache = vv.t.data_ptr();
    a.lengths = lc.data_ptr<int32_t>();
    a.o = o.data_ptr(), a.lse = lse.data_ptr<float>();
    a.B = qv.B, a.Hq = qv.H, a.Hkv = kv.H, a.S_max = kv.S, a.D = qv.D;
    a.q_stride[0] = qv.sb, a.q_stride[1] = qv.sh;
    a.k_stride[0] = kv.sb, a.k_stride[1] = kv.sh, a.k_stride[2] = kv.ss;
    a.v_stride[0] = vv.sb, a.v_stride[1] = vv.sh, a.v_stride[2] = vv.ss;
    a.o_stride[0] = q.size(1) * q.size(3), a.o_stride[1] = q.size(3);
    a.lse_stride[0] = q.size(1);
    a.dtype = DtypeCode(st);
    a.scale = mParam.scale.has_value() ? (float)mParam.scale.value() : std::nanf("");  // NaN: 1/sqrt(D)
    a.chunk = mParam.chunk;
    const size_t ws = dtattn_decode_workspace_size(a.B, a.Hq, a.S_max, a.D, a.chunk);
    at::Tensor wst = at::empty({(int64_t)std::max<size_t>(ws, 1)}, q.options().dtype(at::kByte));
    a.workspace = wst.data_ptr();
    a.workspace_bytes = ws;
    Check(dtattn_decode_splitkv(&a, CurrentStream(q)), "dtattn_decode_splitkv");
    outputs.push_back(o);
    outputs.push_back(lse);
}

namespace {

// A cache written in place: it cannot be copied to fix its layout, so the layout is checked instead.
void CheckCacheLayout(const at::Tensor& c, const char* name) {
    if (c.dim() != 4) Throw(std::string(name) + " must be 4-D");
    if (c.stride(3) != 1) Throw(std::string(name) + " needs a unit stride along D");
    for (int i = 0; i < 3; ++i)
        if ((c.stride(i) * c.element_size()) % 16 != 0)
            Throw(std::string(name) + " strides must be multiples of 16 bytes (it is updated in place)");
    if ((reinterpret_cast<uintptr_t>(c.data_ptr()) & 15u) != 0) Throw(std::string(name) + " must be 16-byte aligned");
}

struct NewTokens {
    View4 k, v;
};

NewTokens CheckNewTokens(const at::Tensor& kn, const at::Tensor& vn, const at::Tensor& kc, int64_t B, int64_t Hkv,
                         int64_t D) {
    if (kn.dim() != 4 || vn.dim() != 4 || kn.sizes() != vn.sizes())
        Throw("k_new and v_new must be 4-D tensors of the same shape [B, Hkv, n_new, D]");
    if (kn.size(0) != B || kn.size(1) != Hkv || kn.size(3) != D)
        Throw("k_new must be [B, Hkv, n_new, D] matching the cache");
    if (kn.scalar_type() != kc.scalar_type() || vn.scalar_type() != kc.scalar_type())
        Throw("new tokens and cache dtypes differ");
    if (kc.scalar_type() != at::kBFloat16 && kc.scalar_type() != at::kHalf && kc.scalar_type() != at::kFloat)
        Throw("the KV cache must be bf16, fp16 or fp32");
    NewTokens r;
    r.k = MakeView4(kn, "k_new");
    r.v = MakeView4(vn, "v_new");
    return r;
}

void CheckLengths(const at::Tensor& len, int64_t B) {
    if (len.scalar_type() != at::kInt || len.dim() != 1 || len.size(0) != B || !len.is_contiguous())
        Throw("lengths must be a contiguous int32 tensor of shape [B] (it is updated in place)");
}

}  // namespace

void KvCacheAppendOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 5 || !inputs[0] || !inputs[1] || !inputs[2] || !inputs[3] || !inputs[4])
        Throw("KvCacheAppendOp expects 5 inputs {k_cache, v_cache, lengths, k_new, v_new}");
    const at::Tensor &kc = *inputs[0], &vc = *inputs[1], &len = *inputs[2], &kn = *inputs[3], &vn = *inputs[4];
    CheckDevice({&kc, &vc, &len, &kn, &vn});
    c10::DeviceGuard guard(kc.device());
    CheckCacheLayout(kc, "k_cache");
    CheckCacheLayout(vc, "v_cache");
    if (kc.sizes() != vc.sizes()) Throw("k_cache and v_cache shapes differ");
    if (vc.scalar_type() != kc.scalar_type()) Throw("k_cache and v_cache dtypes differ");
    const int64_t B = kc.size(0), Hkv = kc.size(1), S_max = kc.size(2), D = kc.size(3);
    CheckLengths(len, B);
    NewTokens nt = CheckNewTokens(kn, vn, kc, B, Hkv, D);
    dtattn_kv_append_args a;
    std::memset(&a, 0, sizeof(a));
    a.k_new = nt.k.t.data_ptr(), a.v_new = nt.v.t.data_ptr();
    a.k_cache = kc.data_ptr(), a.v_cache = vc.data_ptr();
    a.lengths = len.data_ptr<int32_t>();
    a.B = B, a.Hkv = Hkv, a.n_new = kn.size(2), a.S_max = S_max, a.D = D;
    a.k_new_stride[0] = nt.k.sb, a.k_new_stride[1] = nt.k.sh, a.k_new_stride[2] = nt.k.ss;
    a.v_new_stride[0] = nt.v.sb, a.v_new_stride[1] = nt.v.sh, a.v_new_stride[2] = nt.v.ss;
    for (int i = 0; i < 3; ++i) a.k_stride[i] = kc.stride(i), a.v_stride[i] = vc.stride(i);
    a.dtype = DtypeCode(kc.scalar_type());
    Check(dtattn_kv_append(&a, CurrentStream(kc)), "dtattn_kv_append");
    outputs.push_back(kc);
    outputs.push_back(vc);
    outputs.push_back(len);
}

void KvCacheAppendPagedOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 6 || !inputs[0] || !inputs[1] || !inputs[2] || !inputs[3] || !inputs[4] || !inputs[5])
        Throw("KvCacheAppendPagedOp expects 6 inputs {k_pages, v_pages, block_table, lengths, k_new, v_new}");
    const at::Tensor &kp = *inputs[0], &vp = *inputs[1], &bt = *inputs[2], &len = *inputs[3], &kn = *inputs[4],
                     &vn = *inputs[5];
    CheckDevice({&kp, &vp, &bt, &len, &kn, &vn});
    c10::DeviceGuard guard(kp.device());
    CheckCacheLayout(kp, "k_pages");
    CheckCacheLayout(vp, "v_pages");
    if (kp.sizes() != vp.sizes()) Throw("k_pages and v_pages shapes differ");
    if (vp.scalar_type() != kp.scalar_type()) Throw("k_pages and v_pages dtypes differ");
    if (bt.scalar_type() != at::kInt || bt.dim() != 2) Throw("block_table must be an int32 tensor of shape [B, max_pages]");
    const int64_t B = bt.size(0), Hkv = kp.size(1), D = kp.size(3);
    CheckLengths(len, B);
    NewTokens nt = CheckNewTokens(kn, vn, kp, B, Hkv, D);
    at::Tensor btc = bt.stride(1) == 1 ? bt : bt.contiguous();
    dtattn_kv_append_paged_args a;
    std::memset(&a, 0, sizeof(a));
    a.k_new = nt.k.t.data_ptr(), a.v_new = nt.v.t.data_ptr();
    a.k_pages = kp.data_ptr(), a.v_pages = vp.data_ptr();
    a.block_table = btc.data_ptr<int32_t>();
    a.lengths = len.data_ptr<int32_t>();
    a.B = B, a.Hkv = Hkv, a.n_new = kn.size(2), a.D = D;
    a.num_pages = kp.size(0), a.page_size = kp.size(2), a.max_pages = bt.size(1);
    a.k_new_stride[0] = nt.k.sb, a.k_new_stride[1] = nt.k.sh, a.k_new_stride[2] = nt.k.ss;
    a.v_new_stride[0] = nt.v.sb, a.v_new_stride[1] = nt.v.sh, a.v_new_stride[2] = nt.v.ss;
    for (int i = 0; i < 3; ++i) a.k_stride[i] = kp.stride(i), a.v_stride[i] = vp.stride(i);
    a.block_table_stride = btc.stride(0);
    a.dtype = DtypeCode(kp.scalar_type());
    Check(dtattn_kv_append_paged(&a, CurrentStream(kp)), "dtattn_kv_append_paged");
    outputs.push_back(kp);
    outputs.push_back(vp);
    outputs.push_back(len);
}

void SdpaDecodePagedOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 5 || !inputs[0] || !inputs[1] || !inputs[2] || !inputs[3] || !inputs[4])
        Throw("SdpaDecodePagedOp expects 5 inputs {query, k_pages, v_pages, block_table, lengths}");
    const at::Tensor &q = *inputs[0], &kp = *inputs[1], &vp = *inputs[2], &bt = *inputs[3], &len = *inputs[4];
    CheckDevice({&q, &kp, &vp, &bt, &len});
    c10::DeviceGuard guard(q.device());
    if (q.dim() != 4 || kp.dim() != 4 || vp.dim() != 4) Throw("query and page pools must be 4-D");
    if (q.size(2) != 1) Throw("decode query must have one token per sequence ([B, Hq, 1, D])");
    if (kp.sizes() != vp.sizes()) Throw("k_pages and v_pages shapes differ");
    if (q.size(3) != kp.size(3)) Throw("query and page head dims differ");
    if (kp.size(1) <= 0 || q.size(1) % kp.size(1) != 0) Throw("number of query heads must be a multiple of kv heads");
    if (bt.scalar_type() != at::kInt || bt.dim() != 2 || bt.size(0) != q.size(0))
        Throw("block_table must be an int32 tensor of shape [B, max_pages]");
    if (len.scalar_type() != at::kInt || len.dim() != 1 || len.size(0) != q.size(0))
        Throw("lengths must be an int32 tensor of shape [B]");
    const c10::ScalarType st = q.scalar_type();
    if (kp.scalar_type() != st || vp.scalar_type() != st) Throw("query and page dtypes differ");
    if (st != at::kBFloat16 && st != at::kHalf && st != at::kFloat) Throw("decode supports bf16, fp16 and fp32");
    if (mParam.scale.has_value() && !std::isfinite(mParam.scale.value())) Throw("scale must be finite");
    if (kp.stride(3) != 1 || vp.stride(3) != 1) Throw("page pools need a unit stride along D");

    at::Tensor o = at::empty(q.sizes(), q.options());
    at::Tensor lse = at::empty({q.size(0), q.size(1)}, q.options().dtype(at::kFloat));
    if (q.size(0) == 0) {
        outputs.push_back(o);
        outputs.push_back(lse);
        return;
    }
    View4 qv = MakeView4(q, "query");
    at::Tensor btc = bt.stride(1) == 1 ? bt : bt.contiguous();
    at::Tensor lc = len.contiguous();
    dtattn_decode_paged_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = qv.t.data_ptr(), a.k_pages = kp.data_ptr(), a.v_pages = vp.data_ptr();
    a.block_table = btc.data_ptr<int32_t>();
    a.lengths = lc.data_ptr<int32_t>();
    a.o = o.data_ptr(), a.lse = lse.data_ptr<float>();
    a.B = qv.B, a.Hq = qv.H, a.Hkv = kp.size(1), a.D = qv.D;
    a.num_pages = kp.size(0), a.page_size = kp.size(2), a.max_pages = bt.size(1);
    a.q_stride[0] = qv.sb, a.q_stride[1] = qv.sh;
    a.k_stride[0] = kp.stride(0), a.k_stride[1] = kp.stride(1), a.k_stride[2] = kp.stride(2);
    a.v_stride[0] = vp.stride(0), a.v_stride[1] = vp.stride(1), a.v_stride[2] = vp.stride(2);
    a.o_stride[0] = q.size(1) * q.size(3), a.o_stride[1] = q.size(3);
    a.lse_stride[0] = q.size(1);
    a.block_table_stride = btc.stride(0);
    a.dtype = DtypeCode(st);
    a.scale = mParam.scale.has_value() ? (float)mParam.scale.value() : std::nanf("");  // NaN: 1/sqrt(D)
    a.chunk = mParam.chunk;
    const size_t ws = dtattn_decode_paged_workspace_size(a.B, a.Hq, a.max_pages, a.page_size, a.D, a.chunk);
    at::Tensor wst = at::empty({(int64_t)std::max<size_t>(ws, 1)}, q.options().dtype(at::kByte));
    a.workspace = wst.data_ptr();
    a.workspace_bytes = ws;
    Check(dtattn_decode_paged(&a, CurrentStream(q)), "dtattn_decode_paged");
    outputs.push_back(o);
    outputs.push_back(lse);
}

void LseMergeOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.empty() || inputs.size() % 2 != 0) Throw("LseMergeOp expects pairs {O_0, LSE_0, O_1, LSE_1, ...}");
    const int n = (int)inputs.size() / 2;
    if (n > DTATTN_MAX_MERGE_BLOCKS) Throw("too many blocks to merge");
    std::vector<const at::Tensor*> all;
    for (const auto& t : inputs) {
        if (!t.has_value() || !t->defined()) Throw("merge inputs must all be present");
        all.push_back(&*t);
    }
    CheckDevice(all);
    const at::Tensor& o0 = *inputs[0];
    c10::DeviceGuard guard(o0.device());
    const c10::ScalarType st = o0.scalar_type();
    if (DtypeCode(st) < 0 || st == at::kFloat8_e4m3fn) Throw("merge blocks must be bf16, fp16 or fp32");
    std::vector<View4> os;
    std::vector<at::Tensor> lses;
    for (int i = 0; i < n; ++i) {
        const at::Tensor& oi = *inputs[2 * i];
        const at::Tensor& li = *inputs[2 * i + 1];
        if (oi.sizes() != o0.sizes() || oi.scalar_type() != st) Throw("merge blocks must share shape and dtype");
        std::vector<int64_t> ls(o0.sizes().begin(), o0.sizes().end() - 1);
        if (li.sizes().vec() != ls || li.scalar_type() != at::kFloat) Throw("LSE blocks must be fp32 [..., H, S]");
        os.push_back(MakeView4(oi, "O block"));
        lses.push_back(li.contiguous());
    }
    // all blocks must share strides after normalisation
    for (int i = 1; i < n; ++i)
        if (os[i].sb != os[0].sb || os[i].sh != os[0].sh || os[i].ss != os[0].ss) {
            for (auto& v : os) v = MakeView4(v.t.contiguous(), "O block");
            break;
        }
    c10::ScalarType ost = st;
    if (mParam.outKind.has_value()) {
        switch (*mParam.outKind) {
            case DTATTN_BF16: ost = at::kBFloat16; break;
            case DTATTN_FP16: ost = at::kHalf; break;
            case DTATTN_FP32: ost = at::kFloat; break;
            default: Throw("merge output must be bf16, fp16 or fp32");
        }
    }
    at::Tensor o = at::empty(o0.sizes(), o0.options().dtype(ost));
    std::vector<int64_t> ls(o0.sizes().begin(), o0.sizes().end() - 1);
    at::Tensor lse = at::empty(ls, o0.options().dtype(at::kFloat));
    if (o.numel() == 0) {
        outputs.push_back(o);
        outputs.push_back(lse);
        return;
    }
    View4 ov = MakeView4(o, "output");
    dtattn_merge_args a;
    std::memset(&a, 0, sizeof(a));
    a.n_blocks = n;
    for (int i = 0; i < n; ++i) {
        a.o_blocks[i] = os[i].t.data_ptr();
        a.lse_blocks[i] = lses[i].data_ptr<float>();
    }
    a.B = ov.B, a.H = ov.H, a.S = ov.S, a.D = ov.D;
    a.block_o_stride[0] = os[0].sb, a.block_o_stride[1] = os[0].sh, a.block_o_stride[2] = os[0].ss;
    a.block_lse_stride[0] = ov.H * ov.S, a.block_lse_stride[1] = ov.S;
    a.block_dtype = DtypeCode(st);
    a.o = ov.t.data_ptr();
    a.lse = lse.data_ptr<float>();
    a.o_stride[0] = ov.sb, a.o_stride[1] = ov.sh, a.o_stride[2] = ov.ss;
    a.lse_stride[0] = ov.H * ov.S, a.lse_stride[1] = ov.S;
    a.o_dtype = DtypeCode(ost);
    Check(dtattn_lse_merge(&a, CurrentStream(o0)), "dtattn_lse_merge");
    outputs.push_back(o);
    outputs.push_back(lse);
}

LseMergeParam LseMergeOp::ParamFor(std::optional<c10::ScalarType> outDtype) {
    if (!outDtype.has_value()) return LseMergeParam();
    const int32_t code = DtypeCode(*outDtype);
    if (code != DTATTN_BF16 && code != DTATTN_FP16 && code != DTATTN_FP32)
        Throw("merge output must be bf16, fp16 or fp32");
    return LseMergeParam(code);
}

void Fp8QuantizeOp::Compute(const TorchTensorOptArray& inputs, TorchTensorArray& outputs) const {
    if (inputs.size() != 1 || !inputs[0] || !inputs[0]->defined()) Throw("Fp8QuantizeOp expects {x}");
    const at::Tensor& x_ = *inputs[0];
    CheckDevice({&x_});
    c10::DeviceGuard guard(x_.device());
    const int32_t code = DtypeCode(x_.scalar_type());
    if (code != DTATTN_BF16 && code != DTATTN_FP16 && code != DTATTN_FP32) Throw("quantize takes bf16, fp16 or fp32");
    View4 x = MakeView4(x_, "x");
    at::Tensor codes = at::empty(x_.sizes(), x_.options().dtype(at::kFloat8_e4m3fn));
    std::vector<int64_t> ds(x_.sizes().begin(), x_.sizes().end() - 2);
    at::Tensor desc = at::empty(ds, x_.options().dtype(at::kFloat));
    if (codes.numel() > 0) {
        const size_t ws = dtattn_fp8_quantize_workspace_size(x.B, x.H, x.S, x.D);
        at::Tensor wst = at::empty({(int64_t)std::max<size_t>(ws, 1)}, x_.options().dtype(at::kByte));
        const int64_t strides[3] = {x.sb, x.sh, x.ss};
        Check(dtattn_fp8_quantize_per_head(x.t.data_ptr(), code, x.B, x.H, x.S, x.D, strides, codes.data_ptr(),
                                           desc.data_ptr<float>(), wst.data_ptr(), ws, CurrentStream(x_)),
              "dtattn_fp8_quantize_per_head");
    }
    outputs.push_back(codes);
    outputs.push_back(desc);
}

DevicePeaks GetDevicePeaks(int device) {
    dtattn_device_peaks pk;
    Check(dtattn_get_device_peaks(device, &pk), "dtattn_get_device_peaks");
    return {pk.cu_count, pk.clock_hz, pk.bf16_flops, pk.fp8_flops, pk.hbm_bytes_per_s, std::string(pk.arch)};
}

}  // namespace core
}  // namespace dtorch_amd
