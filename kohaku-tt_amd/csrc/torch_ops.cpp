// torch op layer: the reference's op surface on the CUDA/HIP dispatch keys, calling the
// C ABI (include/kohakutt_amd.h) into the gfx950 kernels.
//
// Reference boundary (src/kohakutt_native/csrc/aten):
//   attention/aten_attention.cpp:959-974  aten::_fused_sdp_choice (+ its dispatch stub),
//       aten::_scaled_dot_product_fused_attention_overrideable (+ _backward) on PrivateUse1;
//   nn/aten_norm.cpp:797-811  aten::native_layer_norm, aten::rms_norm (AutogradPrivateUse1);
//   nn/aten_fused.cpp:114-127  ktt::rms_norm(x, weight, bias, eps);
//   attention/aten_varlen.cpp:323-349  ktt::_sdpa_varlen;
//   attention/aten_attention.cpp:935-952  ktt::sdpa_refusal.
// Here the same names are registered on CUDA / AutogradCUDA (ROCm tensors use the CUDA
// key).  torch's scaled_dot_product_attention calls the _fused_sdp_choice dispatch stub
// directly, so the stub's CUDA entry is replaced too; calls the kernels do not take keep
// torch's own choice (at::cuda::_fused_sdp_choice), and norms they do not take go to
// torch's own CUDA kernels.
#include <ATen/ATen.h>
#include <ATen/native/transformers/attention.h>
#include <ATen/ops/_fused_sdp_choice_cuda_dispatch.h>
#include <ATen/ops/native_layer_norm_backward_cuda_dispatch.h>
#include <ATen/ops/native_layer_norm_cuda_dispatch.h>
#include <ATen/ops/rms_norm_compositeimplicitautograd_dispatch.h>
#include <ATen/ops/scaled_dot_product_attention_compositeimplicitautograd_dispatch.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>

#include "../../include/kohakutt_amd.h"

namespace kta {
namespace {

using at::Tensor;
using std::optional;

constexpr double kMaskedLogit = -5e5;

bool env_on(const char* name) {
    const char* v = std::getenv(name);
    return !(v && v[0] == '0');
}

// KMI_ATTENTION=0 / KMI_NORMS=0 (read at load) leave the ops to torch; ktt::_set_enabled
// switches them at run time.
std::atomic<bool> g_attention{env_on("KMI_ATTENTION")};
std::atomic<bool> g_norms{env_on("KMI_NORMS")};
// KMI_PITCHED_OUT=0 (read at load) keeps the attention output dense for head-view inputs.
const bool g_pitched_out = env_on("KMI_PITCHED_OUT");
// Calls the kernels took, per family (ktt::counters).
std::atomic<int64_t> g_attn_calls{0}, g_norm_calls{0}, g_attn_declined{0}, g_attn_bwd_calls{0},
    g_norm_bwd_calls{0};

void check(int status, const char* what) {
    TORCH_CHECK(status == KMI_OK, "kohakutt_amd: ", what, " failed (", status, "): ", kmi_last_error());
}

int code_of(at::ScalarType t) {
    switch (t) {
        case at::kBFloat16: return KMI_BF16;
        case at::kHalf: return KMI_F16;
        case at::kFloat: return KMI_F32;
        case at::kBool: return KMI_BOOL;
        default: return 0;
    }
}

void* stream_of(const Tensor& t) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

// ---------------------------------------------------------------- attention

bool mask_given(const optional<Tensor>& m) { return m.has_value() && m->defined(); }

// Head dims the ops take: up to 256.  The kernels read 16-byte rows (multiples of 8) and
// pad to whole 32-wide MFMA blocks with zeros in registers; other head dims are padded
// with zero columns to a multiple of 8 here (pad_head) and the outputs narrowed back, as
// the reference's flash pads any head dim to whole tiles (aten_attention.cpp:57-60).
bool head_dim_ok(int64_t d) { return d >= 1 && d <= 256; }

// `t` with its last dim padded by zero columns to a multiple of 8 (`t` itself when it is
// one already).  Zero columns of q and k add nothing to the scores and those of v only
// fill output columns that are dropped.
Tensor pad_head(const Tensor& t) {
    const int64_t d = t.size(-1);
    return d % 8 == 0 ? t : at::constant_pad_nd(t, {0, 8 - d % 8}, 0);
}

// Tensors whose data the kernels can read: not meta, not fake / functional wrappers
// (torch.compile and export trace with those; they must take the composite route).
bool real_data(const Tensor& t) {
    constexpr c10::DispatchKeySet traced({c10::DispatchKey::Python, c10::DispatchKey::PythonTLSSnapshot,
                                          c10::DispatchKey::Functionalize});
    return t.defined() && !t.is_meta() && (t.key_set() & traced).empty() && t.has_storage();
}

// Why the kernels do not take SDPA(q, k, v, mask, ...), or "" when they do.  The
// conditions of the reference's fused_refusal (aten_attention.cpp:62-127): 4-D non-empty
// q/k/v of one float type, fp32 only without gradients (cast to bf16 at entry), no
// dropout, one head dim, K/V heads dividing Q heads, causal without a mask, a mask that
// broadcasts to [B, H, Sq, Sk]; plus what these kernels cover: GPU tensors (meta tensors
// answer by their sizes and dtypes), head dims up to 256, bool / bf16 / f16 / f32 / f64
// masks.
std::string sdpa_refusal_impl(const Tensor& q, const Tensor& k, const Tensor& v, const optional<Tensor>& mask,
                              double dropout_p, bool is_causal) {
    if (!g_attention.load()) return "kohakutt_amd attention is switched off";
    const bool grads = q.requires_grad() || k.requires_grad() || v.requires_grad();
    for (const Tensor* t : {&q, &k, &v}) {
        const auto st = t->scalar_type();
        if (!(t->is_cuda() || t->is_meta()) || t->dim() != 4 || t->numel() == 0 ||
            !(st == at::kBFloat16 || st == at::kHalf || (st == at::kFloat && !grads)) ||
            st != q.scalar_type() || t->device() != q.device())
            return "q, k and v must be non-empty 4-D bf16 / fp16 GPU tensors (fp32 without gradients)";
    }
    if (dropout_p != 0.0) return "dropout";
    const int64_t d = q.size(3);
    if (k.size(3) != d || v.size(3) != d) return "q, k and v need one head dim";
    if (!head_dim_ok(d)) return "head dim must be at most 256";
    if (k.size(0) != q.size(0) || v.size(0) != q.size(0) || v.size(1) != k.size(1) || q.size(1) % k.size(1) != 0 ||
        v.size(2) != k.size(2))
        return "q, k and v shapes do not match (K / V heads must divide Q heads)";
    if (is_causal && mask.has_value()) return "causal takes no mask";
    if (mask_given(mask)) {
        const Tensor& m = *mask;
        if (m.device() != q.device()) return "the mask must be on q's device";
        if (m.dim() > 4) return "the mask must broadcast to [B, H, Sq, Sk]";
        const int64_t full[4] = {q.size(0), q.size(1), q.size(2), k.size(2)};
        for (int64_t i = 0; i < m.dim(); ++i) {
            const int64_t s = m.size(m.dim() - 1 - i);
            if (s != 1 && s != full[3 - i]) return "the mask must broadcast to [B, H, Sq, Sk]";
        }
        const auto mt = m.scalar_type();
        if (!(mt == at::kBool || mt == at::kBFloat16 || mt == at::kHalf || mt == at::kFloat || mt == at::kDouble))
            return "mask dtype must be bool or floating";
    }
    return "";
}

// q/k/v as the kernels read them: last-dim stride 1, 16-byte aligned, strides multiples
// of 8 elements, the sequence (row) stride within [0, 2^24]; anything else is copied once.
Tensor kernel_operand(const Tensor& t, int64_t row_dim) {
    bool ok = t.stride(-1) == 1 && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 && t.stride(row_dim) >= 0 &&
              t.stride(row_dim) <= (1 << 24);
    for (int64_t i = 0; ok && i + 1 < t.dim(); ++i) ok = t.stride(i) % 8 == 0;
    return ok ? t : t.contiguous();
}

// The mask as a 4-D strided view broadcast to [B, H, Sq, Sk]; every dim of size 1 gets
// stride 0 (the kernels recognise a key-only padding mask by zero head and query strides).
Tensor mask_operand(const Tensor& m, const Tensor& q, int64_t sk) {
    Tensor x = m;
    if (x.scalar_type() == at::kDouble) x = x.to(at::kFloat);
    while (x.dim() < 4) x = x.unsqueeze(0);
    x = x.expand({q.size(0), q.size(1), q.size(2), sk});
    std::vector<int64_t> strides(x.strides().begin(), x.strides().end());
    for (int i = 0; i < 4; ++i)
        if (x.size(i) == 1) strides[i] = 0;
    return x.as_strided(x.sizes(), strides);
}

struct AttnOut {
    Tensor out, lse;
};

// `t` [B, H, S, D] as a head view of a [B, S, C] row-major projection (a fused qkv or a
// separate one): heads adjacent within a row of pitch C (the reference's head_view,
// core/torch/views.cpp:808-830, without its 32-element tile alignment).
bool head_view(const Tensor& t) {
    if (t.dim() != 4 || t.numel() == 0 || t.stride(3) != 1) return false;
    const int64_t b = t.size(0), h = t.size(1), s = t.size(2), d = t.size(3), c = t.stride(2);
    return (h == 1 || t.stride(1) == d) && c >= h * d && (b == 1 || t.stride(0) == s * c);
}

// The pitched route's output (aten_attention.cpp:605-628): with q, k and v head views of
// [B, S, C] projections, no mask and no gradients, the output is a [B, H, S, D] view of a
// dense [B, S, H D] tensor, so that transposing it back to the projection layout is free.
Tensor attention_output(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, bool masked, const Tensor& q) {
    const int64_t B = q.size(0), H = q.size(1), Sq = q.size(2), D = q.size(3);
    const bool pitched = g_pitched_out && !masked && q_in.size(3) == D && q_in.scalar_type() == at::kBFloat16 &&
                         !q_in.requires_grad() &&
                         !k_in.requires_grad() && !v_in.requires_grad() && head_view(q_in) && head_view(k_in) &&
                         head_view(v_in);
    if (!pitched) return at::empty({B, H, Sq, D}, q.options());
    return at::empty({B, Sq, H * D}, q.options()).as_strided({B, H, Sq, D}, {Sq * H * D, D, H * D, 1});
}

AttnOut run_attention(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, const optional<Tensor>& mask,
                      bool is_causal, optional<double> scale, const Tensor* key_lengths = nullptr) {
    c10::DeviceGuard guard(q_in.device());
    Tensor q = q_in, k = k_in, v = v_in;
    const bool fp32 = q.scalar_type() == at::kFloat;
    if (fp32) {
        // The reference casts fp32 (without gradients) to bf16 at entry and the output
        // back (aten_attention.cpp:400-415).
        q = q.to(at::kBFloat16);
        k = k.to(at::kBFloat16);
        v = v.to(at::kBFloat16);
    }
    const int64_t D0 = q.size(3);  // the caller's head dim (the default scale's)
    q = kernel_operand(pad_head(q), 2);
    k = kernel_operand(pad_head(k), 2);
    v = kernel_operand(pad_head(v), 2);
    const int64_t B = q.size(0), H = q.size(1), Sq = q.size(2), D = q.size(3);
    const int64_t Hk = k.size(1), Sk = k.size(2);
    Tensor out = attention_output(q_in, k_in, v_in, mask_given(mask), q);
    Tensor lse = at::empty({B, H, Sq}, q.options().dtype(at::kFloat));
    kmi_attn_args a{};
    a.q = q.data_ptr();
    a.k = k.data_ptr();
    a.v = v.data_ptr();
    a.out = out.data_ptr();
    a.lse = lse.data_ptr<float>();
    a.dtype = code_of(q.scalar_type());
    a.causal = is_causal ? 1 : 0;
    a.batch = B;
    a.heads_q = H;
    a.heads_kv = Hk;
    a.seq_q = Sq;
    a.seq_k = Sk;
    a.head_dim = D;
    for (int i = 0; i < 3; ++i) {
        a.q_stride[i] = q.stride(i);
        a.k_stride[i] = k.stride(i);
        a.v_stride[i] = v.stride(i);
        a.o_stride[i] = out.stride(i);
        a.lse_stride[i] = lse.stride(i);
    }
    a.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(D0));
    Tensor m;
    if (mask_given(mask)) {
        m = mask_operand(*mask, q, Sk);
        a.mask = m.data_ptr();
        a.mask_dtype = code_of(m.scalar_type());
        a.mask_mode = KMI_MASK_STRIDED;
        for (int i = 0; i < 4; ++i) a.mask_stride[i] = m.stride(i);
    }
    if (key_lengths) a.key_lengths = key_lengths->data_ptr<int32_t>();
    size_t ws = 0;
    check(kmi_attn_workspace_bytes(&a, &ws), "kmi_attn_workspace_bytes");
    Tensor work;
    if (ws) work = at::empty({static_cast<int64_t>(ws)}, q.options().dtype(at::kByte));
    check(kmi_attn_fwd(&a, ws ? work.data_ptr() : nullptr, ws, stream_of(q)), "kmi_attn_fwd");
    g_attn_calls.fetch_add(1);
    if (D0 != D) out = out.narrow(3, 0, D0);
    if (fp32) out = out.to(at::kFloat);
    return {out, lse};
}

using SdpaResult = std::tuple<Tensor, Tensor, Tensor, Tensor, c10::SymInt, c10::SymInt, Tensor, Tensor, Tensor>;

// aten::_scaled_dot_product_fused_attention_overrideable on CUDA (the reference's
// tt_sdpa_overrideable, aten_attention.cpp:389-713): the kernels, or the math route for
// calls they refuse.  The log-sum-exp is always written (fp32, natural log).
SdpaResult sdpa_overrideable(const Tensor& q, const Tensor& k, const Tensor& v, const optional<Tensor>& attn_bias,
                             double dropout_p, bool is_causal, bool return_debug_mask, optional<double> scale) {
    (void)return_debug_mask;
    const int64_t sq = q.size(2), sk = k.size(2);
    const std::string why = sdpa_refusal_impl(q, k, v, attn_bias, dropout_p, is_causal);
    Tensor out, lse;
    if (why.empty()) {
        auto r = run_attention(q, k, v, attn_bias, is_causal, scale);
        out = r.out;
        lse = r.lse;
    } else {
        g_attn_declined.fetch_add(1);
        out = std::get<0>(at::_scaled_dot_product_attention_math(q, k, v, attn_bias, dropout_p, is_causal,
                                                                  std::nullopt, scale, q.size(1) != k.size(1)));
        // No statistics off the kernels: a broadcast (stride 0) placeholder of the right
        // shape, which the backward recognises (kernel-written lse is contiguous).
        lse = at::empty({1}, q.options().dtype(at::kFloat)).expand({q.size(0), q.size(1), sq});
    }
    auto seed = at::empty({}, at::dtype(at::kLong));
    auto offset = at::empty({}, at::dtype(at::kLong));
    return {out, lse, Tensor(), Tensor(), c10::SymInt(sq), c10::SymInt(sk), seed, offset, Tensor()};
}

// The flash backward (kmi_attn_bwd) takes calls whose forward ran the kernels -- their
// lse is a contiguous fp32 [B, H, Sq] (a declined forward leaves a stride-0 one) -- with
// the forward's mask, if any.
bool flash_backward_takes(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& attn_bias,
                          const Tensor& out, const Tensor& lse, const Tensor& grad_out) {
    if (!g_attention.load() || !lse.defined()) return false;
    const auto st = q.scalar_type();
    if (!(st == at::kBFloat16 || st == at::kHalf) || k.scalar_type() != st || v.scalar_type() != st ||
        grad_out.scalar_type() != st || out.scalar_type() != st)
        return false;
    if (q.dim() != 4 || k.dim() != 4 || v.dim() != 4 || !q.is_cuda()) return false;
    const int64_t d = q.size(3);
    if (!head_dim_ok(d) || k.size(3) != d || v.size(3) != d || q.size(1) % k.size(1) != 0) return false;
    if (attn_bias.defined()) {
        // The forward's mask: it took bool or floating masks that broadcast to [B, H, Sq, Sk].
        if (attn_bias.device() != q.device() || attn_bias.dim() > 4) return false;
        const auto mt = attn_bias.scalar_type();
        if (!(mt == at::kBool || mt == at::kBFloat16 || mt == at::kHalf || mt == at::kFloat || mt == at::kDouble))
            return false;
        const int64_t full[4] = {q.size(0), q.size(1), q.size(2), k.size(2)};
        for (int64_t i = 0; i < attn_bias.dim(); ++i) {
            const int64_t sz = attn_bias.size(attn_bias.dim() - 1 - i);
            if (sz != 1 && sz != full[3 - i]) return false;
        }
    }
    return lse.scalar_type() == at::kFloat && lse.dim() == 3 && lse.size(0) == q.size(0) &&
           lse.size(1) == q.size(1) && lse.size(2) == q.size(2) && lse.stride(2) == 1 && lse.stride(1) >= q.size(2);
}

// The operands of one kmi_attn_bwd call.  Dense: [B, H, S, D] tensors, lse [B, H, Sq], an
// optional mask broadcast to [B, H, Sq, Sk].  Varlen (cu_q defined): [T, H, D] tensors,
// lse [H, Tq], device int32 offsets, an optional [Tk] key mask or block-packed mask.
struct BwdCall {
    Tensor grad, q, k, v, out, lse;
    Tensor mask;      // strided (dense [B, H, Sq, Sk] view or varlen [Tk]) or packed
    bool packed = false;
    Tensor mask_offsets;  // varlen packed masks: device int64 [n + 1] block offsets (optional)
    Tensor cu_q, cu_k;
    Tensor key_lengths;  // dense: int32 [B] key counts (optional)
    int64_t nseq = 0, max_q = 0, max_k = 0;
    bool causal = false;
    double scale = 0.0;
};

std::tuple<Tensor, Tensor, Tensor> run_backward(const BwdCall& c) {
    const bool varlen = c.cu_q.defined();
    const int64_t row_dim = varlen ? 0 : 2;
    // Head dims that are not multiples of 8 run zero-padded (pad_head); the gradients are
    // narrowed back below.
    const Tensor q = kernel_operand(pad_head(c.q), row_dim), k = kernel_operand(pad_head(c.k), row_dim),
                 v = kernel_operand(pad_head(c.v), row_dim);
    const Tensor go = kernel_operand(pad_head(c.grad), row_dim);
    const Tensor o = kernel_operand(pad_head(c.out), row_dim);
    Tensor dq = at::empty(q.sizes(), q.options());
    Tensor dk = at::empty(k.sizes(), k.options());
    Tensor dv = at::empty(v.sizes(), v.options());
    kmi_attn_bwd_args a{};
    a.q = q.data_ptr();
    a.k = k.data_ptr();
    a.v = v.data_ptr();
    a.out = o.data_ptr();
    a.grad_out = go.data_ptr();
    a.lse = c.lse.data_ptr<float>();
    a.grad_q = dq.data_ptr();
    a.grad_k = dk.data_ptr();
    a.grad_v = dv.data_ptr();
    a.dtype = code_of(q.scalar_type());
    a.causal = c.causal ? 1 : 0;
    const int64_t D = q.size(-1);
    a.head_dim = D;
    a.head_dim_v = v.size(-1);
    if (varlen) {
        a.batch = c.nseq;
        a.heads_q = q.size(1);
        a.heads_kv = k.size(1);
        a.seq_q = std::max<int64_t>(1, c.max_q);
        a.seq_k = std::max<int64_t>(1, c.max_k);
        a.cu_seqlens_q = c.cu_q.data_ptr<int32_t>();
        a.cu_seqlens_k = c.cu_k.data_ptr<int32_t>();
        a.total_q = q.size(0);
        a.total_k = k.size(0);
        // [T, H, D]: stride[1] heads, stride[2] tokens; lse [H, Tq].
        const Tensor* ts[] = {&q, &k, &v, &o, &go, &dq, &dk, &dv};
        int64_t* ss[] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride, a.do_stride, a.dq_stride, a.dk_stride,
                         a.dv_stride};
        for (int i = 0; i < 8; ++i) {
            ss[i][0] = 0;
            ss[i][1] = ts[i]->stride(1);
            ss[i][2] = ts[i]->stride(0);
        }
        a.lse_stride[0] = 0;
        a.lse_stride[1] = c.lse.stride(0);
        a.lse_stride[2] = c.lse.stride(1);
    } else {
        a.batch = q.size(0);
        a.heads_q = q.size(1);
        a.heads_kv = k.size(1);
        a.seq_q = q.size(2);
        a.seq_k = k.size(2);
        for (int i = 0; i < 3; ++i) {
            a.q_stride[i] = q.stride(i);
            a.k_stride[i] = k.stride(i);
            a.v_stride[i] = v.stride(i);
            a.o_stride[i] = o.stride(i);
            a.do_stride[i] = go.stride(i);
            a.dq_stride[i] = dq.stride(i);
            a.dk_stride[i] = dk.stride(i);
            a.dv_stride[i] = dv.stride(i);
            a.lse_stride[i] = c.lse.stride(i);
        }
    }
    a.scale = c.scale;
    if (c.key_lengths.defined()) a.key_lengths = c.key_lengths.data_ptr<int32_t>();
    if (c.mask.defined()) {
        a.mask = c.mask.data_ptr();
        a.mask_dtype = code_of(c.mask.scalar_type());
        if (c.packed) {
            a.mask_mode = KMI_MASK_PACKED;
            a.mask_numel = c.mask.numel();
            if (c.mask_offsets.defined()) a.mask_offsets = c.mask_offsets.data_ptr<int64_t>();
        } else {
            a.mask_mode = KMI_MASK_STRIDED;
            if (varlen) {
                a.mask_stride[3] = c.mask.stride(0);  // a [Tk] key mask
            } else {
                for (int i = 0; i < 4; ++i) a.mask_stride[i] = c.mask.stride(i);
            }
        }
    }
    size_t ws = 0;
    check(kmi_attn_bwd_workspace_bytes(&a, &ws), "kmi_attn_bwd_workspace_bytes");
    Tensor work = at::empty({static_cast<int64_t>(ws)}, q.options().dtype(at::kByte));
    check(kmi_attn_bwd(&a, work.data_ptr(), ws, stream_of(q)), "kmi_attn_bwd");
    g_attn_bwd_calls.fetch_add(1);
    return {dq.narrow(-1, 0, c.q.size(-1)), dk.narrow(-1, 0, c.k.size(-1)), dv.narrow(-1, 0, c.v.size(-1))};
}

std::tuple<Tensor, Tensor, Tensor> flash_backward(const Tensor& grad_out, const Tensor& q, const Tensor& k,
                                                  const Tensor& v, const Tensor& out, const Tensor& lse,
                                                  const Tensor& attn_bias, bool is_causal, optional<double> scale) {
    BwdCall c;
    c.grad = grad_out;
    c.q = q;
    c.k = k;
    c.v = v;
    c.out = out;
    c.lse = lse;
    if (attn_bias.defined()) c.mask = mask_operand(attn_bias, q, k.size(2));
    c.causal = is_causal;
    c.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(q.size(3)));
    return run_backward(c);
}

// ktt::_sdpa_flash_backward(grad, q, k, v, out, lse, is_causal, scale): the flash
// backward called directly (what the overrideable backward runs for unmasked calls).
std::tuple<Tensor, Tensor, Tensor> sdpa_flash_backward_op(const Tensor& grad, const Tensor& q, const Tensor& k,
                                                          const Tensor& v, const Tensor& out, const Tensor& lse,
                                                          bool is_causal, optional<double> scale) {
    TORCH_CHECK(flash_backward_takes(q, k, v, Tensor(), out, lse, grad),
                "kohakutt_amd: _sdpa_flash_backward needs bf16 / fp16 [B, H, S, D] GPU tensors of one dtype, "
                "a head dim that is a multiple of 8 up to 256, K/V heads dividing Q heads and the forward's "
                "contiguous fp32 lse [B, H, Sq]");
    TORCH_CHECK(grad.sizes() == q.sizes() && out.sizes() == q.sizes(),
                "kohakutt_amd: _sdpa_flash_backward grad and out must be shaped as q");
    c10::DeviceGuard guard(q.device());
    return flash_backward(grad, q, k, v, out, lse, Tensor(), is_causal, scale);
}

// The math backward of the overrideable op, in fp32 (the reference's
// tt_sdpa_overrideable_backward recomputes through math off its training route,
// aten_attention.cpp:716-812).  Probabilities follow the forward's mask semantics.
std::tuple<Tensor, Tensor, Tensor, Tensor> sdpa_overrideable_backward(
    const Tensor& grad_out, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& attn_bias,
    std::array<bool, 4> grad_input_mask, const Tensor& out, const Tensor& logsumexp, const Tensor& cum_seq_q,
    const Tensor& cum_seq_k, c10::SymInt max_q, c10::SymInt max_k, double dropout_p, bool is_causal,
    const Tensor& philox_seed, const Tensor& philox_offset, optional<double> scale) {
    (void)cum_seq_q, (void)cum_seq_k, (void)max_q, (void)max_k;
    (void)philox_seed, (void)philox_offset;
    TORCH_CHECK(dropout_p == 0.0, "kohakutt_amd: attention backward takes no dropout");
    c10::DeviceGuard guard(q.device());
    // A mask that asks for its own gradient takes the fp32 recompute (the kernels give none).
    const bool bias_grad = grad_input_mask[3] && attn_bias.defined() && attn_bias.is_floating_point();
    if (!bias_grad && flash_backward_takes(q, k, v, attn_bias, out, logsumexp, grad_out)) {
        auto g = flash_backward(grad_out, q, k, v, out, logsumexp, attn_bias, is_causal, scale);
        return {grad_input_mask[0] ? std::get<0>(g) : Tensor(), grad_input_mask[1] ? std::get<1>(g) : Tensor(),
                grad_input_mask[2] ? std::get<2>(g) : Tensor(), Tensor()};
    }
    const int64_t H = q.size(1), Hk = k.size(1), Sq = q.size(2), Sk = k.size(2), D = q.size(3);
    const int64_t G = H / Hk;
    const double s = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(D));
    Tensor qf = q.to(at::kFloat), kf = k.to(at::kFloat), vf = v.to(at::kFloat), go = grad_out.to(at::kFloat);
    if (G > 1) {
        kf = kf.repeat_interleave(G, 1);
        vf = vf.repeat_interleave(G, 1);
    }
    Tensor logits = at::matmul(qf, kf.transpose(-2, -1).contiguous()) * s;
    if (attn_bias.defined()) {
        Tensor add = attn_bias.scalar_type() == at::kBool
                         ? at::zeros(attn_bias.sizes(), logits.options()).masked_fill(attn_bias.logical_not(), kMaskedLogit)
                         : attn_bias.to(at::kFloat).clamp_min(kMaskedLogit);
        logits = logits + add;
    }
    if (is_causal) {
        auto keep = at::ones({Sq, Sk}, q.options().dtype(at::kBool)).tril();
        logits = logits.masked_fill(keep.logical_not(), -INFINITY);
    }
    Tensor p = at::softmax(logits, -1);
    Tensor dv = at::matmul(p.transpose(-2, -1).contiguous(), go);
    Tensor dp = at::matmul(go, vf.transpose(-2, -1).contiguous());
    Tensor ds = p * (dp - (dp * p).sum(-1, true));
    Tensor dq = at::matmul(ds, kf) * s;
    Tensor dk = at::matmul(ds.transpose(-2, -1).contiguous(), qf) * s;
    if (G > 1) {
        dk = dk.view({q.size(0), Hk, G, Sk, D}).sum(2);
        dv = dv.view({q.size(0), Hk, G, Sk, D}).sum(2);
    }
    Tensor dbias;
    if (grad_input_mask[3] && attn_bias.defined() && attn_bias.is_floating_point()) {
        dbias = ds.sum_to_size(attn_bias.sizes()).to(attn_bias.scalar_type());
    }
    return {grad_input_mask[0] ? dq.to(q.scalar_type()) : Tensor(),
            grad_input_mask[1] ? dk.to(k.scalar_type()) : Tensor(),
            grad_input_mask[2] ? dv.to(v.scalar_type()) : Tensor(), dbias};
}

// The _fused_sdp_choice dispatch stub's CUDA entry and the aten op: overrideable when
// the kernels take the call (and torch.nn.attention.sdpa_kernel allows that backend),
// torch's own choice otherwise (the reference's tt_fused_sdp_choice,
// aten_attention.cpp:194-219).
int64_t fused_sdp_choice(const Tensor& q, const Tensor& k, const Tensor& v, const optional<Tensor>& mask,
                         double dropout_p, bool is_causal, optional<double> scale, bool enable_gqa) {
    if (at::globalContext().userEnabledOverrideableSDP() &&
        sdpa_refusal_impl(q, k, v, mask, dropout_p, is_causal).empty())
        return static_cast<int64_t>(at::SDPBackend::overrideable);
    return at::cuda::_fused_sdp_choice(q, k, v, mask, dropout_p, is_causal, scale, enable_gqa);
}

// aten::scaled_dot_product_attention on AutogradCUDA: a bool mask reaches the kernels as
// it is (they read bool keep-masks natively), where torch's composite would first turn it
// into an additive mask of the query dtype -- three device kernels per call, about 6 us of
// a config 3 decode.  Everything else (gradients, float masks, no mask, calls the kernels
// do not take, an sdpa_kernel scope without the overrideable backend) runs torch's
// composite, which routes through _fused_sdp_choice as before.  Like the reference's
// route, enable_gqa is not required: K/V heads dividing Q heads is enough.
Tensor sdpa_entry(const Tensor& q, const Tensor& k, const Tensor& v, const optional<Tensor>& mask, double dropout_p,
                  bool is_causal, optional<double> scale, bool enable_gqa) {
    const bool grads = at::GradMode::is_enabled() && (q.requires_grad() || k.requires_grad() || v.requires_grad());
    // Traced (fake / functional) and meta tensors take the composite, which the tracer
    // understands; only tensors with device data reach the kernels from here.
    const bool data = real_data(q) && real_data(k) && real_data(v) && (!mask_given(mask) || real_data(*mask));
    if (!grads && data && mask_given(mask) && mask->scalar_type() == at::kBool &&
        at::globalContext().userEnabledOverrideableSDP() &&
        sdpa_refusal_impl(q, k, v, mask, dropout_p, is_causal).empty()) {
        at::AutoDispatchBelowADInplaceOrView below;
        return run_attention(q, k, v, mask, is_causal, scale).out;
    }
    return at::compositeimplicitautograd::scaled_dot_product_attention(q, k, v, mask, dropout_p, is_causal, scale,
                                                                       enable_gqa);
}

// ktt::sdpa_refusal(q, k, v, mask, dropout_p, is_causal, scale): why the kernels do not
// take this call ("" when they do), from sizes, dtypes and devices only, so meta tensors
// answer too (the reference's schema and dispatch key, aten_attention.cpp:910-952; its
// compile pass asks it on meta tensors, torch_backend/chains.py:595-606).
std::string sdpa_refusal_op(const Tensor& q, const Tensor& k, const Tensor& v, const optional<Tensor>& mask,
                            double dropout_p, bool is_causal, optional<double> scale) {
    (void)scale;  // any scale is taken
    return sdpa_refusal_impl(q, k, v, mask, dropout_p, is_causal);
}

// ---------------------------------------------------------------- key lengths

// ktt::_sdpa_lengths and its companions (the reference's aten_lengths.cpp:28-67 checks,
// 69-101 forward, 103-152 backward, 154-172 supported, 175-197 schemas): batch b's queries
// see keys [0, lengths[b]) with lengths an int32 [B] GPU tensor clamped in-kernel to
// [1, Sk].  No mask is built; the kernels stop at each sequence's length.
void lengths_check(const char* op, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& lengths) {
    for (const Tensor* t : {&q, &k, &v})
        TORCH_CHECK(t->dim() == 4 && t->numel() > 0 && t->is_cuda() &&
                        (t->scalar_type() == at::kBFloat16 || t->scalar_type() == at::kHalf),
                    "kohakutt_amd: ", op, " needs non-empty bf16 / fp16 [batch, heads, sequence, head dim] GPU tensors");
    TORCH_CHECK(k.size(0) == q.size(0) && v.size(0) == q.size(0) && k.size(1) == v.size(1) &&
                    q.size(1) % k.size(1) == 0 && k.size(2) == v.size(2) && k.size(3) == q.size(3),
                "kohakutt_amd: ", op, " q / k / v shapes do not match");
    TORCH_CHECK(lengths.dim() == 1 && lengths.size(0) == q.size(0) && lengths.scalar_type() == at::kInt &&
                    lengths.device() == q.device(),
                "kohakutt_amd: ", op, " key_lengths must be int32 [batch] on q's device");
}

Tensor sdpa_lengths(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& lengths, bool is_causal,
                    optional<double> scale, bool stats) {
    (void)stats;  // the backward recomputes in fp32; it needs no saved statistics
    lengths_check("_sdpa_lengths", q, k, v, lengths);
    const std::string why = sdpa_refusal_impl(q, k, v, std::nullopt, 0.0, is_causal);
    TORCH_CHECK(why.empty(), "kohakutt_amd: _sdpa_lengths: ", why);
    const Tensor len = lengths.contiguous();
    return run_attention(q, k, v, std::nullopt, is_causal, scale, &len).out;
}

bool sdpa_lengths_supported(const Tensor& q, const Tensor& k, const Tensor& v, bool is_causal, bool stats) {
    if (!sdpa_refusal_impl(q, k, v, std::nullopt, 0.0, is_causal).empty()) return false;
    // The backward takes causal with Sq == Sk only (aten_lengths.cpp:115-118).
    return !(stats && is_causal && q.size(2) != k.size(2));
}

std::tuple<Tensor, Tensor, Tensor> sdpa_lengths_backward(const Tensor& grad, const Tensor& out, const Tensor& q,
                                                         const Tensor& k, const Tensor& v, const Tensor& lengths,
                                                         bool is_causal, optional<double> scale) {
    lengths_check("_sdpa_lengths_backward", q, k, v, lengths);
    TORCH_CHECK(!is_causal || q.size(2) == k.size(2), "kohakutt_amd: _sdpa_lengths_backward causal needs Sq == Sk");
    TORCH_CHECK(grad.sizes() == out.sizes() && grad.scalar_type() == q.scalar_type(),
                "kohakutt_amd: _sdpa_lengths_backward grad must be shaped and typed as the output");
    c10::DeviceGuard guard(q.device());
    // The schema carries no statistics: one forward pass on the kernels gives the lse, then
    // the backward kernels stop every batch entry's keys at its length (keys past it get
    // zero gradients).
    const Tensor len = lengths.contiguous();
    const AttnOut fwd = run_attention(q, k, v, std::nullopt, is_causal, scale, &len);
    BwdCall c;
    c.grad = grad;
    c.q = q;
    c.k = k;
    c.v = v;
    c.out = out;
    c.lse = fwd.lse;
    c.key_lengths = len;
    c.causal = is_causal;
    c.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(q.size(3)));
    return run_backward(c);
}

// ---------------------------------------------------------------- varlen

// Per-sequence lengths of host offsets under the reference's rules and messages
// (varlen::intervals, ktt_flash/varlen_plan.hpp:43-82): equal counts starting at 0,
// non-decreasing, a sequence with queries has keys, causal (bottom-right) leaves no query
// without keys.
struct HostLengths {
    int64_t nseq = 0, max_q = 0, max_k = 0, mask_values = 0;
};

HostLengths host_lengths(at::IntArrayRef cu_q, at::IntArrayRef cu_k, bool causal) {
    TORCH_CHECK_VALUE(cu_q.size() >= 2 && cu_q.size() == cu_k.size() && cu_q[0] == 0 && cu_k[0] == 0,
                      "kohakutt_amd: sdpa_varlen needs cumulative offsets [0, ..., total] of equal count for queries "
                      "and keys");
    HostLengths h;
    h.nseq = static_cast<int64_t>(cu_q.size()) - 1;
    for (int64_t i = 0; i < h.nseq; ++i) {
        const int64_t lq = cu_q[i + 1] - cu_q[i], lk = cu_k[i + 1] - cu_k[i];
        TORCH_CHECK_VALUE(lq >= 0 && lk >= 0 && !(lq > 0 && lk == 0),
                          "kohakutt_amd: sdpa_varlen offsets must not decrease, and a sequence with queries needs keys");
        TORCH_CHECK_VALUE(!(causal && lq > lk),
                          "kohakutt_amd: causal sdpa_varlen with more queries than keys in a sequence leaves queries "
                          "without keys");
        h.max_q = std::max(h.max_q, lq);
        h.max_k = std::max(h.max_k, lk);
        h.mask_values += lq * lk;
    }
    return h;
}

Tensor offsets_tensor(at::IntArrayRef cu) {
    Tensor t = at::empty({static_cast<int64_t>(cu.size())}, at::dtype(at::kInt));
    int32_t* d = t.data_ptr<int32_t>();
    for (size_t i = 0; i < cu.size(); ++i) {
        TORCH_CHECK_VALUE(cu[i] >= 0 && cu[i] <= INT32_MAX, "kohakutt_amd: sdpa_varlen offsets must fit int32");
        d[i] = static_cast<int32_t>(cu[i]);
    }
    return t;
}

// ktt::_varlen_plan(cu_q, cu_k, is_causal, scale, key_side): this build's plan of an
// offset set, as CPU tensors the caller keeps on the device (the reference's plan,
// aten_varlen.cpp:32-70, is Tensix tile records and mask tiles).  The kernels need only the
// offsets: records = int32 [2, n + 1] (row 0 the query offsets, row 1 the key offsets);
// masks = int64 [n + 1], entry i = sum_{j<i} Lq_j * Lk_j (where sequence i's block of a
// block-packed per-row mask starts).  The offsets are validated here with the reference's
// rules; key_side gives the same tables (the backward kernels read offsets, not tile rows).
std::tuple<Tensor, Tensor> varlen_plan(at::IntArrayRef cu_q, at::IntArrayRef cu_k, bool is_causal, double scale,
                                       bool key_side) {
    (void)key_side;
    TORCH_CHECK_NOT_IMPLEMENTED(scale > 0, "kohakutt_amd: _varlen_plan: the scale must be positive");
    const HostLengths h = host_lengths(cu_q, cu_k, is_causal);
    Tensor records = at::stack({offsets_tensor(cu_q), offsets_tensor(cu_k)});
    Tensor masks = at::empty({h.nseq + 1}, at::dtype(at::kLong));
    int64_t* m = masks.data_ptr<int64_t>();
    m[0] = 0;
    for (int64_t i = 0; i < h.nseq; ++i) m[i + 1] = m[i] + (cu_q[i + 1] - cu_q[i]) * (cu_k[i + 1] - cu_k[i]);
    return {records, masks};
}

// One packed call's operands (after validation).
struct VarlenCall {
    Tensor q, k, v;                // bf16 / fp16 [T, H, D] (fp32 inputs cast at entry)
    Tensor cu_q, cu_k;             // device int32 [n + 1]
    Tensor mask_offsets;           // device int64 [n + 1] (packed masks; optional)
    int64_t nseq = 0, max_q = 0, max_k = 0;
    bool causal = false;
    double scale = 0.0;
    Tensor mask;                   // [Tk] key mask in logit units, or a block-packed mask
    bool packed = false;
};

// Forward of a packed call: (out [Tq, H, Dv] in the input dtype, lse [H, Tq] fp32).
std::tuple<Tensor, Tensor> run_varlen(const VarlenCall& c, bool fp32) {
    const Tensor q = kernel_operand(pad_head(c.q), 0), k = kernel_operand(pad_head(c.k), 0),
                 v = kernel_operand(pad_head(c.v), 0);
    const int64_t Tq = q.size(0), H = q.size(1), D = q.size(2), Dv = v.size(2), Tk = k.size(0);
    const int64_t Dv0 = c.v.size(2);  // the caller's value dim (v may run zero-padded)
    Tensor out = at::empty({Tq, H, Dv}, q.options());
    Tensor lse = at::empty({H, Tq}, q.options().dtype(at::kFloat));
    if (Tq == 0) {
        if (Dv0 != Dv) out = out.narrow(2, 0, Dv0);
        return {fp32 ? out.to(at::kFloat) : out, lse};
    }
    TORCH_CHECK(Tk > 0, "kohakutt_amd: sdpa_varlen: a sequence with queries needs keys");
    kmi_attn_args a{};
    a.q = q.data_ptr();
    a.k = k.data_ptr();
    a.v = v.data_ptr();
    a.out = out.data_ptr();
    a.lse = lse.data_ptr<float>();
    a.dtype = code_of(q.scalar_type());
    a.causal = c.causal ? 1 : 0;
    a.batch = c.nseq;
    a.heads_q = H;
    a.heads_kv = k.size(1);
    a.seq_q = std::max<int64_t>(1, c.max_q);
    a.seq_k = std::max<int64_t>(1, c.max_k);
    a.head_dim = D;
    a.head_dim_v = static_cast<int32_t>(Dv);
    // [T, H, D] tensors: stride[1] is the head stride, stride[2] the token stride.
    a.q_stride[1] = q.stride(1);
    a.q_stride[2] = q.stride(0);
    a.k_stride[1] = k.stride(1);
    a.k_stride[2] = k.stride(0);
    a.v_stride[1] = v.stride(1);
    a.v_stride[2] = v.stride(0);
    a.o_stride[1] = out.stride(1);
    a.o_stride[2] = out.stride(0);
    a.lse_stride[1] = lse.stride(0);
    a.lse_stride[2] = lse.stride(1);
    a.scale = c.scale;
    a.cu_seqlens_q = c.cu_q.data_ptr<int32_t>();
    a.cu_seqlens_k = c.cu_k.data_ptr<int32_t>();
    a.total_q = Tq;
    a.total_k = Tk;
    if (c.mask.defined()) {
        a.mask = c.mask.data_ptr();
        a.mask_dtype = code_of(c.mask.scalar_type());
        TORCH_CHECK(a.mask_dtype != 0, "kohakutt_amd: sdpa_varlen mask dtype must be bool or floating");
        if (c.packed) {
            a.mask_mode = KMI_MASK_PACKED;
            a.mask_numel = c.mask.numel();
            if (c.mask_offsets.defined()) a.mask_offsets = c.mask_offsets.data_ptr<int64_t>();
        } else {
            a.mask_mode = KMI_MASK_STRIDED;
            a.mask_stride[3] = c.mask.stride(0);
        }
    }
    size_t ws = 0;
    check(kmi_attn_workspace_bytes(&a, &ws), "kmi_attn_workspace_bytes");
    Tensor work;
    if (ws) work = at::empty({static_cast<int64_t>(ws)}, q.options().dtype(at::kByte));
    check(kmi_attn_fwd(&a, ws ? work.data_ptr() : nullptr, ws, stream_of(q)), "kmi_attn_fwd (varlen)");
    g_attn_calls.fetch_add(1);
    if (Dv0 != Dv) out = out.narrow(2, 0, Dv0);
    return {fp32 ? out.to(at::kFloat) : out, lse};
}

// q, k, v of a packed call as the kernels take them: [T, H, D] (v [T, Hk, Dv]) of one
// dtype (fp32 cast to bf16 at entry, like the dense route), K/V heads dividing Q heads.
// The value head dim may differ from q's and k's (the reference's packed op,
// aten_varlen.cpp:160-208).
void packed_operands(const char* op, const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, VarlenCall& c,
                     bool& fp32) {
    TORCH_CHECK(q_in.is_cuda() && k_in.is_cuda() && v_in.is_cuda() && k_in.device() == q_in.device() &&
                    v_in.device() == q_in.device(),
                "kohakutt_amd: ", op, " needs GPU tensors on one device");
    TORCH_CHECK_NOT_IMPLEMENTED(q_in.dim() == 3 && k_in.dim() == 3 && v_in.dim() == 3,
                                "kohakutt_amd: ", op, " takes q [Tq, H, D], k [Tk, Hk, D], v [Tk, Hk, Dv]");
    TORCH_CHECK_NOT_IMPLEMENTED(k_in.size(0) == v_in.size(0) && k_in.size(1) == v_in.size(1) &&
                                    k_in.size(1) > 0 && q_in.size(1) % k_in.size(1) == 0,
                                "kohakutt_amd: ", op, " q / k / v shapes do not match (K / V heads must divide Q heads)");
    TORCH_CHECK_NOT_IMPLEMENTED(q_in.size(2) == k_in.size(2) && head_dim_ok(q_in.size(2)) && head_dim_ok(v_in.size(2)),
                                "kohakutt_amd: ", op, " needs q and k of one head dim and head dims up to 256");
    fp32 = q_in.scalar_type() == at::kFloat;
    c.q = fp32 ? q_in.to(at::kBFloat16) : q_in;
    c.k = fp32 ? k_in.to(at::kBFloat16) : k_in;
    c.v = fp32 ? v_in.to(at::kBFloat16) : v_in;
    const auto st = c.q.scalar_type();
    TORCH_CHECK_NOT_IMPLEMENTED(c.k.scalar_type() == st && c.v.scalar_type() == st &&
                                    (st == at::kBFloat16 || st == at::kHalf),
                                "kohakutt_amd: ", op, " takes bf16 / fp16 tensors of one dtype (or fp32, cast to bf16)");
}

// The reference's key mask form (varlen.py:165-183: bf16 [Tk], already divided by the
// scale, the -5e5 floor divided too) in logit units for the kernels: values at the floor
// (within bf16 rounding) become -inf, which the kernels read as masked.
Tensor key_mask_logits(const Tensor& key_mask, double scale, const Tensor& k) {
    TORCH_CHECK_NOT_IMPLEMENTED(key_mask.dim() == 1 && key_mask.size(0) == k.size(0) && key_mask.is_floating_point(),
                                "kohakutt_amd: _sdpa_varlen the key mask must be floating [key tokens]");
    Tensor m = key_mask.to(k.device(), at::kFloat) * scale;
    return m.masked_fill(m <= kMaskedLogit * (1.0 - 1.0 / 128.0), -INFINITY).contiguous();
}

// Row statistics of _sdpa_varlen outputs, by output storage: the reference keeps them
// with the output's device handle for _sdpa_varlen_backward (aten_varlen.cpp:72-104).
struct StatsEntry {
    c10::weak_intrusive_ptr<c10::StorageImpl> out;
    Tensor lse;
};
std::mutex g_stats_mutex;
std::map<const c10::StorageImpl*, StatsEntry>& stats_table() {
    static auto* table = new std::map<const c10::StorageImpl*, StatsEntry>();
    return *table;
}

void remember_stats(const Tensor& out, const Tensor& lse) {
    std::lock_guard<std::mutex> lock(g_stats_mutex);
    auto& t = stats_table();
    for (auto it = t.begin(); it != t.end();) it = it->second.out.expired() ? t.erase(it) : std::next(it);
    c10::StorageImpl* impl = out.storage().unsafeGetStorageImpl();
    t.insert_or_assign(impl, StatsEntry{out.storage().getWeakStorageImpl(), lse});
}

Tensor stats_of(const Tensor& out) {
    std::lock_guard<std::mutex> lock(g_stats_mutex);
    auto& t = stats_table();
    auto it = t.find(out.storage().unsafeGetStorageImpl());
    if (it == t.end() || it->second.out.expired()) return Tensor();
    return it->second.lse;
}

// ktt::_sdpa_varlen (the reference's schema, aten_varlen.cpp:165-231,328-334): packed q
// [Tq, H, D], k / v [Tk, Hk, D] with host offsets cu_q / cu_k and their _varlen_plan
// tables (plan: records, masks) on q's device; returns (out [Tq, H, D], lse [H, Tq] when
// `stats`, else an empty tensor).  key_mask: the reference's form (bf16 [Tk], divided by
// the scale).  center: the reference's kernel takes centred keys for Tensix numerics (the
// same output); these kernels take the keys as they are.
std::tuple<Tensor, Tensor> sdpa_varlen_ref(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& plan,
                                           const Tensor& masks, at::IntArrayRef cu_q, at::IntArrayRef cu_k,
                                           bool is_causal, optional<double> scale, bool stats,
                                           const optional<Tensor>& key_mask, bool center) {
    (void)center;
    const char* op = "_sdpa_varlen";
    VarlenCall c;
    bool fp32 = false;
    packed_operands(op, q, k, v, c, fp32);
    const HostLengths h = host_lengths(cu_q, cu_k, is_causal);
    TORCH_CHECK_NOT_IMPLEMENTED(cu_q.back() == q.size(0) && cu_k.back() == k.size(0),
                                "kohakutt_amd: ", op, " the offsets must end at the token counts");
    TORCH_CHECK(plan.dim() == 2 && plan.size(0) == 2 && plan.size(1) == h.nseq + 1 && plan.scalar_type() == at::kInt,
                "kohakutt_amd: ", op, " plan must be _varlen_plan's records [2, ", h.nseq + 1, "] of these offsets");
    c10::DeviceGuard guard(q.device());
    const Tensor rec = plan.to(q.device()).contiguous();
    c.cu_q = rec[0];
    c.cu_k = rec[1];
    c.nseq = h.nseq;
    c.max_q = h.max_q;
    c.max_k = h.max_k;
    c.causal = is_causal;
    c.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(q.size(2)));
    if (mask_given(key_mask)) c.mask = key_mask_logits(*key_mask, c.scale, c.k);
    (void)masks;  // per-row mask offsets: the reference's schema carries no per-row mask
    auto [out, lse] = run_varlen(c, fp32);
    if (!stats) return {out, at::empty({0}, q.options().dtype(at::kFloat))};
    remember_stats(out, lse);
    return {out, lse};
}

// ktt::_sdpa_varlen_backward (the reference's schema, aten_varlen.cpp:237-319,336-340):
// (dq, dk, dv) of a _sdpa_varlen call with `stats` from its output `out`, in one set of
// kernel launches over every sequence (the forward's key mask and causal rule).
std::tuple<Tensor, Tensor, Tensor> sdpa_varlen_backward_ref(
    const Tensor& grad, const Tensor& out, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& plan,
    const Tensor& masks, const Tensor& key_plan, const Tensor& key_masks, at::IntArrayRef cu_q, at::IntArrayRef cu_k,
    bool is_causal, optional<double> scale, const optional<Tensor>& key_mask) {
    (void)masks, (void)key_plan, (void)key_masks;
    const char* op = "_sdpa_varlen_backward";
    VarlenCall c;
    bool fp32 = false;
    packed_operands(op, q, k, v, c, fp32);
    TORCH_CHECK_NOT_IMPLEMENTED(!fp32, "kohakutt_amd: ", op, " takes bf16 / fp16 tensors");
    const HostLengths h = host_lengths(cu_q, cu_k, is_causal);
    TORCH_CHECK_NOT_IMPLEMENTED(cu_q.back() == q.size(0) && cu_k.back() == k.size(0),
                                "kohakutt_amd: ", op, " the offsets must end at the token counts");
    TORCH_CHECK_NOT_IMPLEMENTED(grad.sizes() == out.sizes() && grad.scalar_type() == q.scalar_type() &&
                                    out.dim() == 3 && out.size(0) == q.size(0) && out.size(1) == q.size(1) &&
                                    out.size(2) == v.size(2),
                                "kohakutt_amd: ", op, " grad and out must be the forward's [query tokens, heads, value dim]");
    const Tensor lse = stats_of(out);
    TORCH_CHECK_NOT_IMPLEMENTED(lse.defined(), "kohakutt_amd: ", op,
                                " out is not an output of _sdpa_varlen with statistics");
    TORCH_CHECK(plan.dim() == 2 && plan.size(0) == 2 && plan.size(1) == h.nseq + 1 && plan.scalar_type() == at::kInt,
                "kohakutt_amd: ", op, " plan must be _varlen_plan's records [2, ", h.nseq + 1, "] of these offsets");
    c10::DeviceGuard guard(q.device());
    const Tensor rec = plan.to(q.device()).contiguous();
    BwdCall b;
    b.grad = grad;
    b.q = q;
    b.k = k;
    b.v = v;
    b.out = out;
    b.lse = lse;
    b.cu_q = rec[0];
    b.cu_k = rec[1];
    b.nseq = h.nseq;
    b.max_q = h.max_q;
    b.max_k = h.max_k;
    b.causal = is_causal;
    b.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(q.size(2)));
    if (mask_given(key_mask)) b.mask = key_mask_logits(*key_mask, b.scale, k);
    return run_backward(b);
}

// The offsets of a call that holds them as tensors: device int32 copies, and (when they
// are host tensors) their validated lengths.  Device offsets are trusted: the kernels clamp
// them into the packed token ranges, and max_q / max_k must cover every sequence.
struct OffsetArgs {
    Tensor cu_q, cu_k;
    bool host = false;
    HostLengths h;
};

OffsetArgs offset_args(const char* op, const Tensor& cu_q_in, const Tensor& cu_k_in, bool causal, int64_t tq,
                       int64_t tk, int64_t max_q, int64_t max_k, const Tensor& q) {
    TORCH_CHECK(cu_q_in.dim() == 1 && cu_k_in.dim() == 1 && cu_q_in.numel() >= 2 && cu_k_in.numel() == cu_q_in.numel(),
                "kohakutt_amd: ", op, " needs cumulative offsets [0, ..., total] of equal count for queries and keys");
    OffsetArgs o;
    o.host = !cu_q_in.is_cuda() && !cu_k_in.is_cuda();
    if (o.host) {
        const Tensor hq = cu_q_in.to(at::kLong).contiguous(), hk = cu_k_in.to(at::kLong).contiguous();
        const at::IntArrayRef aq(hq.data_ptr<int64_t>(), hq.numel()), ak(hk.data_ptr<int64_t>(), hk.numel());
        o.h = host_lengths(aq, ak, causal);
        TORCH_CHECK_VALUE(aq.back() == tq && ak.back() == tk, "kohakutt_amd: ", op,
                          " the offsets must end at the token counts");
        TORCH_CHECK_VALUE(max_q >= o.h.max_q && max_k >= o.h.max_k, "kohakutt_amd: ", op, " max_q / max_k (", max_q,
                          ", ", max_k, ") are below the longest sequence (", o.h.max_q, ", ", o.h.max_k, ")");
    }
    o.cu_q = cu_q_in.to(q.device(), at::kInt).contiguous();
    o.cu_k = cu_k_in.to(q.device(), at::kInt).contiguous();
    return o;
}

// ktt::_sdpa_varlen_offsets: this build's packed op with the offsets as tensors (host or
// device; device offsets need no host sync, so the call can be captured in a graph) --
// what kohakutt_amd.sdpa_varlen and torch_attn::_varlen_attn call.  key_mask: [Tk] bool
// keep-mask or additive (logit units); packed_mask: every sequence's row-major
// [Lq_i, Lk_i] block, concatenated (bool or additive, shared by the heads, usable with
// is_causal).  v may carry its own head dim: returns (out [Tq, H, Dv], lse [H, Tq] fp32).
std::tuple<Tensor, Tensor> sdpa_varlen_offsets(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in,
                                               const Tensor& cu_q_in, const Tensor& cu_k_in, int64_t max_q,
                                               int64_t max_k, bool is_causal, optional<double> scale,
                                               const optional<Tensor>& key_mask, const optional<Tensor>& packed_mask) {
    const char* op = "_sdpa_varlen_offsets";
    VarlenCall c;
    bool fp32 = false;
    packed_operands(op, q_in, k_in, v_in, c, fp32);
    TORCH_CHECK(!(mask_given(key_mask) && mask_given(packed_mask)),
                "kohakutt_amd: sdpa_varlen takes key_mask or packed_mask, not both");
    c10::DeviceGuard guard(q_in.device());
    const OffsetArgs o = offset_args(op, cu_q_in, cu_k_in, is_causal, q_in.size(0), k_in.size(0), max_q, max_k, c.q);
    c.cu_q = o.cu_q;
    c.cu_k = o.cu_k;
    c.nseq = cu_q_in.numel() - 1;
    c.max_q = max_q;
    c.max_k = max_k;
    c.causal = is_causal;
    c.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(q_in.size(2)));
    if (mask_given(key_mask)) {
        Tensor m = *key_mask;
        TORCH_CHECK(m.dim() == 1 && m.size(0) == k_in.size(0), "kohakutt_amd: sdpa_varlen key_mask must be [",
                    k_in.size(0), "] (one value per packed key)");
        if (m.scalar_type() == at::kDouble) m = m.to(at::kFloat);
        c.mask = m.to(q_in.device()).contiguous();
    } else if (mask_given(packed_mask)) {
        Tensor m = *packed_mask;
        if (o.host)
            TORCH_CHECK(m.numel() == o.h.mask_values, "kohakutt_amd: sdpa_varlen packed mask must hold sum(Lq_i * Lk_i) = ",
                        o.h.mask_values, " values, got ", m.numel());
        if (m.scalar_type() == at::kDouble) m = m.to(at::kFloat);
        c.mask = m.to(q_in.device()).contiguous().view({-1});
        TORCH_CHECK(c.mask.numel() > 0, "kohakutt_amd: sdpa_varlen packed mask is empty");
        c.packed = true;
        // Block offsets: prefix sums of Lq_i * Lk_i on the device (no host sync).
        const Tensor lq = (c.cu_q.slice(0, 1) - c.cu_q.slice(0, 0, -1)).to(at::kLong);
        const Tensor lk = (c.cu_k.slice(0, 1) - c.cu_k.slice(0, 0, -1)).to(at::kLong);
        c.mask_offsets = at::cat({at::zeros({1}, lq.options()), (lq * lk).cumsum(0)});
    }
    return run_varlen(c, fp32);
}

// ktt::_sdpa_varlen_offsets_backward: (dq, dk, dv) of a _sdpa_varlen_offsets call from
// its output and lse, in one set of kernel launches over every sequence.
std::tuple<Tensor, Tensor, Tensor> sdpa_varlen_offsets_backward(
    const Tensor& grad, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out, const Tensor& lse,
    const Tensor& cu_q_in, const Tensor& cu_k_in, int64_t max_q, int64_t max_k, bool is_causal,
    optional<double> scale, const optional<Tensor>& key_mask, const optional<Tensor>& packed_mask) {
    const char* op = "_sdpa_varlen_offsets_backward";
    VarlenCall c;
    bool fp32 = false;
    packed_operands(op, q, k, v, c, fp32);
    TORCH_CHECK_NOT_IMPLEMENTED(!fp32, "kohakutt_amd: ", op, " takes bf16 / fp16 tensors");
    TORCH_CHECK(grad.dim() == 3 && grad.size(0) == q.size(0) && grad.size(1) == q.size(1) &&
                    grad.size(2) == v.size(2) && out.sizes() == grad.sizes() && grad.scalar_type() == q.scalar_type(),
                "kohakutt_amd: ", op, " grad and out must be [query tokens, heads, value dim] in q's dtype");
    TORCH_CHECK(lse.dim() == 2 && lse.size(0) == q.size(1) && lse.size(1) == q.size(0) &&
                    lse.scalar_type() == at::kFloat,
                "kohakutt_amd: ", op, " lse must be the forward's fp32 [H, Tq]");
    c10::DeviceGuard guard(q.device());
    const OffsetArgs o = offset_args(op, cu_q_in, cu_k_in, is_causal, q.size(0), k.size(0), max_q, max_k, q);
    BwdCall b;
    b.grad = grad;
    b.q = q;
    b.k = k;
    b.v = v;
    b.out = out;
    b.lse = lse.contiguous();
    b.cu_q = o.cu_q;
    b.cu_k = o.cu_k;
    b.nseq = cu_q_in.numel() - 1;
    b.max_q = max_q;
    b.max_k = max_k;
    b.causal = is_causal;
    b.scale = scale.has_value() ? *scale : 1.0 / std::sqrt(static_cast<double>(q.size(2)));
    if (mask_given(key_mask)) {
        Tensor m = *key_mask;
        if (m.scalar_type() == at::kDouble) m = m.to(at::kFloat);
        b.mask = m.to(q.device()).contiguous();
    } else if (mask_given(packed_mask)) {
        Tensor m = *packed_mask;
        if (m.scalar_type() == at::kDouble) m = m.to(at::kFloat);
        b.mask = m.to(q.device()).contiguous().view({-1});
        b.packed = true;
        const Tensor lq = (o.cu_q.slice(0, 1) - o.cu_q.slice(0, 0, -1)).to(at::kLong);
        const Tensor lk = (o.cu_k.slice(0, 1) - o.cu_k.slice(0, 0, -1)).to(at::kLong);
        b.mask_offsets = at::cat({at::zeros({1}, lq.options()), (lq * lk).cumsum(0)});
    }
    return run_backward(b);
}

// ---------------------------------------------------------------- norms

bool norm_dtype(at::ScalarType t) { return t == at::kBFloat16 || t == at::kHalf || t == at::kFloat; }

// True when the kernels take a norm of x over its trailing `normalized` dims with
// parameters `params` (undefined, or GPU tensors with `width` elements).  Mirrors the
// reference's own_norm (aten_norm.cpp:22-40), widened to any trailing dims.
bool norms_take(const Tensor& x, int64_t width, std::initializer_list<const optional<Tensor>*> params) {
    if (!g_norms.load() || !x.is_cuda() || x.numel() == 0 || !norm_dtype(x.scalar_type()) || width <= 0) return false;
    for (const auto* p : params) {
        if (*p && (*p)->defined() &&
            (!(*p)->is_cuda() || (*p)->device() != x.device() || (*p)->numel() != width ||
             !norm_dtype((*p)->scalar_type())))
            return false;
    }
    return true;
}

// Weight / bias as the kernels read them: contiguous, one type that is x's or fp32.
void norm_params(const Tensor& x, optional<Tensor>& w, optional<Tensor>& b) {
    const bool hw = w && w->defined(), hb = b && b->defined();
    auto st = hw ? w->scalar_type() : (hb ? b->scalar_type() : x.scalar_type());
    const bool same = (!hw || w->scalar_type() == st) && (!hb || b->scalar_type() == st);
    if (!same || (st != x.scalar_type() && st != at::kFloat)) st = at::kFloat;
    if (hw) w = w->to(st).contiguous();
    if (hb) b = b->to(st).contiguous();
}

std::tuple<Tensor, Tensor, Tensor> native_layer_norm(const Tensor& input, at::IntArrayRef normalized_shape,
                                                     const optional<Tensor>& weight, const optional<Tensor>& bias,
                                                     double eps) {
    const int64_t nd = static_cast<int64_t>(normalized_shape.size());
    bool shape_ok = nd >= 1 && nd <= input.dim();
    for (int64_t i = 0; shape_ok && i < nd; ++i) shape_ok = input.size(input.dim() - nd + i) == normalized_shape[i];
    int64_t width = 1;
    for (auto s : normalized_shape) width *= s;
    if (!shape_ok || !norms_take(input, width, {&weight, &bias}))
        return at::cuda::native_layer_norm(input, normalized_shape, weight, bias, eps);
    c10::DeviceGuard guard(input.device());
    Tensor x = input.contiguous();
    optional<Tensor> w = weight, b = bias;
    norm_params(x, w, b);
    const int64_t rows = x.numel() / width;
    std::vector<int64_t> stat_sizes(input.sizes().begin(), input.sizes().end());
    for (int64_t i = input.dim() - nd; i < input.dim(); ++i) stat_sizes[i] = 1;
    Tensor y = at::empty_like(x);
    Tensor mean = at::empty(stat_sizes, x.options().dtype(at::kFloat));
    Tensor rstd = at::empty(stat_sizes, x.options().dtype(at::kFloat));
    const bool hw = w && w->defined(), hb = b && b->defined();
    check(kmi_layer_norm_fwd(x.data_ptr(), hw ? w->data_ptr() : nullptr, hb ? b->data_ptr() : nullptr, y.data_ptr(),
                             mean.data_ptr<float>(), rstd.data_ptr<float>(), rows, width, code_of(x.scalar_type()),
                             hw ? code_of(w->scalar_type()) : 0, hb ? code_of(b->scalar_type()) : 0, eps,
                             stream_of(x)),
          "kmi_layer_norm_fwd");
    g_norm_calls.fetch_add(1);
    return {y, mean, rstd};
}

// aten::native_layer_norm_backward on CUDA (the reference's own backward programs,
// aten_norm.cpp:130-224,811): the one-pass kernel (kmi_layer_norm_bwd) when the forward's
// statistics are this build's fp32 ones and the rows are whole 16-byte vectors of at most
// 256 vectors; torch's CUDA kernel otherwise.
std::tuple<Tensor, Tensor, Tensor> native_layer_norm_backward(const Tensor& grad_out, const Tensor& input,
                                                              at::IntArrayRef normalized_shape, const Tensor& mean,
                                                              const Tensor& rstd, const optional<Tensor>& weight,
                                                              const optional<Tensor>& bias,
                                                              std::array<bool, 3> output_mask) {
    const int64_t nd = static_cast<int64_t>(normalized_shape.size());
    int64_t width = 1;
    for (auto s : normalized_shape) width *= s;
    const bool hw = weight && weight->defined(), hb = bias && bias->defined();
    const auto wt = hw ? weight->scalar_type() : input.scalar_type();
    const int xs = input.element_size();
    bool take = g_norms.load() && input.is_cuda() && norm_dtype(input.scalar_type()) && input.numel() > 0 &&
                grad_out.scalar_type() == input.scalar_type() && grad_out.sizes() == input.sizes() && nd >= 1 &&
                nd <= input.dim() && mean.scalar_type() == at::kFloat && rstd.scalar_type() == at::kFloat &&
                mean.numel() * width == input.numel() && rstd.numel() == mean.numel() && width % (16 / xs) == 0 &&
                width / (16 / xs) <= 4 * 64 && (!hw || wt == input.scalar_type() || wt == at::kFloat) &&
                (!hb || bias->scalar_type() == wt) && real_data(input) && real_data(grad_out);
    if (!take)
        return at::cuda::native_layer_norm_backward(grad_out, input, normalized_shape, mean, rstd, weight, bias,
                                                    output_mask);
    c10::DeviceGuard guard(input.device());
    // The one-pass kernel reads whole 16-byte vectors of x and dy and the matching run of
    // weight elements.  A contiguous view at an odd storage offset, or a weight sliced
    // from a flat parameter buffer, is copied once into a fresh (aligned) allocation;
    // torch's own kernel is no fallback here, as it refuses an fp32 weight on bf16 rows.
    const auto aligned_to = [](const Tensor& t, int64_t bytes) {
        const Tensor c = t.contiguous();
        if (reinterpret_cast<uintptr_t>(c.data_ptr()) % static_cast<uintptr_t>(bytes) == 0) return c;
        return c.clone(at::MemoryFormat::Contiguous);
    };
    const Tensor x = aligned_to(input, 16), gy = aligned_to(grad_out, 16);
    const Tensor w = hw ? aligned_to(*weight, (16 / xs) * static_cast<int64_t>(c10::elementSize(wt))) : Tensor();
    const Tensor m = mean.contiguous(), r = rstd.contiguous();
    const int64_t rows = x.numel() / width;
    Tensor dx = at::empty_like(x);
    Tensor dw = (output_mask[1] && hw) ? at::empty_like(w) : Tensor();
    Tensor db = (output_mask[2] && hb) ? at::empty({width}, x.options().dtype(wt)).view(bias->sizes()) : Tensor();
    size_t ws = 0;
    check(kmi_layer_norm_bwd_workspace_bytes(rows, width, &ws), "kmi_layer_norm_bwd_workspace_bytes");
    Tensor work;
    if ((dw.defined() || db.defined()) && ws) work = at::empty({static_cast<int64_t>(ws)}, x.options().dtype(at::kByte));
    check(kmi_layer_norm_bwd(gy.data_ptr(), x.data_ptr(), m.data_ptr<float>(), r.data_ptr<float>(),
                             hw ? w.data_ptr() : nullptr, dx.data_ptr(), dw.defined() ? dw.data_ptr() : nullptr,
                             db.defined() ? db.data_ptr() : nullptr, rows, width, code_of(x.scalar_type()),
                             hw ? code_of(wt) : 0, db.defined() ? code_of(wt) : 0,
                             work.defined() ? work.data_ptr() : nullptr, ws, stream_of(x)),
          "kmi_layer_norm_bwd");
    g_norm_bwd_calls.fetch_add(1);
    return {output_mask[0] ? dx.view(input.sizes()) : Tensor(), dw, db};
}

// y, rstd of RMSNorm over the trailing dims (width elements per row), optional bias.
std::tuple<Tensor, Tensor> rms_forward(const Tensor& input, int64_t width, optional<Tensor> w, optional<Tensor> b,
                                       double eps, int64_t nd) {
    c10::DeviceGuard guard(input.device());
    Tensor x = input.contiguous();
    norm_params(x, w, b);
    const int64_t rows = x.numel() / width;
    std::vector<int64_t> stat_sizes(input.sizes().begin(), input.sizes().end());
    for (int64_t i = input.dim() - nd; i < input.dim(); ++i) stat_sizes[i] = 1;
    Tensor y = at::empty_like(x);
    Tensor rstd = at::empty(stat_sizes, x.options().dtype(at::kFloat));
    const bool hw = w && w->defined(), hb = b && b->defined();
    check(kmi_rms_norm_fwd(x.data_ptr(), hw ? w->data_ptr() : nullptr, hb ? b->data_ptr() : nullptr, y.data_ptr(),
                           rstd.data_ptr<float>(), rows, width, code_of(x.scalar_type()),
                           hw ? code_of(w->scalar_type()) : 0, hb ? code_of(b->scalar_type()) : 0, eps, stream_of(x)),
          "kmi_rms_norm_fwd");
    g_norm_calls.fetch_add(1);
    return {y, rstd};
}

// RMSNorm with gradients: the kernel forward, an fp32 backward from the saved rstd (the
// reference's RmsNormFunction, aten_norm.cpp:548-599).
struct RmsNormFn : public torch::autograd::Function<RmsNormFn> {
    // The weight travels as an optional: an undefined Tensor argument is taken for a
    // variable by the Function machinery (which then asks it for its device).
    static Tensor forward(torch::autograd::AutogradContext* ctx, const Tensor& x, const optional<Tensor>& wo,
                          int64_t nd, double eps) {
        int64_t width = 1;
        for (int64_t i = x.dim() - nd; i < x.dim(); ++i) width *= x.size(i);
        const Tensor w = wo.has_value() ? *wo : Tensor();
        auto [y, rstd] = rms_forward(x, width, wo, std::nullopt, eps, nd);
        ctx->save_for_backward({x, w, rstd});
        ctx->saved_data["nd"] = nd;
        return y;
    }
    static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                   torch::autograd::variable_list grads) {
        auto saved = ctx->get_saved_variables();
        const Tensor& x = saved[0];
        const Tensor& w = saved[1];
        const Tensor& rstd = saved[2];
        const int64_t nd = ctx->saved_data["nd"].toInt();
        std::vector<int64_t> dims;
        for (int64_t i = x.dim() - nd; i < x.dim(); ++i) dims.push_back(i);
        int64_t width = 1;
        for (auto d : dims) width *= x.size(d);
        if (g_norms.load() && code_of(x.scalar_type()) != 0 && code_of(x.scalar_type()) != KMI_BOOL &&
            (!w.defined() || (code_of(w.scalar_type()) != 0 && code_of(w.scalar_type()) != KMI_BOOL)) &&
            rstd.scalar_type() == at::kFloat && rstd.is_contiguous()) {
            // The kernels: dx per row, dw as a fixed-order column sum (kmi_rms_norm_bwd).
            c10::DeviceGuard guard(x.device());
            const Tensor xc = x.contiguous(), gc = grads[0].to(x.scalar_type()).contiguous();
            const Tensor wc = w.defined() ? w.contiguous() : Tensor();
            const int64_t rows = xc.numel() / width;
            Tensor dx = at::empty_like(xc);
            Tensor dw = w.defined() ? at::empty_like(wc) : Tensor();
            size_t ws = 0;
            check(kmi_rms_norm_bwd_workspace_bytes(rows, width, &ws), "kmi_rms_norm_bwd_workspace_bytes");
            Tensor work;
            if (w.defined() && ws) work = at::empty({static_cast<int64_t>(ws)}, xc.options().dtype(at::kByte));
            check(kmi_rms_norm_bwd(gc.data_ptr(), xc.data_ptr(), w.defined() ? wc.data_ptr() : nullptr,
                                   rstd.data_ptr<float>(), dx.data_ptr(), w.defined() ? dw.data_ptr() : nullptr, rows,
                                   width, code_of(xc.scalar_type()), w.defined() ? code_of(wc.scalar_type()) : 0,
                                   work.defined() ? work.data_ptr() : nullptr, ws, stream_of(xc)),
                  "kmi_rms_norm_bwd");
            g_norm_bwd_calls.fetch_add(1);
            return {dx, dw, Tensor(), Tensor()};
        }
        Tensor g = grads[0].to(at::kFloat), xf = x.to(at::kFloat);
        Tensor xhat = xf * rstd;
        Tensor gw = w.defined() ? g * w.to(at::kFloat) : g;
        Tensor dx = rstd * (gw - xhat * (gw * xhat).sum(dims, true) / static_cast<double>(width));
        Tensor dw;
        if (w.defined()) {
            std::vector<int64_t> lead;
            for (int64_t i = 0; i < x.dim() - nd; ++i) lead.push_back(i);
            dw = lead.empty() ? (g * xhat) : (g * xhat).sum(lead);
            dw = dw.reshape(w.sizes()).to(w.scalar_type());
        }
        return {dx.to(x.scalar_type()), dw, Tensor(), Tensor()};
    }
};

// aten::rms_norm at AutogradCUDA (the reference registers it at AutogradPrivateUse1,
// aten_norm.cpp:604-652,797-799); eps defaults to float32 epsilon.
Tensor rms_norm(const Tensor& input, c10::SymIntArrayRef normalized_shape, const optional<Tensor>& weight,
                optional<double> eps) {
    const double e = eps.value_or(static_cast<double>(std::numeric_limits<float>::epsilon()));
    const int64_t nd = static_cast<int64_t>(normalized_shape.size());
    bool shape_ok = nd >= 1 && nd <= input.dim();
    int64_t width = 1;
    for (int64_t i = 0; shape_ok && i < nd; ++i) {
        const auto s = normalized_shape[i].maybe_as_int();
        shape_ok = s.has_value() && input.size(input.dim() - nd + i) == *s;
        if (shape_ok) width *= *s;
    }
    if (!shape_ok || !norms_take(input, width, {&weight}) || !real_data(input) ||
        (weight && weight->defined() && !real_data(*weight)))
        return at::compositeimplicitautograd::rms_norm_symint(input, normalized_shape, weight, eps);
    const bool hw = weight && weight->defined();
    const bool grads = at::GradMode::is_enabled() && (input.requires_grad() || (hw && weight->requires_grad()));
    if (grads) return RmsNormFn::apply(input, hw ? weight : optional<Tensor>(), nd, e);
    at::AutoDispatchBelowADInplaceOrView below;
    return std::get<0>(rms_forward(input, width, weight, std::nullopt, e, nd));
}

// ktt::rms_norm(x, weight, bias, eps): RMSNorm over the last dim with an optional bias,
// one kernel on GPU tensors (aten_fused.cpp:60-85), the fp32 composite elsewhere
// (aten_fused.cpp:13-28).
Tensor ktt_rms_norm_cuda(const Tensor& x, const optional<Tensor>& weight, const optional<Tensor>& bias, double eps) {
    TORCH_CHECK(x.dim() >= 1, "ktt::rms_norm needs at least one dim");
    const int64_t width = x.size(-1);
    if (!norms_take(x, width, {&weight, &bias})) {
        optional<Tensor> w;
        if (weight && weight->defined()) w = weight->to(at::kFloat);
        Tensor y = at::rms_norm(x.to(at::kFloat), {width}, w, eps);
        if (bias && bias->defined()) y = y + bias->to(at::kFloat);
        return y.to(x.scalar_type());
    }
    return std::get<0>(rms_forward(x, width, weight, bias, eps, 1));
}

Tensor ktt_rms_norm_composite(const Tensor& x, const optional<Tensor>& weight, const optional<Tensor>& bias,
                              double eps) {
    optional<Tensor> w;
    if (weight && weight->defined()) w = weight->to(at::kFloat);
    Tensor y = at::rms_norm(x.to(at::kFloat), {x.size(-1)}, w, eps);
    if (bias && bias->defined()) y = y + bias->to(at::kFloat);
    return y.to(x.scalar_type());
}

// ---------------------------------------------------------------- control

void set_enabled(bool attention, bool norms) {
    g_attention.store(attention);
    g_norms.store(norms);
}

std::vector<int64_t> counters() {
    return {g_attn_calls.load(), g_attn_declined.load(), g_norm_calls.load(),
            g_attention.load() ? 1 : 0, g_norms.load() ? 1 : 0, g_attn_bwd_calls.load(), g_norm_bwd_calls.load()};
}

void reset_counters() {
    g_attn_bwd_calls.store(0);
    g_norm_bwd_calls.store(0);
    g_attn_calls.store(0);
    g_attn_declined.store(0);
    g_norm_calls.store(0);
}

// Installs the CUDA entry of the _fused_sdp_choice stub at load time.
struct StubInstall {
    StubInstall() { at::native::_fused_sdp_choice_stub.set_cuda_dispatch_ptr(&fused_sdp_choice); }
} g_stub_install;

}  // namespace
}  // namespace kta

TORCH_LIBRARY(ktt, m) {
    m.def("rms_norm(Tensor x, Tensor? weight, Tensor? bias, float eps) -> Tensor");  // aten_fused.cpp:114-116
    // The reference's packed-attention ops (aten_varlen.cpp:323-341).
    m.def("_varlen_plan(int[] cu_q, int[] cu_k, bool is_causal, float scale, bool key_side) -> (Tensor, Tensor)",
          &kta::varlen_plan);
    m.def(
        "_sdpa_varlen(Tensor q, Tensor k, Tensor v, Tensor plan, Tensor masks, int[] cu_q, int[] cu_k, "
        "bool is_causal, float? scale, bool stats, Tensor? key_mask=None, bool center=False) -> (Tensor, Tensor)");
    m.def(
        "_sdpa_varlen_backward(Tensor grad, Tensor out, Tensor q, Tensor k, Tensor v, Tensor plan, Tensor masks, "
        "Tensor key_plan, Tensor key_masks, int[] cu_q, int[] cu_k, bool is_causal, float? scale, "
        "Tensor? key_mask=None) -> (Tensor, Tensor, Tensor)");
    // This build's packed op with tensor offsets (host or device) and block-packed masks.
    m.def(
        "_sdpa_varlen_offsets(Tensor q, Tensor k, Tensor v, Tensor cu_seq_q, Tensor cu_seq_k, int max_q, int max_k, "
        "bool is_causal=False, float? scale=None, Tensor? key_mask=None, Tensor? packed_mask=None) -> (Tensor, Tensor)");
    m.def(
        "_sdpa_varlen_offsets_backward(Tensor grad, Tensor q, Tensor k, Tensor v, Tensor out, Tensor lse, "
        "Tensor cu_seq_q, Tensor cu_seq_k, int max_q, int max_k, bool is_causal=False, float? scale=None, "
        "Tensor? key_mask=None, Tensor? packed_mask=None) -> (Tensor, Tensor, Tensor)");
    m.def("sdpa_refusal(Tensor q, Tensor k, Tensor v, Tensor? mask, float dropout_p, bool is_causal, float? scale) "
          "-> str");
    m.def("_set_enabled(bool attention, bool norms) -> ()", TORCH_FN(kta::set_enabled));
    m.def("counters() -> int[]", TORCH_FN(kta::counters));
    m.def("_sdpa_flash_backward(Tensor grad, Tensor q, Tensor k, Tensor v, Tensor out, Tensor lse, "
          "bool is_causal, float? scale=None) -> (Tensor, Tensor, Tensor)");
    m.def("_sdpa_lengths_supported(Tensor q, Tensor k, Tensor v, bool is_causal, bool stats) -> bool");
    m.def("_sdpa_lengths(Tensor q, Tensor k, Tensor v, Tensor lengths, bool is_causal, float? scale, bool stats) "
          "-> Tensor");
    m.def("_sdpa_lengths_backward(Tensor grad, Tensor out, Tensor q, Tensor k, Tensor v, Tensor lengths, "
          "bool is_causal, float? scale) -> (Tensor, Tensor, Tensor)");
    m.def("reset_counters() -> ()", TORCH_FN(kta::reset_counters));
}

TORCH_LIBRARY_IMPL(ktt, CUDA, m) {
    m.impl("rms_norm", TORCH_FN(kta::ktt_rms_norm_cuda));
    m.impl("_sdpa_varlen", TORCH_FN(kta::sdpa_varlen_ref));
    m.impl("_sdpa_varlen_backward", TORCH_FN(kta::sdpa_varlen_backward_ref));
    m.impl("_sdpa_varlen_offsets", TORCH_FN(kta::sdpa_varlen_offsets));
    m.impl("_sdpa_varlen_offsets_backward", TORCH_FN(kta::sdpa_varlen_offsets_backward));
    m.impl("_sdpa_flash_backward", TORCH_FN(kta::sdpa_flash_backward_op));
    m.impl("_sdpa_lengths", TORCH_FN(kta::sdpa_lengths));
    m.impl("_sdpa_lengths_supported", TORCH_FN(kta::sdpa_lengths_supported));
    m.impl("_sdpa_lengths_backward", TORCH_FN(kta::sdpa_lengths_backward));
}

TORCH_LIBRARY_IMPL(ktt, CompositeExplicitAutograd, m) {
    m.impl("rms_norm", TORCH_FN(kta::ktt_rms_norm_composite));
    m.impl("sdpa_refusal", TORCH_FN(kta::sdpa_refusal_op));
}

TORCH_LIBRARY_IMPL(aten, CUDA, m) {
    m.impl("_fused_sdp_choice", TORCH_FN(kta::fused_sdp_choice));
    m.impl("_scaled_dot_product_fused_attention_overrideable", TORCH_FN(kta::sdpa_overrideable));
    m.impl("_scaled_dot_product_fused_attention_overrideable_backward", TORCH_FN(kta::sdpa_overrideable_backward));
    m.impl("native_layer_norm", TORCH_FN(kta::native_layer_norm));
    m.impl("native_layer_norm_backward", TORCH_FN(kta::native_layer_norm_backward));
}

TORCH_LIBRARY_IMPL(aten, AutogradCUDA, m) {
    m.impl("rms_norm", TORCH_FN(kta::rms_norm));
    m.impl("scaled_dot_product_attention", TORCH_FN(kta::sdpa_entry));
}
