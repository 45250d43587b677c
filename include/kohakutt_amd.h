/*
 * kohakutt_amd -- C ABI of the MI355X (gfx950) attention + norm hot path.
 *
 * This is the build's own thin layer under its torch ops (the ktt:: operators and the
 * aten overrides that make it a drop-in): plain C, device pointers, int64 sizes and
 * element strides, dtype codes and an opaque stream (a hipStream_t passed as void*).  No
 * torch or HIP types cross it.  It does not stand in for the reference's C API
 * (py_bridge/ktt_capi.h, a handle API of ktt_h tensors freed with ktt_release): each
 * entry point below does the device work of one of the reference's bridge functions,
 * named at the entry point, on caller-owned device memory.
 *
 * Conventions (the error model follows the reference's C API, ktt_capi.h:1-3 and
 * capi.cpp:19,58-79: a failure code plus a thread_local message):
 *   - every entry point returns KMI_OK (0) or a negative kmi_status; the message of the
 *     last failure on the calling thread is kmi_last_error();
 *   - arguments are validated on the host before anything is enqueued: a rejected call
 *     launches nothing;
 *   - work is enqueued on `stream` and never synchronised; nothing is allocated: split-KV
 *     partials and backward partial sums go to the caller's workspace (the *_bytes
 *     queries), or, for kmi_attn_fwd_noalloc, to a device array of the library;
 *   - calls are thread-safe (no mutable global state besides the thread_local error and
 *     kmi_attn_fwd_noalloc's device array, which calls overlapping on one device share).
 */
#ifndef KOHAKUTT_AMD_H
#define KOHAKUTT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KMI_ABI_VERSION 4

/* Element types of operands. */
enum kmi_dtype {
    KMI_BF16 = 1,
    KMI_F16 = 2,
    KMI_F32 = 3,
    KMI_BOOL = 4 /* one byte, nonzero = keep */
};

enum kmi_status {
    KMI_OK = 0,
    KMI_EINVAL = -1,       /* malformed arguments (shapes, strides, pointers) */
    KMI_EUNSUPPORTED = -2, /* well-formed but outside what the kernels take */
    KMI_EHIP = -3,         /* a HIP runtime error at launch */
    KMI_EWORKSPACE = -4    /* workspace missing or too small */
};

/* How kmi_attn_args.mask is laid out. */
enum kmi_mask_mode {
    KMI_MASK_NONE = 0,
    /* element (b, h, i, j) at mask + b*s[0] + h*s[1] + i*s[2] + j*s[3] (stride 0 =
     * broadcast).  Varlen calls index it with packed token indices: (h, t_q, t_k) at
     * mask + h*s[1] + t_q*s[2] + t_k*s[3] (a [Tk] key mask is s = {0, 0, 0, 1}). */
    KMI_MASK_STRIDED = 1,
    /* varlen only: sequence i's row-major [Lq_i, Lk_i] block follows sequence i-1's;
     * element (h, r, c) of sequence i at mask + sum_{j<i} Lq_j*Lk_j + h*s[1] + r*Lk_i + c. */
    KMI_MASK_PACKED = 2
};

/*
 * Attention forward: out = softmax(scale * q k^T + mask) v per (batch, query head),
 * query head h reading K/V head h / (heads_q / heads_kv).
 *
 * Does the device work of the reference's bridge::sdpa (device_attention.cpp:265-497)
 * for the dense route and of bridge::sdpa_varlen (device_attention.cpp:681-761) for
 * packed sequences.
 *
 * Dense: q [B, Hq, Sq, D], k/v [B, Hkv, Sk, D], out [B, Hq, Sq, D]; *_stride give the
 *   element strides of the batch, head and sequence dims (the head-dim stride is 1).
 * Varlen (cu_seqlens_q != NULL): `batch` sequences; q [Tq, Hq, D], k/v [Tk, Hkv, D]
 *   indexed by packed token; stride[0] is ignored; cu_seqlens_* are device int32
 *   [batch + 1] offsets, seq_q / seq_k are the longest sequence lengths (grid bounds).
 * causal: 0 none; 1 causal.  Dense causal is top-left (query i sees keys <= i, the
 *   reference's aten_attention.cpp:106-107); varlen causal is bottom-right (query r sees
 *   the first min(Lk, r + 1 + Lk - Lq) keys, varlen_plan.hpp:70).
 * Masks: bool keeps nonzero keys; float masks are added to the logits; both are clamped
 *   at -5e5 (the reference's kMaskedLogit), so a masked key gets exactly zero weight when
 *   its row keeps any key and a fully-masked row is the softmax over its raw scores.
 * lse (optional, fp32, natural log): dense [B, Hq, Sq] / varlen [Hq, Tq] with strides
 *   lse_stride (batch, head, seq); varlen ignores lse_stride[0].
 * Supported: dtype BF16 or F16, head_dim (and head_dim_v) a multiple of 8 up to 256,
 * heads_kv dividing heads_q.
 */
typedef struct kmi_attn_args {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    float* lse;
    int32_t dtype;
    int32_t causal;
    int64_t batch, heads_q, heads_kv, seq_q, seq_k, head_dim;
    int64_t q_stride[3];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int64_t lse_stride[3];
    double scale;
    const void* mask;
    int32_t mask_dtype;
    int32_t mask_mode;
    int64_t mask_stride[4];
    /* KMI_MASK_PACKED: elements in the mask; reads past it count as masked. */
    int64_t mask_numel;
    const int32_t* cu_seqlens_q;
    const int32_t* cu_seqlens_k;
    /* varlen: packed token counts Tq / Tk.  The kernels clamp every offset into
     * [0, total] (so malformed device offsets cannot read or write out of bounds; they are
     * validated where the caller holds them on the host). */
    int64_t total_q, total_k;
    /* 0: chosen by the library (split-KV for short query tiles over long key ranges);
     * 1: no split; n > 1: at most n key splits. */
    int32_t num_splits;
    /* ABI 4: the value head dim Dv (0: head_dim).  v [.., Dv] and out [.., Dv]; q and k
     * keep head_dim.  A multiple of 8 up to 256.  The reference's packed op takes it
     * (aten_varlen.cpp:160-208: v [Tk, Hk, Dv], out [Tq, H, Dv]); the kernels run at the
     * larger of the two dims, padded, so dense calls take it too. */
    int32_t head_dim_v;
    /* Dense calls only (ABI 2; NULL: every key).  Device int32 [batch]: sequence b's
     * queries see keys [0, L_b), L_b = key_lengths[b] clamped to [1, seq_k]; no mask is
     * built or read and key tiles past L_b are not loaded.  Query rows past L_b still see
     * the first L_b keys.  Composes with causal (top-left).  Does the
     * work of the reference's bridge::sdpa_lengths behind ktt::_sdpa_lengths (aten_lengths.cpp:69-101,
     * 175-197; docs/reference/kernels/flash.md, Key lengths). */
    const int32_t* key_lengths;
    /* ABI 3, varlen with KMI_MASK_PACKED (NULL: the kernels add up the block sizes): device
     * int64 [batch + 1], entry i = sum_{j<i} Lq_j * Lk_j, where sequence i's block starts. */
    const int64_t* mask_offsets;
} kmi_attn_args;

/* Bytes of workspace kmi_attn_fwd needs for `args` (0 when it does not split). */
int kmi_attn_workspace_bytes(const kmi_attn_args* args, size_t* bytes);

/*
 * Enqueues the attention forward of `args` on `stream` (hipStream_t).  Split decode calls
 * merge their splits in the same launch through a library-owned counter array (one slab
 * per stream for the first 16 streams of a device; other streams merge in a second launch
 * with the same arithmetic).
 */
int kmi_attn_fwd(const kmi_attn_args* args, void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * kmi_attn_fwd without a workspace argument and without any allocation: for callers that
 * cannot allocate (code under HIP graph capture, serving loops, hosts that forbid
 * hipMalloc).  No counterpart in the reference.  Split-KV partials go to a file-scope
 * device array of the library (16 MiB per device, held for the life of the process); a
 * call whose kmi_attn_workspace_bytes exceed it returns KMI_EUNSUPPORTED and launches
 * nothing.  Calls that overlap on one device share that array and race; calls in one
 * stream order do not.
 */
int kmi_attn_fwd_noalloc(const kmi_attn_args* args, void* stream);

/*
 * Attention backward of a kmi_attn_fwd call (dense or varlen, causal or not, masked or
 * not): dq, dk, dv of out = softmax(scale * q k^T + mask) v given grad_out and the
 * forward's lse (fp32 natural log, as kmi_attn_fwd writes it).  The probabilities are
 * recomputed per tile from lse with the forward's mask rules (a row whose lse carries the
 * -5e5 offset of a fully-masked row takes its raw scores); nothing of size Sq x Sk is
 * stored.  GQA: dk / dv of a K/V head sum its query heads.  Layouts as kmi_attn_fwd's
 * (dense: element strides of the batch, head and sequence dims; varlen: [T, H, D] with
 * stride[1] the head and stride[2] the token stride, lse [Hq, Tq]); head-dim stride 1;
 * q, k, v, out, grad_out 16-byte aligned with strides multiples of 8 (row strides below
 * 2^25 elements).  Masks take the
 * forward's modes and strides and get no gradient.  Workspace:
 * kmi_attn_bwd_workspace_bytes, 16-byte aligned (fp32 row dot products; when the query
 * rows of a key tile or the key tiles of a query block are split over workgroups, also
 * fp32 dK / dV and dQ partials, added in a fixed order).
 * Does the work of the reference's flash backward behind tt_sdpa_overrideable_backward's stats
 * route (aten_attention.cpp:716-812; bridge in device_attention.cpp:1208-1281;
 * docs/reference/kernels/flash.md:151-206) and its packed backward behind
 * ktt::_sdpa_varlen_backward (aten_varlen.cpp:237-319).  Supported: BF16 / F16, head
 * dims that are multiples of 8 up to 256.
 */
typedef struct kmi_attn_bwd_args {
    const void* q;
    const void* k;
    const void* v;
    const void* out;
    const void* grad_out;
    const float* lse;
    void* grad_q;
    void* grad_k;
    void* grad_v;
    int32_t dtype;
    int32_t causal;
    int64_t batch, heads_q, heads_kv, seq_q, seq_k, head_dim;
    int64_t q_stride[3];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int64_t do_stride[3];
    int64_t dq_stride[3];
    int64_t dk_stride[3];
    int64_t dv_stride[3];
    int64_t lse_stride[3];
    double scale;
    /* ABI 3: the forward's mask (as in kmi_attn_args) and varlen offsets (cu_seqlens_q !=
     * NULL: `batch` packed sequences, seq_q / seq_k the longest lengths).  With device
     * offsets seq_q / seq_k must cover every sequence (the host cannot check them): the
     * backward sizes its grids and partial sums from them, and gradient rows past them
     * hold unspecified values. */
    const void* mask;
    int32_t mask_dtype;
    int32_t mask_mode;
    int64_t mask_stride[4];
    int64_t mask_numel;
    const int64_t* mask_offsets;
    const int32_t* cu_seqlens_q;
    const int32_t* cu_seqlens_k;
    int64_t total_q, total_k;
    /* Dense calls only (NULL: every key): the forward's key_lengths (kmi_attn_args). */
    const int32_t* key_lengths;
    /* ABI 4: the value head dim Dv (0: head_dim): v, out, grad_out and grad_v [.., Dv]. */
    int64_t head_dim_v;
} kmi_attn_bwd_args;

/* Bytes of workspace kmi_attn_bwd needs for `args`. */
int kmi_attn_bwd_workspace_bytes(const kmi_attn_bwd_args* args, size_t* bytes);

/* Enqueues the attention backward of `args` on `stream` (hipStream_t). */
int kmi_attn_bwd(const kmi_attn_bwd_args* args, void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * LayerNorm forward over rows of `width` contiguous elements:
 *   y = (x - mean) * rstd * weight + bias, rstd = 1 / sqrt(max(var, 0) + eps),
 * mean / rstd written as fp32 [rows] (either may be NULL).  weight / bias may be NULL;
 * x / y dtype BF16, F16 or F32; weight / bias BF16, F16 or F32.
 * Does the work of the reference's bridge::layer_norm (device_norm.cpp:235-300;
 * ktt_norm::forward, ktt_norm/program.cpp:436).
 */
int kmi_layer_norm_fwd(const void* x, const void* weight, const void* bias, void* y,
                       float* mean, float* rstd, int64_t rows, int64_t width,
                       int32_t x_dtype, int32_t w_dtype, int32_t b_dtype, double eps,
                       void* stream);

/*
 * RMSNorm forward: y = x * rstd * weight (+ bias), rstd = 1 / sqrt(mean(x^2) + eps),
 * rstd written as fp32 [rows] (may be NULL).
 * Does the work of the reference's bridge::rms_norm (device_norm.cpp:203-233) and of
 * ktt::rms_norm with bias (aten_fused.cpp:60-85).
 */
int kmi_rms_norm_fwd(const void* x, const void* weight, const void* bias, void* y,
                     float* rstd, int64_t rows, int64_t width, int32_t x_dtype,
                     int32_t w_dtype, int32_t b_dtype, double eps, void* stream);

/*
 * RMSNorm backward over rows of `width` contiguous elements, from the forward's fp32 rstd:
 *   dx = rstd * (dy * weight) - x * rstd^3 * mean(dy * weight * x)   (per row),
 *   dweight = sum over rows of dy * x * rstd                          (per column).
 * dy / dx have x's dtype (BF16, F16 or F32); weight / dweight w_dtype; weight may be NULL
 * (then dweight must be NULL).  dweight needs kmi_rms_norm_bwd_workspace_bytes of fp32
 * workspace (per-block column sums, added in a fixed order: deterministic).  Rows of
 * whole 16-byte vectors take one pass over dy and x (as kmi_layer_norm_bwd); others an
 * element path.
 * Does the work of the reference's RMSNorm training backward (RmsNormFunction, aten_norm.cpp:
 * 548-599; ktt_norm backward and column-sum programs, layernorm.md:90-102).
 */
int kmi_rms_norm_bwd_workspace_bytes(int64_t rows, int64_t width, size_t* bytes);

int kmi_rms_norm_bwd(const void* dy, const void* x, const void* weight, const float* rstd,
                     void* dx, void* dweight, int64_t rows, int64_t width, int32_t x_dtype,
                     int32_t w_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * LayerNorm backward over rows of `width` contiguous elements, from the forward's fp32
 * mean and rstd:
 *   xh = (x - mean) * rstd, g = dy * weight (dy without a weight),
 *   dx = rstd * (g - mean_row(g) - xh * mean_row(g * xh))            (per row),
 *   dweight = sum over rows of dy * xh, dbias = sum over rows of dy   (per column).
 * dy / dx have x's dtype (BF16, F16 or F32); weight / dweight w_dtype (x's or F32);
 * dbias b_dtype; weight, dweight and dbias may be NULL (dweight needs weight).  Rows must
 * be whole 16-byte vectors, 16-byte aligned, at most 256 vectors (else KMI_EUNSUPPORTED).
 * dx in one pass over dy and x; dweight / dbias from per-block partial sums added in a
 * fixed order (deterministic), in kmi_layer_norm_bwd_workspace_bytes of fp32 workspace.
 * Does the work of the reference's native_layer_norm_backward on its own programs
 * (aten_norm.cpp:130-224,811; ktt_norm bwd_* and colsum_* programs, layernorm.md:90-102).
 */
int kmi_layer_norm_bwd_workspace_bytes(int64_t rows, int64_t width, size_t* bytes);

int kmi_layer_norm_bwd(const void* dy, const void* x, const float* mean, const float* rstd,
                       const void* weight, void* dx, void* dweight, void* dbias, int64_t rows,
                       int64_t width, int32_t x_dtype, int32_t w_dtype, int32_t b_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* The message of the last failed call on this thread ("" if none). */
const char* kmi_last_error(void);

/* KMI_ABI_VERSION of the loaded library. */
int kmi_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KOHAKUTT_AMD_H */
