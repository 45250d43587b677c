// Attention forward, host side: argument checks, the launch plan and the C ABI entry
// points (kmi_attn_workspace_bytes, kmi_attn_fwd).  The kernels are in
// attention_kernels.hpp, instantiated per padded head dim in attention_d<D>.hip; what they
// compute and how is described there.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "attention_params.hpp"

namespace kmi {
namespace fwd {
namespace {


// The value / output head dim, and the padded dim the kernels run at (the larger of q's
// and v's).
int64_t value_dim(const kmi_attn_args* a) { return a->head_dim_v > 0 ? a->head_dim_v : a->head_dim; }
int kernel_dim(const kmi_attn_args* a) { return padded_head_dim(std::max<int64_t>(a->head_dim, value_dim(a))); }

const char* check_args(const kmi_attn_args* a) {
    if (!a) return "null args";
    if (a->dtype != KMI_BF16 && a->dtype != KMI_F16) return "dtype must be BF16 or F16";
    if (!head_dim_supported(a->head_dim)) return "head_dim must be a multiple of 8 up to 256";
    if (a->head_dim_v != 0 && !head_dim_supported(a->head_dim_v))
        return "head_dim_v must be 0 or a multiple of 8 up to 256";
    if (a->batch <= 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->seq_q < 0 || a->seq_k <= 0)
        return "sizes must be positive (seq_q may be 0)";
    if (a->heads_q % a->heads_kv != 0) return "heads_kv must divide heads_q";
    if (a->key_lengths && a->cu_seqlens_q) return "key_lengths are for dense calls (varlen has cu_seqlens_k)";
    if (!a->q || !a->k || !a->v || !a->out) return "null q, k, v or out";
    for (const void* ptr : {a->q, a->k, a->v})
        if (reinterpret_cast<uintptr_t>(ptr) % 16) return "q, k and v must be 16-byte aligned";
    if (reinterpret_cast<uintptr_t>(a->out) % 8) return "out must be 8-byte aligned";
    for (int i = 0; i < 3; ++i) {
        if (a->q_stride[i] % 8 || a->k_stride[i] % 8 || a->v_stride[i] % 8)
            return "q, k and v strides must be multiples of 8 elements";
        if (a->o_stride[i] % 4) return "out strides must be multiples of 4 elements";
    }
    if (a->k_stride[2] < 0 || a->k_stride[2] > (1 << 24) || a->v_stride[2] < 0 || a->v_stride[2] > (1 << 24))
        return "k and v row strides must be within [0, 2^24] elements";
    if (a->seq_q > (1 << 30) / 64 || a->seq_k > (1 << 30) || a->heads_q > 65536)
        return "sizes too large";
    const bool varlen = a->cu_seqlens_q != nullptr;
    if (varlen != (a->cu_seqlens_k != nullptr)) return "cu_seqlens_q and cu_seqlens_k go together";
    if (varlen && (a->total_q < 0 || a->total_k <= 0 || a->total_q > (1 << 30) / 64 || a->total_k > (1 << 30)))
        return "varlen totals out of range";
    if (a->mask_mode != KMI_MASK_NONE) {
        if (!a->mask) return "mask_mode set without a mask";
        if (a->mask_dtype < KMI_BF16 || a->mask_dtype > KMI_BOOL) return "bad mask dtype";
        if (a->mask_mode == KMI_MASK_PACKED && !varlen) return "packed masks are varlen only";
        if (a->mask_mode != KMI_MASK_STRIDED && a->mask_mode != KMI_MASK_PACKED) return "bad mask mode";
        if (a->mask_mode == KMI_MASK_PACKED && a->mask_numel <= 0) return "packed masks need mask_numel";
        if (a->mask_mode == KMI_MASK_PACKED && a->mask_stride[1] != 0) return "packed masks are shared by the heads";
    }
    return nullptr;
}

// KMI_ATTN_NQB=1|2|4 (read once) pins the 16-row blocks of a workgroup; by default a
// workgroup holds 64 rows for padded head dim 64, 32 up to 128 and 16 above (its
// wavefronts read each K/V tile once for all those rows: 4 * rows FLOPs per LDS byte).
int nqb_override() {
    static const int v = [] {
        const char* e = std::getenv("KMI_ATTN_NQB");
        return e ? std::atoi(e) : 0;
    }();
    return v;
}

// KMI_ATTN_PIPE=0 (read once) keeps head-dim-64 prefill calls on attn_fwd_kernel.
bool pipe_enabled() {
    static const bool v = [] {
        const char* e = std::getenv("KMI_ATTN_PIPE");
        return !(e && std::atoi(e) == 0);
    }();
    return v;
}

// KMI_ATTN_DECODE_FUSED=0 (read once) merges decode splits in a separate launch.
bool decode_fused_enabled() {
    static const bool v = [] {
        const char* e = std::getenv("KMI_ATTN_DECODE_FUSED");
        return !(e && std::atoi(e) == 0);
    }();
    return v;
}

// KMI_ATTN_SPLITS=n (read once) pins the split-KV count of calls the plan would split.
int splits_override() {
    static const int v = [] {
        const char* e = std::getenv("KMI_ATTN_SPLITS");
        return e ? std::atoi(e) : 0;
    }();
    return v;
}

// The row-block counts a padded head dim is instantiated for: 1, 2 up to 128, 4 at 64
// (masked: 2 at 64, 1 above).
bool nqb_allowed(int dp, int nqb, bool masked) {
    if (masked) return nqb == 1 || (nqb == 2 && dp == 64);
    return nqb == 1 || (nqb == 2 && dp <= 128) || (nqb == 4 && dp == 64);
}

Plan make_plan(const kmi_attn_args* a) {
    Plan pl{};
    const int64_t G = a->heads_q / a->heads_kv;
    const int64_t vrows = a->seq_q * G;
    const int64_t units = a->batch * a->heads_kv;
    const int dp = padded_head_dim(std::max<int64_t>(a->head_dim, value_dim(a)));
    int nqb = dp == 64 ? 4 : (dp <= 128 ? 2 : 1);
    // Fewer rows per workgroup when the larger tile would leave under two workgroups per
    // CU, and short query tiles (decode: Sq x G rows per K/V head) take only what they have.
    if (nqb == 4 && ceil_div(vrows, 64) * units < 512) nqb = 2;
    // Under one 32-row workgroup per CU: 16-row workgroups (twice the workgroups to
    // overlap each other's latency; C2 at batch 1: 6.5 -> 5.3 us).
    if (nqb == 2 && ceil_div(vrows, 32) * units < 256) nqb = 1;
    while (nqb > 1 && vrows <= 16 * (nqb / 2)) nqb /= 2;
    // Masked variants carry the prefetched mask values: one row block fewer keeps them
    // at two wavefronts per SIMD.
    if (a->mask_mode != KMI_MASK_NONE) nqb = std::min(nqb, dp == 64 ? 2 : 1);
    const int forced = nqb_override();
    if (nqb_allowed(dp, forced, a->mask_mode != KMI_MASK_NONE)) nqb = forced;
    // K or V rows that overlap in memory (a row stride below the head dim, from an
    // as_strided view) take the 16-row variants, whose tile loads read each row in full
    // (the LDS DMA variants' ranges assume whole strides per row).
    const bool overlap = (a->k_stride[2] > 0 && a->k_stride[2] < a->head_dim) ||
                         (a->v_stride[2] > 0 && a->v_stride[2] < value_dim(a));
    if (overlap) nqb = 1;
    pl.nqb = nqb;
    const int64_t bm = 16 * pl.nqb;
    pl.nx = static_cast<int>(ceil_div(vrows, bm));
    const int64_t nk = ceil_div(a->seq_k, WN);
    const int64_t base = static_cast<int64_t>(pl.nx) * units;
    // Split the keys across workgroups when the query tiles alone leave most CUs idle
    // (decode): about two workgroups per CU, at least one tile per wavefront per split.
    int64_t splits = 1;
    if (a->num_splits == 0) {
        if (base < 128 && nk >= 8) {
            splits = std::min<int64_t>(ceil_div(512, base), nk / NWAVES);
            if (splits_override() > 0) splits = std::min<int64_t>(splits_override(), nk);
        }
    } else {
        splits = std::max<int64_t>(1, std::min<int64_t>(a->num_splits, nk));
    }
    pl.tiles_per_split = static_cast<int>(ceil_div(nk, splits));
    pl.splits = static_cast<int>(ceil_div(nk, pl.tiles_per_split));
    // Decode (at most 16 rows per K/V head): four wavefronts per workgroup deal the key
    // tiles round-robin and merge in LDS; about one workgroup per CU in all, at most 32 per
    // unit (the split counter's bits), at least one tile per wavefront.  One workgroup per
    // unit writes the output directly.  (Fewer, longer splits: each split costs the merge a
    // partial and each workgroup a fixed start-up; C3 at 16 splits and the 128-unit sweep at
    // 2 ran faster than at 32 and 4.)
    pl.decode = vrows <= 16 && a->num_splits != 1;
    if (pl.decode) {
        const int64_t most = std::max<int64_t>(1, ceil_div(nk, NWAVES));
        int64_t wgs = std::min<int64_t>({ceil_div(256, units), int64_t{32}, most});
        if (a->num_splits > 1) wgs = std::min<int64_t>(a->num_splits, most);
        if (splits_override() > 0) wgs = std::min<int64_t>(splits_override(), most);
        // The partials (fp32, [splits][rows][Hq][D]) stay under 2^31 bytes: the kernels
        // address them with 32-bit buffer offsets.
        const int64_t rows = a->cu_seqlens_q ? a->total_q : a->batch * a->seq_q;
        const int64_t per_split = rows * a->heads_q * (dp + 2) * static_cast<int64_t>(sizeof(float));
        wgs = std::max<int64_t>(1, std::min<int64_t>(wgs, ((int64_t{1} << 31) - 1) / std::max<int64_t>(per_split, 1)));
        pl.splits = static_cast<int>(wgs);
        pl.tiles_per_split = static_cast<int>(ceil_div(nk, wgs));
        pl.nqb = 1;
        pl.nx = 1;
    }
    // Short unmasked, non-causal key ranges (at most 8 tiles): each wavefront takes its own
    // row block and every key tile, so no wavefront waits on a merge -- when that still
    // gives every CU a workgroup.
    if (!pl.decode && pl.splits == 1 && !a->causal && a->mask_mode == KMI_MASK_NONE && nk <= 8 && dp <= 128) {
        int q = dp == 64 ? (ceil_div(vrows, 256) * units >= 512 ? 4 : 2) : 1;
        if (nqb_allowed(dp, forced, false)) q = forced;
        if (overlap) q = 1;
        const int64_t nx_rs = ceil_div(vrows, NWAVES * 16 * q);
        if (nx_rs * units >= 256) {
            pl.rs = true;
            pl.rs_shared = nk <= kRsTiles;
            pl.nqb = q;
            pl.nx = static_cast<int>(nx_rs);
        }
    }
    // Causal head-dim-64 unmasked dense prefill with 16-byte output rows: the kernel of
    // attention_pipe.hip (non-causal calls keep 64-row tiles, which read K/V from L2 half
    // as often per row).
    bool out16 = reinterpret_cast<uintptr_t>(a->out) % 16 == 0;
    for (int i = 0; i < 3; ++i) out16 = out16 && a->o_stride[i] % 8 == 0;
    // Its buffer resources span a unit's keys with 32-bit offsets.
    const bool span32 = a->seq_k * std::max<int64_t>({a->k_stride[2], a->v_stride[2], 64}) * 2 < (int64_t{1} << 31);
    pl.pipe = a->causal && !pl.decode && !pl.rs && pl.splits == 1 && a->mask_mode == KMI_MASK_NONE && !a->cu_seqlens_q &&
              !a->key_lengths && a->head_dim == 64 && value_dim(a) == 64 && out16 && span32 && pipe_enabled();
    pl.rows_total = a->cu_seqlens_q ? a->total_q : a->batch * a->seq_q;
    pl.ws_bytes = 0;
    return pl;
}

// Split partials are indexed by query row: b * Sq + i (dense) or the packed token (varlen).
template <typename T>
hipError_t launch_dim(const AttnParams& p, const Plan& pl, hipStream_t s) {
    if (pl.pipe) return launch_pipe<T>(p, s);
    switch (padded_head_dim(std::max(p.d, p.dv))) {
        case 32: return launch_all<T, 32>(p, pl, s);
        case 64: return launch_all<T, 64>(p, pl, s);
        case 96: return launch_all<T, 96>(p, pl, s);
        case 128: return launch_all<T, 128>(p, pl, s);
        case 192: return launch_all<T, 192>(p, pl, s);
        default: return launch_all<T, 256>(p, pl, s);
    }
}

size_t ws_bytes_for(const kmi_attn_args* a, const Plan& pl) {
    if (pl.splits <= 1) return 0;
    return static_cast<size_t>(pl.splits) * pl.rows_total * a->heads_q * (kernel_dim(a) + 2) *
           sizeof(float);
}


}  // namespace

// Compute units of the current device (cached per device id).
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Enqueues a checked, planned call; `workspace` holds the plan's split partials (when it
// splits).
int enqueue(const kmi_attn_args* a, const Plan& pl, void* workspace, void* stream, const char* name) {
    AttnParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.out = a->out;
    p.lse = a->lse;
    for (int i = 0; i < 3; ++i) {
        p.qs[i] = a->q_stride[i];
        p.ks[i] = a->k_stride[i];
        p.vs[i] = a->v_stride[i];
        p.os[i] = a->o_stride[i];
        p.ls[i] = a->lse_stride[i];
    }
    p.mask = a->mask_mode == KMI_MASK_NONE ? nullptr : a->mask;
    p.mask_mode = a->mask_mode;
    p.mask_dtype = a->mask_dtype;
    for (int i = 0; i < 4; ++i) p.ms[i] = a->mask_stride[i];
    p.mask_numel = a->mask_numel;
    p.mask_off = a->mask_mode == KMI_MASK_PACKED ? a->mask_offsets : nullptr;
    {
        p.mask_vec4 = a->mask_mode == KMI_MASK_PACKED || (a->mask_mode == KMI_MASK_STRIDED && a->mask_stride[3] == 1);
    }
    p.cu_q = a->cu_seqlens_q;
    p.cu_k = a->cu_seqlens_k;
    p.klen = a->key_lengths;
    p.batch = static_cast<int>(a->batch);
    p.hq = static_cast<int>(a->heads_q);
    p.hkv = static_cast<int>(a->heads_kv);
    p.group = p.hq / p.hkv;
    p.seq_q = static_cast<int>(a->seq_q);
    p.seq_k = static_cast<int>(a->seq_k);
    p.d = static_cast<int>(a->head_dim);
    p.dv = static_cast<int>(value_dim(a));
    p.causal = a->causal ? 1 : 0;
    p.scale_log2 = static_cast<float>(a->scale * 1.4426950408889634);
    p.splits = pl.splits;
    p.tiles_per_split = pl.tiles_per_split;
    p.nx = pl.nx;
    p.rows_total = pl.rows_total;
    p.rs_shared = pl.rs && pl.rs_shared ? 1 : 0;
    p.total_q = static_cast<int>(a->total_q);
    p.total_k = static_cast<int>(a->total_k);
    p.fd_splits = fast_div(static_cast<uint32_t>(p.splits));
    p.fd_units = fast_div(static_cast<uint32_t>(p.batch * p.hkv));
    p.fd_hkv = fast_div(static_cast<uint32_t>(p.hkv));
    p.fd_group = fast_div(static_cast<uint32_t>(p.group));
    if (pl.splits > 1) {
        p.part_o = static_cast<float*>(workspace);
        p.part_lse = p.part_o + static_cast<size_t>(pl.splits) * p.rows_total * p.hq * kernel_dim(a);
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (pl.decode && pl.splits > 1 && pl.splits <= 32)
        p.ctr = decode_counters(s, static_cast<int64_t>(p.batch) * p.hkv);
    const hipError_t err = a->dtype == KMI_BF16 ? launch_dim<bf16>(p, pl, s) : launch_dim<f16>(p, pl, s);
    return hip_status(err, name);
}

// Scratch of kmi_attn_fwd_noalloc: split-KV partials in a file-scope device array (each
// device holds its own copy for the life of the process), so that entry point allocates
// nothing.  Calls that overlap on one device share it and race; every partial a call's
// merge reads is written by that call first, so nothing needs clearing between calls.
constexpr size_t kScratchBytes = size_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The scratch's device address on the current device, looked up once per device (with
// that device current); nullptr when the lookup fails.
void* scratch_on_current_device() {
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        addr[dev] = ptr;
    }
    return addr[dev];
}

// Decode split counters: kCtrSlabs slabs of kCtrUnits 64-bit words, zero from the load of
// the code object on and left zero by every merge (the last workgroup of a unit clears its
// word).  A slab belongs to one stream for the life of the process, so calls on one
// stream (which run in order) share it and calls on different streams never do; a stream
// beyond the slab count, or a call over more units, merges in a separate launch instead
// (the same arithmetic, so the results do not depend on which).
constexpr int kCtrSlabs = 16;
constexpr int kCtrUnits = 4096;
static __device__ __align__(256) unsigned long long decode_ctr[kCtrSlabs * kCtrUnits];

unsigned long long* decode_counters(hipStream_t stream, int64_t units) {
    if (units > kCtrUnits || !decode_fused_enabled()) return nullptr;
    static std::mutex mu;
    static unsigned long long* base[64] = {};
    static hipStream_t owner[64][kCtrSlabs] = {};
    static int used[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!base[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(decode_ctr)) != hipSuccess) return nullptr;
        base[dev] = static_cast<unsigned long long*>(ptr);
    }
    for (int i = 0; i < used[dev]; ++i)
        if (owner[dev][i] == stream) return base[dev] + static_cast<size_t>(i) * kCtrUnits;
    if (used[dev] == kCtrSlabs) return nullptr;
    owner[dev][used[dev]] = stream;
    return base[dev] + static_cast<size_t>(used[dev]++) * kCtrUnits;
}

}  // namespace fwd
}  // namespace kmi

extern "C" int kmi_attn_workspace_bytes(const kmi_attn_args* args, size_t* bytes) {
    using namespace kmi;
    using namespace kmi::fwd;
    if (!bytes) return fail(KMI_EINVAL, "kmi_attn_workspace_bytes: null bytes");
    if (const char* why = check_args(args)) return fail(KMI_EINVAL, std::string("kmi_attn_workspace_bytes: ") + why);
    *bytes = ws_bytes_for(args, make_plan(args));
    return KMI_OK;
}

extern "C" int kmi_attn_fwd(const kmi_attn_args* a, void* workspace, size_t workspace_bytes, void* stream) {
    using namespace kmi;
    using namespace kmi::fwd;
    if (const char* why = check_args(a)) return fail(KMI_EINVAL, std::string("kmi_attn_fwd: ") + why);
    if (a->seq_q == 0) return KMI_OK;
    const Plan pl = make_plan(a);
    const size_t need = ws_bytes_for(a, pl);
    if (need > 0 && (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16))
        return fail(KMI_EWORKSPACE, "kmi_attn_fwd: workspace missing, misaligned or smaller than "
                                    "kmi_attn_workspace_bytes");
    return enqueue(a, pl, workspace, stream, "kmi_attn_fwd");
}

extern "C" int kmi_attn_fwd_noalloc(const kmi_attn_args* a, void* stream) {
    using namespace kmi;
    using namespace kmi::fwd;
    if (const char* why = check_args(a)) return fail(KMI_EINVAL, std::string("kmi_attn_fwd_noalloc: ") + why);
    if (a->seq_q == 0) return KMI_OK;
    const Plan pl = make_plan(a);
    const size_t need = ws_bytes_for(a, pl);
    if (need > kScratchBytes)
        return fail(KMI_EUNSUPPORTED, "kmi_attn_fwd_noalloc: the call needs " + std::to_string(need) +
                                          " bytes of split-KV scratch, beyond the library's " +
                                          std::to_string(kScratchBytes) +
                                          "; call kmi_attn_fwd with a workspace of kmi_attn_workspace_bytes");
    void* ws = nullptr;
    if (need > 0) {
        ws = scratch_on_current_device();
        if (!ws) return fail(KMI_EHIP, "kmi_attn_fwd_noalloc: the scratch address of the current device is unknown");
    }
    return enqueue(a, pl, ws, stream, "kmi_attn_fwd_noalloc");
}
