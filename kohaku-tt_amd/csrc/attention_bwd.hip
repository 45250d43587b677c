// Attention backward on gfx950 (flash-style: nothing of size Sq x Sk is stored).
//
// The reference's training route recomputes the probabilities from the forward's row
// statistics and runs a dQ pass and a dK/dV pass (docs/reference/kernels/flash.md,
// "Backward", flash.md:151-206; ktt_flash/bw_*.cpp; bridge in device_attention.cpp:
// 1208-1281).  Here, for unmasked dense calls (causal top-left or not, GQA, head dim 64
// or 128, bf16 / fp16):
//
//   attn_bwd_dq      one workgroup per (sequence, query head, 64-row block): the row dots
//                    Dr = sum_d dO O (fp32, kept for the next kernel), then over the key
//                    tiles it sees P = exp2(c S - lse2), dP = dO V^T, dS = P (dP - Dr),
//                    dQ += dS K
//   attn_bwd_dkdv    one workgroup per (sequence, query head, 64-key tile): for every
//                    32-row query block that sees the tile the same P / dS; dV += P^T dO,
//                    dK += dS^T Q (fp32 accumulators in registers).  Without GQA or query
//                    splits it writes dK / dV; otherwise fp32 partials that
//   attn_bwd_group_sum adds over each K/V head's query heads in a fixed order (no atomics)
//
// S = Q K^T, dP = dO V^T and the three gradient products run on
// v_mfma_f32_16x16x32_{bf16,f16}.  Every operand is read from LDS along its contraction
// index (16 contiguous bytes per lane): tiles needed with either index contiguous are
// staged twice, row-major and transposed.  lse is the forward's natural-log row LSE.
#include <algorithm>

#include "common.hpp"

namespace kmi {
namespace {

constexpr int BT = 32;          // keys per K/V tile and rows per query block
constexpr int TP = BT + 8;      // pitch of transposed / [32][32] tiles (elements)
constexpr int BWD_THREADS = 256;
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct BwdMfma;
template <>
struct BwdMfma<bf16> {
    typedef bf16x8 v8;
    static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct BwdMfma<f16> {
    typedef f16x8 v8;
    static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

struct BwdParams {
    const void *q, *k, *v, *o, *dout;
    const float* lse;
    void *dq, *dk, *dv;
    float* dr;  // [batch][hq][seq_q] fp32 workspace
    // GQA (group > 1): per-query-head dK / dV partials [batch][hq][seq_k][D] fp32, summed
    // over each group by attn_bwd_group_sum; null when every K/V head has one query head.
    float *pdk, *pdv;
    // dK / dV workgroups per (query head, key tile): split q takes query blocks q, q + qsplit,
    // ...; with qsplit > 1 every split writes fp32 partials (indexed [b][h][split][key][D]).
    int qsplit;
    // dQ workgroups per (query head, row block): split k takes key tiles k, k + ksplit, ...;
    // with ksplit > 1 every split writes fp32 partials pdq [b][h][split][row][D].
    int ksplit;
    float* pdq;
    int64_t qs[3], ks[3], vs[3], os[3], dos[3], dqs[3], dks[3], dvs[3], ls[3];
    int batch, hq, hkv, group, seq_q, seq_k, causal;
    float scale, c2;  // c2 = scale * log2(e)
};

// Staging of rows [r0, r0 + 32) of a [S, D] operand (row stride rs elements) in two steps:
// loads into registers (D / 64 16-byte chunks per thread, zeros past the end), issued a
// tile ahead, and their LDS stores, row-major at pitch D + 8 and, when dstT is set,
// transposed ([D][TP]).  Consecutive lanes take consecutive rows of one 8-column chunk, so
// the transposed 2-byte stores of a wavefront spread over the banks (with consecutive
// chunks per lane every chunk's column block starts on the same bank).
template <int D>
struct TileRegs {
    u32x4 v[D / 64];
};

template <typename T, int D>
__device__ __forceinline__ void load_regs(const T* src, int64_t rs, int r0, int nrows, TileRegs<D>& t) {
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
        const int c = threadIdx.x + BWD_THREADS * j;
        const int r = c % BT, ch = c / BT;
        const int row = min(r0 + r, nrows - 1);  // in range; rows past the end are dropped below
        const u32x4 val = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(row) * rs + 8 * ch);
        t.v[j] = r0 + r < nrows ? val : u32x4{0u, 0u, 0u, 0u};
    }
}

template <typename T, int D>
__device__ __forceinline__ void store_regs(const TileRegs<D>& t, T* dst, T* dstT) {
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
        const int c = threadIdx.x + BWD_THREADS * j;
        const int r = c % BT, ch = c / BT;
        *reinterpret_cast<u32x4*>(dst + r * (D + 8) + 8 * ch) = t.v[j];
        if (dstT) {
            const auto e = __builtin_bit_cast(typename BwdMfma<T>::v8, t.v[j]);
#pragma unroll
            for (int i = 0; i < 8; ++i) dstT[(8 * ch + i) * TP + r] = e[i];
        }
    }
}

template <typename T, int D>
__device__ __forceinline__ void stage_rows_stats(const BwdParams& p, int b, int h, int r0, float* lse2, float* drs) {
    if (threadIdx.x < BT) {
        const int i = r0 + threadIdx.x;
        const bool ok = i < p.seq_q;
        lse2[threadIdx.x] = ok ? p.lse[b * p.ls[0] + h * p.ls[1] + static_cast<int64_t>(i) * p.ls[2]] * kLog2e
                               : INFINITY;
        drs[threadIdx.x] = ok ? p.dr[(static_cast<int64_t>(b) * p.hq + h) * p.seq_q + i] : 0.f;
    }
}

// dK / dV: a workgroup takes KW keys, wavefront w owns keys [k0 + 16 w, + 16) with its K
// and V fragments in registers (the A operands of S^T = K Q^T and dP^T = V dO^T).  Per
// 32-row query block the workgroup stages Q and dO (row-major and transposed) once; each
// wavefront then forms P^T and dS^T of its keys, passes them through its own LDS rows (one
// wavefront's LDS accesses stay in order: no barrier) and accumulates dV += P^T dO and
// dK += dS^T Q.  Two barriers per query block.
constexpr int KW = 64;

template <typename T, int D>
__global__ __launch_bounds__(BWD_THREADS) void attn_bwd_dkdv(const BwdParams p) {
    typedef typename BwdMfma<T>::v8 v8;
    constexpr int RP = D + 8;
    constexpr int DC = D / 32, DB = D / 16;
    __shared__ __align__(16) T qs[BT * RP];
    __shared__ __align__(16) T dos[BT * RP];
    __shared__ __align__(16) T qt[D * TP];
    __shared__ __align__(16) T dot[D * TP];
    __shared__ __align__(16) T pt[4 * 16 * TP];   // per wavefront: P^T [16 keys][32 rows]
    __shared__ __align__(16) T dst[4 * 16 * TP];  // per wavefront: dS^T
    __shared__ float lse2[BT], drs[BT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4, l16 = lane & 15;
    const int ntk = (p.seq_k + KW - 1) / KW;
    const int qsp = blockIdx.x % p.qsplit;
    const int tile = (blockIdx.x / p.qsplit) % ntk;
    const int bh = blockIdx.x / (p.qsplit * ntk);  // (sequence, query head)
    const int b = bh / p.hq, h = bh - b * p.hq;
    const int kvh = h / p.group;
    const int k0 = tile * KW;
    const int kw0 = k0 + 16 * wave;  // this wavefront's first key

    // K / V fragments: lane (g4, l16) holds key kw0 + l16, dims 32 c + 8 g4 .. + 7.
    v8 kf[DC], vf[DC];
    {
        const int key = kw0 + l16;
        const int kc = min(key, p.seq_k - 1);
        const T* kp = static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1] + static_cast<int64_t>(kc) * p.ks[2];
        const T* vp = static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1] + static_cast<int64_t>(kc) * p.vs[2];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const u32x4 kx = *reinterpret_cast<const u32x4*>(kp + 32 * c + 8 * g4);
            const u32x4 vx = *reinterpret_cast<const u32x4*>(vp + 32 * c + 8 * g4);
            kf[c] = __builtin_bit_cast(v8, key < p.seq_k ? kx : u32x4{0u, 0u, 0u, 0u});
            vf[c] = __builtin_bit_cast(v8, key < p.seq_k ? vx : u32x4{0u, 0u, 0u, 0u});
        }
    }
    f32x4 dk[DB], dv[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) dk[i] = dv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    T* ptw = pt + wave * 16 * TP;
    T* dsw = dst + wave * 16 * TP;

    // Causal (top-left): a query block sees this tile only if its last position reaches k0.
    const int rstart = (p.causal ? (k0 / BT) * BT : 0) + qsp * BT;
    const int rstep = p.qsplit * BT;
    const T* qbase = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1];
    const T* dobase = static_cast<const T*>(p.dout) + b * p.dos[0] + h * p.dos[1];
    TileRegs<D> qr, dor;
    if (rstart < p.seq_q) {
        load_regs<T, D>(qbase, p.qs[2], rstart, p.seq_q, qr);
        load_regs<T, D>(dobase, p.dos[2], rstart, p.seq_q, dor);
    }
    for (int r0 = rstart; r0 < p.seq_q; r0 += rstep) {
        __syncthreads();  // the previous block's LDS reads are done
        store_regs<T, D>(qr, qs, qt);
        store_regs<T, D>(dor, dos, dot);
        stage_rows_stats<T, D>(p, b, h, r0, lse2, drs);
        __syncthreads();
        if (r0 + rstep < p.seq_q) {  // the next block's loads overlap this block's products
            load_regs<T, D>(qbase, p.qs[2], r0 + rstep, p.seq_q, qr);
            load_regs<T, D>(dobase, p.dos[2], r0 + rstep, p.seq_q, dor);
        }
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            // S^T and dP^T of this wavefront's 16 keys x rows rb 16 .. + 15: lane (g4, l16)
            // gets keys 4 g4 + j, row l16.
            f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dpt = st;
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const v8 qb = *reinterpret_cast<const v8*>(qs + (rb * 16 + l16) * RP + 32 * c + 8 * g4);
                const v8 ob = *reinterpret_cast<const v8*>(dos + (rb * 16 + l16) * RP + 32 * c + 8 * g4);
                st = BwdMfma<T>::run(kf[c], qb, st);
                dpt = BwdMfma<T>::run(vf[c], ob, dpt);
            }
            const int rl = rb * 16 + l16;
            const int pos = r0 + rl;
            const float l2 = lse2[rl], dr = drs[rl];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = kw0 + 4 * g4 + j;
                const bool keep = key < p.seq_k && (!p.causal || key <= pos);
                // Rows past the end carry lse2 = +inf: their P is exactly 0.
                const float e = keep ? __builtin_amdgcn_exp2f(st[j] * p.c2 - l2) : 0.f;
                ptw[(4 * g4 + j) * TP + rl] = from_f32<T>(e);
                dsw[(4 * g4 + j) * TP + rl] = from_f32<T>(e * (dpt[j] - dr));
            }
        }
        // The compiler keeps these LDS reads after the stores above (same arrays); the
        // hardware runs one wavefront's LDS accesses in order.
        __asm__ volatile("" ::: "memory");
        const v8 pa = *reinterpret_cast<const v8*>(ptw + l16 * TP + 8 * g4);
        const v8 sa = *reinterpret_cast<const v8*>(dsw + l16 * TP + 8 * g4);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const v8 ob = *reinterpret_cast<const v8*>(dot + (db * 16 + l16) * TP + 8 * g4);
            const v8 qb = *reinterpret_cast<const v8*>(qt + (db * 16 + l16) * TP + 8 * g4);
            dv[db] = BwdMfma<T>::run(pa, ob, dv[db]);
            dk[db] = BwdMfma<T>::run(sa, qb, dk[db]);
        }
    }
    // Lane (g4, l16) of block db holds keys kw0 + 4 g4 + j, dim db 16 + l16.
    if (p.pdk) {
        const int64_t base = ((static_cast<int64_t>(b) * p.hq + h) * p.qsplit + qsp) * p.seq_k;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = db * 16 + l16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = kw0 + 4 * g4 + j;
                if (key < p.seq_k) {
                    p.pdk[(base + key) * D + d] = dk[db][j] * p.scale;
                    p.pdv[(base + key) * D + d] = dv[db][j];
                }
            }
        }
        return;
    }
    T* dkp = static_cast<T*>(p.dk) + b * p.dks[0] + kvh * p.dks[1];
    T* dvp = static_cast<T*>(p.dv) + b * p.dvs[0] + kvh * p.dvs[1];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const int d = db * 16 + l16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = kw0 + 4 * g4 + j;
            if (key < p.seq_k) {
                dkp[static_cast<int64_t>(key) * p.dks[2] + d] = from_f32<T>(dk[db][j] * p.scale);
                dvp[static_cast<int64_t>(key) * p.dvs[2] + d] = from_f32<T>(dv[db][j]);
            }
        }
    }
}

// dK / dV of a K/V head: the sum of its query heads' fp32 partials (and of their query
// splits), in a fixed order.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_group_sum(const BwdParams p) {
    constexpr int Q = D / 4;  // float4 items per key row
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t items = static_cast<int64_t>(p.batch) * p.hkv * p.seq_k * Q;
    if (item >= items) return;
    const int c = static_cast<int>(item % Q);
    const int key = static_cast<int>((item / Q) % p.seq_k);
    const int64_t bk = item / (static_cast<int64_t>(Q) * p.seq_k);  // b * hkv + kvh
    const int b = static_cast<int>(bk / p.hkv), kvh = static_cast<int>(bk % p.hkv);
    f32x4 sk = f32x4{0.f, 0.f, 0.f, 0.f}, sv = sk;
    for (int g = 0; g < p.group; ++g) {
        for (int q = 0; q < p.qsplit; ++q) {
            const int64_t row =
                ((static_cast<int64_t>(b) * p.hq + kvh * p.group + g) * p.qsplit + q) * p.seq_k + key;
            sk += *reinterpret_cast<const f32x4*>(p.pdk + row * D + 4 * c);
            sv += *reinterpret_cast<const f32x4*>(p.pdv + row * D + 4 * c);
        }
    }
    T* dkp = static_cast<T*>(p.dk) + b * p.dks[0] + kvh * p.dks[1] + static_cast<int64_t>(key) * p.dks[2] + 4 * c;
    T* dvp = static_cast<T*>(p.dv) + b * p.dvs[0] + kvh * p.dvs[1] + static_cast<int64_t>(key) * p.dvs[2] + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        dkp[e] = from_f32<T>(sk[e]);
        dvp[e] = from_f32<T>(sv[e]);
    }
}

// dQ: a workgroup takes QW query rows, wavefront w owns rows [r0 + 16 w, + 16) with its Q
// and dO fragments in registers (the A operands of S = Q K^T and dP = dO V^T).  Per
// 32-key tile the workgroup stages K (row-major and transposed) and V once; each wavefront
// forms dS of its rows, passes it through its own LDS rows and accumulates dQ += dS K.
constexpr int QW = 64;

template <typename T, int D>
__global__ __launch_bounds__(BWD_THREADS) void attn_bwd_dq(const BwdParams p) {
    typedef typename BwdMfma<T>::v8 v8;
    constexpr int RP = D + 8;
    constexpr int DC = D / 32, DB = D / 16;
    __shared__ __align__(16) T ks[BT * RP];
    __shared__ __align__(16) T vs[BT * RP];
    __shared__ __align__(16) T kt[D * TP];
    __shared__ __align__(16) T dss[4 * 16 * TP];  // per wavefront: dS [16 rows][32 keys]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4, l16 = lane & 15;
    const int nqb = (p.seq_q + QW - 1) / QW;
    const int ksp = blockIdx.x % p.ksplit;
    const int qb = (blockIdx.x / p.ksplit) % nqb;
    const int bh = blockIdx.x / (p.ksplit * nqb);
    const int b = bh / p.hq, h = bh - b * p.hq;
    const int kvh = h / p.group;
    const int r0 = qb * QW;
    const int rw0 = r0 + 16 * wave;  // this wavefront's first row

    // Q / dO fragments: lane (g4, l16) holds row rw0 + l16, dims 32 c + 8 g4 .. + 7; the
    // row statistics of row rw0 + 4 g4 + j (the rows of its accumulator lanes).  The row
    // dot D = sum(dO * O) is formed here from the same dO fragments and written for the
    // dK / dV kernel, which runs after this one.
    v8 qf[DC], of[DC];
    float rdot = 0.f;
    {
        const int row = rw0 + l16;
        const int rc = min(row, p.seq_q - 1);
        const T* qp = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1] + static_cast<int64_t>(rc) * p.qs[2];
        const T* op = static_cast<const T*>(p.dout) + b * p.dos[0] + h * p.dos[1] + static_cast<int64_t>(rc) * p.dos[2];
        const T* outp = static_cast<const T*>(p.o) + b * p.os[0] + h * p.os[1] + static_cast<int64_t>(rc) * p.os[2];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const u32x4 qx = *reinterpret_cast<const u32x4*>(qp + 32 * c + 8 * g4);
            const u32x4 ox = *reinterpret_cast<const u32x4*>(op + 32 * c + 8 * g4);
            const v8 yv = *reinterpret_cast<const v8*>(outp + 32 * c + 8 * g4);
            qf[c] = __builtin_bit_cast(v8, row < p.seq_q ? qx : u32x4{0u, 0u, 0u, 0u});
            of[c] = __builtin_bit_cast(v8, row < p.seq_q ? ox : u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int e = 0; e < 8; ++e) rdot += to_f32(of[c][e]) * to_f32(yv[e]);
        }
    }
    // The four lanes of a row (g4 = 0..3) each hold a quarter of its dims.
    rdot += __shfl_xor(rdot, 16, kWave);
    rdot += __shfl_xor(rdot, 32, kWave);
    if (ksp == 0 && g4 == 0 && rw0 + l16 < p.seq_q) p.dr[(static_cast<int64_t>(b) * p.hq + h) * p.seq_q + rw0 + l16] = rdot;
    float l2[4], drv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = rw0 + 4 * g4 + j;
        const int rc = min(row, p.seq_q - 1);
        const float lv = p.lse[b * p.ls[0] + h * p.ls[1] + static_cast<int64_t>(rc) * p.ls[2]];
        const float dv = __shfl(rdot, 4 * g4 + j, kWave);  // lane 4 g4 + j holds that row's dot
        // Rows past the end: lse2 = +inf makes their P exactly 0.
        l2[j] = row < p.seq_q ? lv * kLog2e : INFINITY;
        drv[j] = row < p.seq_q ? dv : 0.f;
    }
    f32x4 dq[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) dq[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    T* dsw = dss + wave * 16 * TP;

    const int kend = p.causal ? min(p.seq_k, r0 + QW) : p.seq_k;
    const T* kbase = static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1];
    const T* vbase = static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1];
    TileRegs<D> kr, vr;
    const int kstep = p.ksplit * BT;
    load_regs<T, D>(kbase, p.ks[2], ksp * BT, p.seq_k, kr);
    load_regs<T, D>(vbase, p.vs[2], ksp * BT, p.seq_k, vr);
    for (int k0 = ksp * BT; k0 < kend; k0 += kstep) {
        __syncthreads();
        store_regs<T, D>(kr, ks, kt);
        store_regs<T, D>(vr, vs, nullptr);
        __syncthreads();
        if (k0 + kstep < kend) {  // the next tile's loads overlap this tile's products
            load_regs<T, D>(kbase, p.ks[2], k0 + kstep, p.seq_k, kr);
            load_regs<T, D>(vbase, p.vs[2], k0 + kstep, p.seq_k, vr);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            // S and dP of this wavefront's 16 rows x keys kb 16 .. + 15: lane (g4, l16)
            // gets rows 4 g4 + j, key l16.
            f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f}, dpv = sv;
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const v8 kbv = *reinterpret_cast<const v8*>(ks + (kb * 16 + l16) * RP + 32 * c + 8 * g4);
                const v8 vbv = *reinterpret_cast<const v8*>(vs + (kb * 16 + l16) * RP + 32 * c + 8 * g4);
                sv = BwdMfma<T>::run(qf[c], kbv, sv);
                dpv = BwdMfma<T>::run(of[c], vbv, dpv);
            }
            const int key = k0 + kb * 16 + l16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int pos = rw0 + 4 * g4 + j;
                const bool keep = key < p.seq_k && (!p.causal || key <= pos);
                const float e = keep ? __builtin_amdgcn_exp2f(sv[j] * p.c2 - l2[j]) : 0.f;
                dsw[(4 * g4 + j) * TP + kb * 16 + l16] = from_f32<T>(e * (dpv[j] - drv[j]));
            }
        }
        // The compiler keeps this LDS read after the stores above (same array); the hardware
        // runs one wavefront's LDS accesses in order.
        __asm__ volatile("" ::: "memory");
        const v8 da = *reinterpret_cast<const v8*>(dsw + l16 * TP + 8 * g4);
#pragma unroll
        for (int db = 0; db < DB; ++db)
            dq[db] = BwdMfma<T>::run(da, *reinterpret_cast<const v8*>(kt + (db * 16 + l16) * TP + 8 * g4), dq[db]);
    }
    // Lane (g4, l16) of block db holds rows rw0 + 4 g4 + j, dim db 16 + l16.
    if (p.pdq) {
        float* dst = p.pdq + ((static_cast<int64_t>(b) * p.hq + h) * p.ksplit + ksp) * p.seq_q * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = db * 16 + l16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = rw0 + 4 * g4 + j;
                if (row < p.seq_q) dst[static_cast<int64_t>(row) * D + d] = dq[db][j] * p.scale;
            }
        }
        return;
    }
    T* dqp = static_cast<T*>(p.dq) + b * p.dqs[0] + h * p.dqs[1];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const int d = db * 16 + l16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = rw0 + 4 * g4 + j;
            if (row < p.seq_q) dqp[static_cast<int64_t>(row) * p.dqs[2] + d] = from_f32<T>(dq[db][j] * p.scale);
        }
    }
}

// dQ: the sum of the key splits' fp32 partials, in split order.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_sum(const BwdParams p) {
    constexpr int Q = D / 4;
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t items = static_cast<int64_t>(p.batch) * p.hq * p.seq_q * Q;
    if (item >= items) return;
    const int c = static_cast<int>(item % Q);
    const int row = static_cast<int>((item / Q) % p.seq_q);
    const int64_t bh = item / (static_cast<int64_t>(Q) * p.seq_q);
    const int b = static_cast<int>(bh / p.hq), h = static_cast<int>(bh % p.hq);
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < p.ksplit; ++k)
        acc += *reinterpret_cast<const f32x4*>(p.pdq + ((bh * p.ksplit + k) * p.seq_q + row) * D + 4 * c);
    T* dst = static_cast<T*>(p.dq) + b * p.dqs[0] + h * p.dqs[1] + static_cast<int64_t>(row) * p.dqs[2] + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(acc[e]);
}

const char* check_bwd(const kmi_attn_bwd_args* a) {
    if (!a) return "null args";
    if (a->dtype != KMI_BF16 && a->dtype != KMI_F16) return "dtype must be BF16 or F16";
    if (a->head_dim != 64 && a->head_dim != 128) return "head_dim must be 64 or 128";
    if (a->batch <= 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->seq_q <= 0 || a->seq_k <= 0)
        return "sizes must be positive";
    if (a->heads_q % a->heads_kv != 0) return "heads_kv must divide heads_q";
    if (a->batch * a->heads_q * a->seq_q > (int64_t{1} << 31) || a->seq_q > (1 << 30) || a->seq_k > (1 << 30))
        return "sizes too large";
    const void* ptrs[] = {a->q, a->k, a->v, a->out, a->grad_out, a->lse, a->grad_q, a->grad_k, a->grad_v};
    for (const void* ptr : ptrs)
        if (!ptr) return "null tensor pointer";
    const void* vec[] = {a->q, a->k, a->v, a->out, a->grad_out};
    for (const void* ptr : vec)
        if (reinterpret_cast<uintptr_t>(ptr) % 16) return "q, k, v, out and grad_out must be 16-byte aligned";
    const int64_t* strides[] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride, a->do_stride};
    for (const int64_t* s : strides)
        for (int i = 0; i < 3; ++i)
            if (s[i] < 0 || s[i] % 8) return "q, k, v, out and grad_out strides must be non-negative multiples of 8";
    return nullptr;
}

// dK / dV query splits: enough workgroups for about two per CU (at most 4 splits, at most
// one per 32-row query block).
int bwd_qsplit(const kmi_attn_bwd_args* a) {
    const int64_t wgs = a->batch * a->heads_q * ceil_div(a->seq_k, KW);
    int64_t qs = std::min<int64_t>(4, std::max<int64_t>(1, ceil_div(512, wgs)));
    return static_cast<int>(std::min<int64_t>(qs, ceil_div(a->seq_q, BT)));
}

// dQ key splits, by the same rule over (query head, 64-row block) workgroups.
int bwd_ksplit(const kmi_attn_bwd_args* a) {
    const int64_t wgs = a->batch * a->heads_q * ceil_div(a->seq_q, QW);
    int64_t ks = std::min<int64_t>(4, std::max<int64_t>(1, ceil_div(512, wgs)));
    return static_cast<int>(std::min<int64_t>(ks, ceil_div(a->seq_k, BT)));
}

// Workspace floats: row dot products (padded to 16 bytes); with GQA or query splits the
// dK / dV partials; with key splits the dQ partials.
struct BwdLayout {
    size_t dr, part, pdq;
};

BwdLayout bwd_layout(const kmi_attn_bwd_args* a) {
    BwdLayout l{};
    l.dr = static_cast<size_t>(ceil_div(a->batch * a->heads_q * a->seq_q, 4) * 4);
    const int qs = bwd_qsplit(a);
    if (a->heads_q != a->heads_kv || qs > 1) l.part = static_cast<size_t>(a->batch * a->heads_q * qs * a->seq_k * a->head_dim);
    const int ks = bwd_ksplit(a);
    if (ks > 1) l.pdq = static_cast<size_t>(a->batch * a->heads_q * ks * a->seq_q * a->head_dim);
    return l;
}

size_t bwd_ws_bytes(const kmi_attn_bwd_args* a) {
    const BwdLayout l = bwd_layout(a);
    return (l.dr + 2 * l.part + l.pdq) * sizeof(float);
}

template <typename T, int D>
hipError_t launch_bwd(const BwdParams& p, hipStream_t s) {
    const int64_t ntk = ceil_div(p.seq_k, KW), nqb = ceil_div(p.seq_q, QW);
    // dQ first: it writes the row dots that dK / dV read.
    hipLaunchKernelGGL((attn_bwd_dq<T, D>),
                       dim3(static_cast<unsigned>(static_cast<int64_t>(p.batch) * p.hq * nqb * p.ksplit)),
                       dim3(BWD_THREADS), 0, s, p);
    if (p.pdq) {
        const int64_t items = static_cast<int64_t>(p.batch) * p.hq * p.seq_q * (D / 4);
        hipLaunchKernelGGL((attn_bwd_dq_sum<T, D>), dim3(static_cast<unsigned>(ceil_div(items, 256))), dim3(256), 0, s,
                           p);
    }
    hipLaunchKernelGGL((attn_bwd_dkdv<T, D>),
                       dim3(static_cast<unsigned>(static_cast<int64_t>(p.batch) * p.hq * ntk * p.qsplit)),
                       dim3(BWD_THREADS), 0, s, p);
    if (p.pdk) {
        const int64_t items = static_cast<int64_t>(p.batch) * p.hkv * p.seq_k * (D / 4);
        hipLaunchKernelGGL((attn_bwd_group_sum<T, D>), dim3(static_cast<unsigned>(ceil_div(items, 256))), dim3(256), 0,
                           s, p);
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace kmi

extern "C" int kmi_attn_bwd_workspace_bytes(const kmi_attn_bwd_args* a, size_t* bytes) {
    using namespace kmi;
    if (!bytes) return fail(KMI_EINVAL, "kmi_attn_bwd_workspace_bytes: null bytes");
    if (const char* why = check_bwd(a)) return fail(KMI_EINVAL, std::string("kmi_attn_bwd_workspace_bytes: ") + why);
    *bytes = bwd_ws_bytes(a);
    return KMI_OK;
}

extern "C" int kmi_attn_bwd(const kmi_attn_bwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
    using namespace kmi;
    if (const char* why = check_bwd(a)) return fail(KMI_EINVAL, std::string("kmi_attn_bwd: ") + why);
    const size_t need = bwd_ws_bytes(a);
    if (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16)
        return fail(KMI_EWORKSPACE, "kmi_attn_bwd: workspace missing or smaller than kmi_attn_bwd_workspace_bytes");
    BwdParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->out;
    p.dout = a->grad_out;
    p.lse = a->lse;
    p.dq = a->grad_q;
    p.dk = a->grad_k;
    p.dv = a->grad_v;
    p.dr = static_cast<float*>(workspace);
    p.qsplit = bwd_qsplit(a);
    p.ksplit = bwd_ksplit(a);
    {
        // Partials start 16-byte aligned after the row dot products (D is a multiple of 4).
        const BwdLayout l = bwd_layout(a);
        if (l.part) {
            p.pdk = p.dr + l.dr;
            p.pdv = p.pdk + l.part;
        }
        if (l.pdq) p.pdq = p.dr + l.dr + 2 * l.part;
    }
    for (int i = 0; i < 3; ++i) {
        p.qs[i] = a->q_stride[i];
        p.ks[i] = a->k_stride[i];
        p.vs[i] = a->v_stride[i];
        p.os[i] = a->o_stride[i];
        p.dos[i] = a->do_stride[i];
        p.dqs[i] = a->dq_stride[i];
        p.dks[i] = a->dk_stride[i];
        p.dvs[i] = a->dv_stride[i];
        p.ls[i] = a->lse_stride[i];
    }
    p.batch = static_cast<int>(a->batch);
    p.hq = static_cast<int>(a->heads_q);
    p.hkv = static_cast<int>(a->heads_kv);
    p.group = p.hq / p.hkv;
    p.seq_q = static_cast<int>(a->seq_q);
    p.seq_k = static_cast<int>(a->seq_k);
    p.causal = a->causal ? 1 : 0;
    p.scale = static_cast<float>(a->scale);
    p.c2 = static_cast<float>(a->scale * 1.4426950408889634);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t err;
    if (a->dtype == KMI_BF16)
        err = a->head_dim == 64 ? launch_bwd<bf16, 64>(p, s) : launch_bwd<bf16, 128>(p, s);
    else
        err = a->head_dim == 64 ? launch_bwd<f16, 64>(p, s) : launch_bwd<f16, 128>(p, s);
    return hip_status(err, "kmi_attn_bwd");
}
