// Attention backward on gfx950 (flash-style: nothing of size Sq x Sk is stored).
//
// The reference's training route recomputes the probabilities from the forward's row
// statistics and runs a dQ pass and a dK/dV pass (docs/reference/kernels/flash.md,
// "Backward", flash.md:151-206; ktt_flash/bw_*.cpp; bridge in device_attention.cpp:
// 1208-1281), for dense calls and for packed sequences (aten_varlen.cpp:237-319, with a
// key mask).  Here, for dense and packed (varlen) calls, causal or not, with or without a
// mask (the forward's modes), GQA, any head dim that is a multiple of 8 up to 256 (padded
// to DP with zeros in registers), bf16 / fp16:
//
//   attn_bwd_rowdot  the row dots Dr = sum_d dO O (fp32) of every query row and head
//   attn_bwd_grads   one launch of both gradient passes, their workgroups interleaved:
//     dQ             per (sequence, query head, 64-row block, key split): over the key
//                    tiles it sees P = exp2(c S + mask - lse2), dP = dO V^T,
//                    dS = P (dP - Dr), dQ += dS K
//     dK / dV        per (sequence, K/V head, 64-key tile, split): over the (query head
//                    of the group, 32-row query block) items that see the tile -- split
//                    s takes items s, s + splits, ... -- the same P / dS; dV += P^T dO,
//                    dK += dS^T Q in fp32 registers.  One split: it writes dK / dV;
//                    several: fp32 partials per split that
//   attn_bwd_sums    adds in split order (no atomics: repeat calls are bit-identical),
//                    together with the key-split dQ partials
//
// Probabilities follow the forward exactly: keys past the causal limit or masked
// (logit <= -5e5) get P = 0; a row whose lse carries the -5e5 offset of a fully-masked
// row (the forward ran it over its raw scores) takes every visible key's raw score.
// S = Q K^T, dP = dO V^T and the three gradient products run on
// v_mfma_f32_16x16x32_{bf16,f16}; tiles are staged row-major once, and an operand needed
// along the other index comes out of the same tile through gfx950's transposed LDS reads
// (tr_frag).  lse is the forward's natural-log row LSE.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"

namespace kmi {
namespace {

constexpr int BT = 32;          // keys per K/V tile and rows per query block
constexpr int PP = 20;          // pitch of a wavefront's [32][16] P / dS tiles (elements; 16, 24, 28, 40, 48 measured slower)
constexpr int BWD_THREADS = 256;
constexpr float kLog2e = 1.4426950408889634f;
// A forward lse below this carries the -5e5 offset of a row with no kept key.
constexpr float kRawLse = 0.5f * kMaskedLogit;

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

// gfx950's transposed LDS read: within each 16-lane group, output lane j, slot s receives
// element j % 4 of the 4-element chunk that source lane 4 s + j / 4 addressed.  Source lane
// k of group g pointing at M[row(g, k / 4)][col0 + 4 (k % 4)] so delivers M[row(g, s)][col0
// + j] to lane j, slot s.  tr_frag reads an operand of a product contracted over the 32
// rows of a row-major tile: lane (g, l) gets column col0 + l of rows 4 g + s (slots 0..3)
// and 16 + 4 g + s (slots 4..7).  Both operands of such a product come from tr_frag, so
// their k orders agree (P, dS and dS^T are stored row-major for that, 8 bytes per lane).
template <typename T>
__device__ __forceinline__ typename BwdMfma<T>::v8 tr_frag(const T* tile, int pitch, int col0, int g4, int l16) {
    const T* src = tile + (4 * g4 + (l16 >> 2)) * pitch + col0 + 4 * (l16 & 3);
    u32x2 lo, hi;
    if constexpr (std::is_same<T, bf16>::value) {
        typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 x4;
        lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                           (__attribute__((address_space(3))) x4*)(const_cast<T*>(src))));
        hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                           (__attribute__((address_space(3))) x4*)(const_cast<T*>(src + 16 * pitch))));
    } else {
        typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 x4;
        lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                           (__attribute__((address_space(3))) x4*)(const_cast<T*>(src))));
        hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                           (__attribute__((address_space(3))) x4*)(const_cast<T*>(src + 16 * pitch))));
    }
    return __builtin_bit_cast(typename BwdMfma<T>::v8, u32x4{lo[0], lo[1], hi[0], hi[1]});
}


struct BwdParams {
    const void *q, *k, *v, *o, *dout;
    const float* lse;
    void *dq, *dk, *dv;
    float* dr;  // [hq][rows_total] fp32 row dots
    // dK / dV partials [hkv][splits][keys_total][DP] fp32 (splits > 1), else null.
    float *pdk, *pdv;
    // dQ partials [hq][ksplit][rows_total][DP] fp32 (ksplit > 1), else null.
    float* pdq;
    int splits, ksplit;
    int64_t qs[3], ks[3], vs[3], os[3], dos[3], dqs[3], dks[3], dvs[3], ls[3];
    const void* mask;
    int64_t ms[4];
    int64_t mask_numel;
    int mask_mode;
    const int64_t* mask_off;
    const int32_t *cu_q, *cu_k;
    const int32_t* klen;  // dense key lengths [batch] (or null)
    int total_q, total_k;
    int batch, hq, hkv, group, seq_q, seq_k, causal;
    int d, dval;  // q / k and v / out head dims (DP: the larger, padded)
    int64_t rows_total, keys_total;
    float scale, c2;  // c2 = scale * log2(e)
};

// One sequence's geometry: query rows [q0, q0 + lq) and keys [k0, k0 + lk) of the packed
// (varlen) tensors, or the whole batch entry (dense); causal: row i sees keys
// j <= i + coff (top-left dense: coff = 0; bottom-right varlen: coff = lk - lq).
struct Geo {
    int q0, lq, k0, lk, coff;
    int64_t row_base, key_base;       // row / key index in [rows_total] / [keys_total]
    int64_t qb, kb, vb, ob, dob, dqb, dkb, dvb, lb;  // batch-entry element offsets (dense)
    int64_t mbase;                    // the mask element of (head 0, row 0, key 0)
    int64_t mrow;                     // mask elements per query row
    int64_t mkey;                     // mask elements per key
    int64_t mend;                     // mask elements (reads at or past it count as masked)
};

__device__ __forceinline__ Geo geo_of(const BwdParams& p, int seq) {
    Geo g;
    if (p.cu_q) {
        g.q0 = min(max(p.cu_q[seq], 0), p.total_q);
        g.lq = min(min(max(p.cu_q[seq + 1], g.q0), p.total_q) - g.q0, p.seq_q);
        g.k0 = min(max(p.cu_k[seq], 0), p.total_k);
        g.lk = min(min(max(p.cu_k[seq + 1], g.k0), p.total_k) - g.k0, p.seq_k);
        g.coff = g.lk - g.lq;
        g.row_base = g.q0;
        g.key_base = g.k0;
        g.qb = g.kb = g.vb = g.ob = g.dob = g.dqb = g.dkb = g.dvb = g.lb = 0;
    } else {
        g.q0 = 0;
        g.lq = p.seq_q;
        g.k0 = 0;
        g.lk = p.klen ? min(max(p.klen[seq], 1), p.seq_k) : p.seq_k;
        g.coff = 0;
        g.row_base = static_cast<int64_t>(seq) * p.seq_q;
        g.key_base = static_cast<int64_t>(seq) * p.seq_k;
        g.qb = seq * p.qs[0];
        g.kb = seq * p.ks[0];
        g.vb = seq * p.vs[0];
        g.ob = seq * p.os[0];
        g.dob = seq * p.dos[0];
        g.dqb = seq * p.dqs[0];
        g.dkb = seq * p.dks[0];
        g.dvb = seq * p.dvs[0];
        g.lb = seq * p.ls[0];
    }
    g.mbase = 0;
    g.mrow = 0;
    g.mkey = 0;
    g.mend = INT64_MAX;
    if (p.mask_mode == KMI_MASK_PACKED) {
        int64_t off = 0;
        if (p.mask_off) {
            off = p.mask_off[seq];
        } else {
            for (int s = 0; s < seq; ++s) {
                const int a0 = min(max(p.cu_q[s], 0), p.total_q), a1 = min(max(p.cu_q[s + 1], a0), p.total_q);
                const int b0 = min(max(p.cu_k[s], 0), p.total_k), b1 = min(max(p.cu_k[s + 1], b0), p.total_k);
                off += static_cast<int64_t>(a1 - a0) * (b1 - b0);
            }
        }
        g.mbase = off;
        g.mrow = g.lk;
        g.mkey = 1;
        g.mend = p.mask_numel;
    } else if (p.mask_mode == KMI_MASK_STRIDED) {
        g.mbase = p.cu_q ? static_cast<int64_t>(g.q0) * p.ms[2] + static_cast<int64_t>(g.k0) * p.ms[3] : seq * p.ms[0];
        g.mrow = p.ms[2];
        g.mkey = p.ms[3];
    }
    return g;
}

// The mask logit of (head h, row i, key j) of a sequence (0 without a mask).
template <int MK>
__device__ __forceinline__ float mask_at(const BwdParams& p, const Geo& g, int h, int i, int j) {
    if constexpr (MK == MK_NONE) {
        return 0.f;
    } else {
        typedef typename MaskRaw<MK>::type R;
        const int64_t idx = g.mbase + h * p.ms[1] + i * g.mrow + j * g.mkey;
        if (idx >= g.mend) return kMaskedLogit;
        return mask_logit_of<MK>(static_cast<const R*>(p.mask)[idx]);
    }
}

// Row statistics of row i (i < lq): base-2 lse of the row's softmax and whether the row
// ran over its raw scores (no kept key in the forward).  Rows past the end or without
// keys get +inf (P = 0).
__device__ __forceinline__ void row_stats(float lse_nat, bool valid, float& lse2, bool& raw) {
    raw = valid && lse_nat < kRawLse;
    const float l = raw ? lse_nat - kMaskedLogit : lse_nat;
    lse2 = (valid && l != -INFINITY) ? l * kLog2e : INFINITY;
}

// Staging of rows [r0, r0 + 32) of a [S, D] operand (row stride rs elements) in two steps:
// loads into registers (16-byte chunks), issued a tile ahead, and their LDS stores,
// row-major at pitch DP + 16 (8 or 24 measured slower).  The loads go through a buffer
// resource over the tile's rows, built in scalar registers per tile, at byte offsets each
// thread fixes once per call (TileOffs): a tile costs no per-lane address arithmetic.
// Chunks past the head dim carry an offset past every range and rows past the last one
// lie past the range's end, so both read zeros (overlapping rows, a stride below the head
// dim, read their real, finite data there, which gets zero weight).
template <int DP>
struct TileRegs {
    static constexpr int NV = BT * DP / 8;  // 16-byte chunks of a tile
    static constexpr int PER = (NV + BWD_THREADS - 1) / BWD_THREADS;
    u32x4 v[PER];
};

template <int DP>
struct TileOffs {
    uint32_t o[TileRegs<DP>::PER];
};

constexpr uint32_t kNoChunk = 0x80000000u;  // past every tile's range (the host keeps ranges below 2^31 bytes)

template <typename T, int DP>
__device__ __forceinline__ TileOffs<DP> tile_offs(int64_t rs, int d) {
    TileOffs<DP> t;
#pragma unroll
    for (int j = 0; j < TileRegs<DP>::PER; ++j) {
        const int c = threadIdx.x + BWD_THREADS * j;
        const int r = c % BT, ch = c / BT;
        t.o[j] = (c < TileRegs<DP>::NV && 8 * ch < d) ? static_cast<uint32_t>(r * rs * sizeof(T)) + 16u * ch : kNoChunk;
    }
    return t;
}

template <typename T, int DP>
__device__ __forceinline__ void load_regs(const T* src, int64_t rs, int r0, int nrows, int d, const TileOffs<DP>& off,
                                          TileRegs<DP>& t) {
    const int n = min(BT, nrows - r0);
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(
        src + r0 * rs, rows_extent(n, static_cast<uint32_t>(rs * sizeof(T)), static_cast<uint32_t>(d * sizeof(T))));
#pragma unroll
    for (int j = 0; j < TileRegs<DP>::PER; ++j) t.v[j] = buffer_load16(r, off.o[j]);
}

template <typename T, int DP>
__device__ __forceinline__ void store_regs(const TileRegs<DP>& t, T* dst) {
#pragma unroll
    for (int j = 0; j < TileRegs<DP>::PER; ++j) {
        const int c = threadIdx.x + BWD_THREADS * j;
        if (c >= TileRegs<DP>::NV) break;
        const int r = c % BT, ch = c / BT;
        *reinterpret_cast<u32x4*>(dst + r * (DP + 16) + 8 * ch) = t.v[j];
    }
}

// A 16-byte fragment of row `row` (< nrows) at column `col` of a [S, D] operand, zeros
// past the last row or the head dim.
template <typename T>
__device__ __forceinline__ u32x4 frag(const T* base, int64_t rs, int row, int nrows, int col, int d) {
    const int rc = min(max(row, 0), nrows - 1);
    const int cc = min(col, d - 8);
    const u32x4 x = *reinterpret_cast<const u32x4*>(base + static_cast<int64_t>(rc) * rs + cc);
    return (row >= 0 && row < nrows && col < d) ? x : u32x4{0u, 0u, 0u, 0u};
}

// dK / dV: a workgroup takes KW keys of one K/V head; wavefront w owns keys
// [kt0 + 16 w, + 16) with its K and V fragments in registers (the A operands of
// S^T = K Q^T and dP^T = V dO^T).  Per (query head, 32-row query block) item the
// workgroup stages Q and dO (row-major) once; each wavefront then forms P^T
// and dS^T of its keys, passes them through its own LDS rows (one wavefront's LDS accesses
// stay in order: no barrier) and accumulates dV += P^T dO and dK += dS^T Q over every
// query head of the group.  Two barriers per item.
constexpr int KW = 64;

template <typename T, int DP, int MK, bool DV>
__device__ __forceinline__ void attn_bwd_dkdv(const BwdParams& p, const int bid) {
    typedef typename BwdMfma<T>::v8 v8;
    // v / dO / out width: a separate value dim only in the DV instances (one width keeps
    // the equal-dim kernels' registers).
    const int dval = DV ? p.dval : p.d;
    constexpr int RP = DP + 16;
    constexpr int DC = DP / 32, DB = DP / 16;
    __shared__ __align__(16) T qs[BT * RP];
    __shared__ __align__(16) T dos[BT * RP];
    __shared__ __align__(16) T pt[4 * BT * PP];   // per wavefront: P [32 rows][16 keys]
    __shared__ __align__(16) T dst[4 * BT * PP];  // per wavefront: dS [32 rows][16 keys]
    __shared__ float lse2[BT], drs[BT];
    __shared__ int raws[BT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4, l16 = lane & 15;
    const int ntk = (p.seq_k + KW - 1) / KW;
    const int split = bid % p.splits;
    const int tile = (bid / p.splits) % ntk;
    const int bkv = bid / (p.splits * ntk);  // (sequence, K/V head)
    const int seq = bkv / p.hkv, kvh = bkv - seq * p.hkv;
    const Geo g = geo_of(p, seq);
    const int kt0 = tile * KW;
    // Keys written: the sequence's (varlen) or every key row of the batch entry (dense:
    // keys past a key length get zero gradients).
    const int kwrite = p.cu_q ? g.lk : p.seq_k;
    if (kt0 >= kwrite) return;  // uniform: no barrier has run
    const int kw0 = kt0 + 16 * wave;  // this wavefront's first key

    // K / V fragments: lane (g4, l16) holds key kw0 + l16, dims 32 c + 8 g4 .. + 7.
    v8 kf[DC], vf[DC];
    {
        const T* kp = static_cast<const T*>(p.k) + g.kb + kvh * p.ks[1] + static_cast<int64_t>(g.k0) * p.ks[2];
        const T* vp = static_cast<const T*>(p.v) + g.vb + kvh * p.vs[1] + static_cast<int64_t>(g.k0) * p.vs[2];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            kf[c] = __builtin_bit_cast(v8, frag(kp, p.ks[2], kw0 + l16, g.lk, 32 * c + 8 * g4, p.d));
            vf[c] = __builtin_bit_cast(v8, frag(vp, p.vs[2], kw0 + l16, g.lk, 32 * c + 8 * g4, dval));
        }
    }
    f32x4 dk[DB], dv[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) dk[i] = dv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    T* ptw = pt + wave * BT * PP;
    T* dsw = dst + wave * BT * PP;

    // Items: (query head of the group, 32-row query block), blocks from the first that
    // sees this tile (causal: rows i >= kt0 - coff); split s takes items s, s + splits, ...
    const int rfirst = p.causal ? max(0, kt0 - g.coff) / BT : 0;
    const int nblk = (kt0 < g.lk && g.lq > rfirst * BT) ? (g.lq + BT - 1) / BT - rfirst : 0;
    const int items = nblk * p.group;
    // Item it = gi nblk + bi is query head kvh G + gi, rows (rfirst + bi) 32 ..; the walk
    // it, it + splits, ... steps (gi, bi) by (splits / nblk, splits % nblk) with one carry
    // (no division per item).
    const int sp_g = nblk > 0 ? p.splits / nblk : 0, sp_b = p.splits - sp_g * nblk;
    auto step = [&](int& gi, int& bi) {
        gi += sp_g;
        bi += sp_b;
        if (bi >= nblk) {
            bi -= nblk;
            ++gi;
        }
    };
    auto item_at = [&](int gi, int bi, int& h, int& r0) {
        h = kvh * p.group + gi;
        r0 = (rfirst + bi) * BT;
    };
    auto q_of = [&](int h) {
        return static_cast<const T*>(p.q) + g.qb + h * p.qs[1] + static_cast<int64_t>(g.q0) * p.qs[2];
    };
    auto do_of = [&](int h) {
        return static_cast<const T*>(p.dout) + g.dob + h * p.dos[1] + static_cast<int64_t>(g.q0) * p.dos[2];
    };
    TileRegs<DP> qr, dor;
    const TileOffs<DP> oq = tile_offs<T, DP>(p.qs[2], p.d), odo = tile_offs<T, DP>(p.dos[2], dval);
    // Row statistics of an item's rows, loaded with its Q and dO a whole item ahead by
    // wavefront 0 (a uniform branch), lane l holding row l % BT (both halves the same).
    const int srow = lane & (BT - 1);
    float lv_n = 0.f, dr_n = 0.f;
    auto load_stats = [&](int h, int r0) {
        if (wave == 0) {
            const int ic = min(r0 + srow, g.lq - 1);
            lv_n = p.lse[g.lb + h * p.ls[1] + static_cast<int64_t>(g.q0 + ic) * p.ls[2]];
            dr_n = p.dr[h * p.rows_total + g.row_base + ic];
        }
    };
    int gi = nblk > 0 ? split / nblk : 0, bi = split - gi * nblk;
    if (split < items) {
        int h, r0;
        item_at(gi, bi, h, r0);
        load_regs<T, DP>(q_of(h), p.qs[2], r0, g.lq, p.d, oq, qr);
        load_regs<T, DP>(do_of(h), p.dos[2], r0, g.lq, dval, odo, dor);
        load_stats(h, r0);
    }
    for (int it = split; it < items; it += p.splits) {
        int h, r0;
        item_at(gi, bi, h, r0);
        step(gi, bi);  // (gi, bi) is now the next item's
        __syncthreads();  // the previous item's LDS reads are done
        store_regs<T, DP>(qr, qs);
        store_regs<T, DP>(dor, dos);
        if (wave == 0) {  // lanes l and l + 32 write the same values
            const bool ok = r0 + srow < g.lq;
            float l2;
            bool raw;
            row_stats(lv_n, ok, l2, raw);
            lse2[srow] = l2;
            raws[srow] = raw ? 1 : 0;
            drs[srow] = ok ? dr_n : 0.f;
        }
        __syncthreads();
        if (it + p.splits < items) {  // the next item's loads overlap this item's products
            int h2, r2;
            item_at(gi, bi, h2, r2);
            load_regs<T, DP>(q_of(h2), p.qs[2], r2, g.lq, p.d, oq, qr);
            load_regs<T, DP>(do_of(h2), p.dos[2], r2, g.lq, dval, odo, dor);
            load_stats(h2, r2);
        }
        // Unmasked items whose 32 rows see all of this wavefront's 16 keys (uniform): no
        // per-element causal or key-tail test.
        const bool full = MK == MK_NONE && kw0 + 15 < g.lk && (!p.causal || kw0 + 15 <= r0 + g.coff);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            // S^T and dP^T of this wavefront's 16 keys x rows rb 16 .. + 15: lane (g4, l16)
            // gets keys 4 g4 + j, row l16.
            f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f}, dpt = st;
            // Issue priority over the MFMA sections (here and below): a wavefront with
            // products to issue wins the arbitration over those forming P and dS (C4 varlen
            // backward 267 -> 262 us, C1 109 -> 108 us).
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const v8 qb = *reinterpret_cast<const v8*>(qs + (rb * 16 + l16) * RP + 32 * c + 8 * g4);
                const v8 ob = *reinterpret_cast<const v8*>(dos + (rb * 16 + l16) * RP + 32 * c + 8 * g4);
                st = BwdMfma<T>::run(kf[c], qb, st);
                dpt = BwdMfma<T>::run(vf[c], ob, dpt);
            }
            __builtin_amdgcn_s_setprio(0);
            const int rl = rb * 16 + l16;
            const int row = r0 + rl;
            const float l2 = lse2[rl], dr = drs[rl];
            const bool raw = raws[rl] != 0;
            typedef T t4 __attribute__((ext_vector_type(4)));
            t4 pv, sv;
            // Rows past the end carry lse2 = +inf: their P is exactly 0.
            if (full) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float e = __builtin_amdgcn_exp2f(st[j] * p.c2 - l2);
                    pv[j] = from_f32<T>(e);
                    sv[j] = from_f32<T>(e * (dpt[j] - dr));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int key = kw0 + 4 * g4 + j;
                    bool keep = key < g.lk && (!p.causal || key <= row + g.coff);
                    float add = 0.f;
                    if constexpr (MK != MK_NONE) {
                        const float ml = (keep && row < g.lq) ? mask_at<MK>(p, g, h, row, key) : 0.f;
                        keep = keep && (raw || ml > kMaskedLogit);
                        add = raw ? 0.f : ml * kLog2e;
                    }
                    const float e = keep ? __builtin_amdgcn_exp2f(st[j] * p.c2 + add - l2) : 0.f;
                    pv[j] = from_f32<T>(e);
                    sv[j] = from_f32<T>(e * (dpt[j] - dr));
                }
            }
            // Row rl, keys 4 g4 .. + 3: one 8-byte store each.
            *reinterpret_cast<t4*>(ptw + rl * PP + 4 * g4) = pv;
            *reinterpret_cast<t4*>(dsw + rl * PP + 4 * g4) = sv;
        }
        // The compiler keeps these LDS reads after the stores above (same arrays); the
        // hardware runs one wavefront's LDS accesses in order.
        __asm__ volatile("" ::: "memory");
        // P^T and dS^T fragments (key l16, rows in tr_frag's order) by transposed reads.
        const v8 pa = tr_frag<T>(ptw, PP, 0, g4, l16);
        const v8 sa = tr_frag<T>(dsw, PP, 0, g4, l16);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            // dO^T and Q^T straight from the row-major tiles (transposed reads).
            const v8 ob = tr_frag<T>(dos, RP, 16 * db, g4, l16);
            const v8 qb = tr_frag<T>(qs, RP, 16 * db, g4, l16);
            dv[db] = BwdMfma<T>::run(pa, ob, dv[db]);
            dk[db] = BwdMfma<T>::run(sa, qb, dk[db]);
        }
        __builtin_amdgcn_s_setprio(0);
    }
    // Lane (g4, l16) of block db holds keys kw0 + 4 g4 + j, dim db 16 + l16.
    if (p.pdk) {
        const int64_t base = (static_cast<int64_t>(kvh) * p.splits + split) * p.keys_total + g.key_base;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = db * 16 + l16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int key = kw0 + 4 * g4 + j;
                if (key < kwrite) {
                    if (d < p.d) p.pdk[(base + key) * DP + d] = dk[db][j] * p.scale;
                    if (d < dval) p.pdv[(base + key) * DP + d] = dv[db][j];
                }
            }
        }
        return;
    }
    T* dkp = static_cast<T*>(p.dk) + g.dkb + kvh * p.dks[1] + static_cast<int64_t>(g.k0) * p.dks[2];
    T* dvp = static_cast<T*>(p.dv) + g.dvb + kvh * p.dvs[1] + static_cast<int64_t>(g.k0) * p.dvs[2];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const int d = db * 16 + l16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = kw0 + 4 * g4 + j;
            if (key < kwrite) {
                if (d < p.d) dkp[static_cast<int64_t>(key) * p.dks[2] + d] = from_f32<T>(dk[db][j] * p.scale);
                if (d < dval) dvp[static_cast<int64_t>(key) * p.dvs[2] + d] = from_f32<T>(dv[db][j]);
            }
        }
    }
}

// Partials a sum kernel loads before it adds them.
constexpr int kSumBatch = 8;

// dQ: a workgroup takes QW query rows (16 per wavefront).
constexpr int QW = 64;

// The row dots D = sum(dO * O) (fp32) of every query row and head, read by both gradient
// passes, which run concurrently: one workgroup per (sequence, query head, QW-row block),
// 16 rows per wavefront.  A row's CH = dval / 8 16-byte chunks go to CP (CH rounded up to
// a power of two) adjacent lanes, so that each load instruction reads whole rows
// contiguously; the lanes' partial dots meet in a butterfly over those CP lanes.
template <typename T, int DP, bool DV>
__global__ __launch_bounds__(BWD_THREADS) void attn_bwd_rowdot(const BwdParams p) {
    const int dval = DV ? p.dval : p.d;
    constexpr int CP = DP / 8 > 16 ? 32 : (DP / 8 > 8 ? 16 : (DP / 8 > 4 ? 8 : 4));  // lanes per row (>= DP / 8)
    constexpr int RPI = kWave / CP;  // rows per load instruction
    constexpr int NI = 16 / RPI;     // instructions for the wavefront's 16 rows
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // Heads fastest: workgroups that run together read the same query rows of every head
    // (one contiguous span per token in packed [T, H, D] layouts).
    const int nqb = (p.seq_q + QW - 1) / QW;
    const int h = blockIdx.x % p.hq;
    const int sq = blockIdx.x / p.hq;
    const int seq = sq / nqb, qb = sq - seq * nqb;
    const Geo g = geo_of(p, seq);
    if (qb * QW >= g.lq) return;
    const T* dp = static_cast<const T*>(p.dout) + g.dob + h * p.dos[1] + static_cast<int64_t>(g.q0) * p.dos[2];
    const T* op = static_cast<const T*>(p.o) + g.ob + h * p.os[1] + static_cast<int64_t>(g.q0) * p.os[2];
    const int c = lane % CP;
    const int row0 = qb * QW + 16 * wave + lane / CP;
    u32x4 dv[NI], ov[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = min(row0 + RPI * i, g.lq - 1);
        const int col = min(8 * c, dval - 8);
        dv[i] = *reinterpret_cast<const u32x4*>(dp + static_cast<int64_t>(row) * p.dos[2] + col);
        ov[i] = *reinterpret_cast<const u32x4*>(op + static_cast<int64_t>(row) * p.os[2] + col);
    }
    typedef typename BwdMfma<T>::v8 v8;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const v8 a = __builtin_bit_cast(v8, dv[i]), b = __builtin_bit_cast(v8, ov[i]);
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dot += to_f32(a[e]) * to_f32(b[e]);
        if (8 * c >= dval) dot = 0.f;
#pragma unroll
        for (int o = CP / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o, kWave);
        const int row = row0 + RPI * i;
        if (c == 0 && row < g.lq) p.dr[h * p.rows_total + g.row_base + row] = dot;
    }
}

// dK / dV rows from the splits' fp32 partials, added in split order.  One item per
// (K/V head, key row, 4 head-dim columns).
template <typename T, int DP>
__device__ __forceinline__ void kv_sum_item(const BwdParams& p, const int64_t item) {
    const int nq = max(p.d, p.dval) / 4;  // float4 items per key row (head dims are multiples of 8)
    const int64_t items = static_cast<int64_t>(p.hkv) * p.keys_total * nq;
    if (item >= items) return;
    const int c = static_cast<int>(item % nq);
    const int64_t krow = (item / nq) % p.keys_total;
    const int kvh = static_cast<int>(item / (static_cast<int64_t>(nq) * p.keys_total));
    f32x4 sk = f32x4{0.f, 0.f, 0.f, 0.f}, sv = sk;
    auto at = [&](int s) { return ((static_cast<int64_t>(kvh) * p.splits + s) * p.keys_total + krow) * DP + 4 * c; };
    // Eight splits' partials are loaded before they are added (in split order, so the
    // sums are those of a plain loop): one round trip per eight splits instead of one each.
    int s = 0;
    for (; s + kSumBatch <= p.splits; s += kSumBatch) {
        f32x4 bk[kSumBatch], bv[kSumBatch];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j) {
            bk[j] = *reinterpret_cast<const f32x4*>(p.pdk + at(s + j));
            bv[j] = *reinterpret_cast<const f32x4*>(p.pdv + at(s + j));
        }
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j) {
            sk += bk[j];
            sv += bv[j];
        }
    }
    for (; s < p.splits; ++s) {
        sk += *reinterpret_cast<const f32x4*>(p.pdk + at(s));
        sv += *reinterpret_cast<const f32x4*>(p.pdv + at(s));
    }
    int64_t koff, voff;
    if (p.cu_q) {
        koff = krow * p.dks[2];
        voff = krow * p.dvs[2];
    } else {
        const int64_t b = krow / p.seq_k, key = krow - b * p.seq_k;
        koff = b * p.dks[0] + key * p.dks[2];
        voff = b * p.dvs[0] + key * p.dvs[2];
    }
    T* dkp = static_cast<T*>(p.dk) + koff + kvh * p.dks[1] + 4 * c;
    T* dvp = static_cast<T*>(p.dv) + voff + kvh * p.dvs[1] + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (4 * c < p.d) dkp[e] = from_f32<T>(sk[e]);
        if (4 * c < p.dval) dvp[e] = from_f32<T>(sv[e]);
    }
}

// dQ: a workgroup takes QW query rows, wavefront w owns rows [r0 + 16 w, + 16) with its Q
// and dO fragments in registers (the A operands of S = Q K^T and dP = dO V^T).  Per
// 32-key tile the workgroup stages K and V (row-major) once; each wavefront
// forms dS of its rows, passes it through its own LDS rows and accumulates dQ += dS K.

template <typename T, int DP, int MK, bool DV>
__device__ __forceinline__ void attn_bwd_dq(const BwdParams& p, const int bid) {
    typedef typename BwdMfma<T>::v8 v8;
    // v / dO / out width: a separate value dim only in the DV instances (one width keeps
    // the equal-dim kernels' registers).
    const int dval = DV ? p.dval : p.d;
    constexpr int RP = DP + 16;
    constexpr int DC = DP / 32, DB = DP / 16;
    __shared__ __align__(16) T ks[BT * RP];
    __shared__ __align__(16) T vs[BT * RP];
    __shared__ __align__(16) T dss[4 * BT * PP];  // per wavefront: dS^T [32 keys][16 rows]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4, l16 = lane & 15;
    const int nqb = (p.seq_q + QW - 1) / QW;
    const int ksp = bid % p.ksplit;
    const int qb = (bid / p.ksplit) % nqb;
    const int bh = bid / (p.ksplit * nqb);
    const int seq = bh / p.hq, h = bh - seq * p.hq;
    const int kvh = h / p.group;
    const Geo g = geo_of(p, seq);
    const int r0 = qb * QW;
    if (r0 >= g.lq || g.lk <= 0) return;  // uniform: no barrier has run
    const int rw0 = r0 + 16 * wave;  // this wavefront's first row

    // Q / dO fragments: lane (g4, l16) holds row rw0 + l16, dims 32 c + 8 g4 .. + 7; the
    // row statistics and row dots (attn_bwd_rowdot's) of rows rw0 + 4 g4 + j (the rows of
    // its accumulator lanes).
    v8 qf[DC], of[DC];
    {
        const T* qp = static_cast<const T*>(p.q) + g.qb + h * p.qs[1] + static_cast<int64_t>(g.q0) * p.qs[2];
        const T* dp = static_cast<const T*>(p.dout) + g.dob + h * p.dos[1] + static_cast<int64_t>(g.q0) * p.dos[2];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const int col = 32 * c + 8 * g4;
            qf[c] = __builtin_bit_cast(v8, frag(qp, p.qs[2], rw0 + l16, g.lq, col, p.d));
            of[c] = __builtin_bit_cast(v8, frag(dp, p.dos[2], rw0 + l16, g.lq, col, dval));
        }
    }
    float l2[4], drv[4];
    bool raw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = rw0 + 4 * g4 + j;
        const int rc = min(row, g.lq - 1);
        const float lv = p.lse[g.lb + h * p.ls[1] + static_cast<int64_t>(g.q0 + rc) * p.ls[2]];
        const float dv = p.dr[h * p.rows_total + g.row_base + rc];
        row_stats(lv, row < g.lq, l2[j], raw[j]);
        drv[j] = row < g.lq ? dv : 0.f;
    }
    f32x4 dq[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) dq[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    T* dsw = dss + wave * BT * PP;

    // Causal: the block's last row sees keys up to its position + coff.
    const int kend = p.causal ? min(g.lk, max(0, min(r0 + QW, g.lq) - 1 + g.coff + 1)) : g.lk;
    const T* kbase = static_cast<const T*>(p.k) + g.kb + kvh * p.ks[1] + static_cast<int64_t>(g.k0) * p.ks[2];
    const T* vbase = static_cast<const T*>(p.v) + g.vb + kvh * p.vs[1] + static_cast<int64_t>(g.k0) * p.vs[2];
    TileRegs<DP> kr, vr;
    const TileOffs<DP> okk = tile_offs<T, DP>(p.ks[2], p.d), ovv = tile_offs<T, DP>(p.vs[2], dval);
    const int kstep = p.ksplit * BT;
    if (ksp * BT < kend) {
        load_regs<T, DP>(kbase, p.ks[2], ksp * BT, g.lk, p.d, okk, kr);
        load_regs<T, DP>(vbase, p.vs[2], ksp * BT, g.lk, dval, ovv, vr);
    }
    for (int k0 = ksp * BT; k0 < kend; k0 += kstep) {
        __syncthreads();
        store_regs<T, DP>(kr, ks);
        store_regs<T, DP>(vr, vs);
        __syncthreads();
        if (k0 + kstep < kend) {  // the next tile's loads overlap this tile's products
            load_regs<T, DP>(kbase, p.ks[2], k0 + kstep, g.lk, p.d, okk, kr);
            load_regs<T, DP>(vbase, p.vs[2], k0 + kstep, g.lk, dval, ovv, vr);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            // S and dP of this wavefront's 16 rows x keys kb 16 .. + 15: lane (g4, l16)
            // gets rows 4 g4 + j, key l16.
            f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f}, dpv = sv;
            __builtin_amdgcn_s_setprio(1);  // (as in attn_bwd_dkdv)
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const v8 kbv = *reinterpret_cast<const v8*>(ks + (kb * 16 + l16) * RP + 32 * c + 8 * g4);
                const v8 vbv = *reinterpret_cast<const v8*>(vs + (kb * 16 + l16) * RP + 32 * c + 8 * g4);
                sv = BwdMfma<T>::run(qf[c], kbv, sv);
                dpv = BwdMfma<T>::run(of[c], vbv, dpv);
            }
            __builtin_amdgcn_s_setprio(0);
            const int key = k0 + kb * 16 + l16;
            typedef T t4 __attribute__((ext_vector_type(4)));
            t4 dsv;
            // Unmasked key blocks that all of this wavefront's 16 rows see (uniform): no
            // per-element causal or key-tail test.
            const int kb0 = k0 + kb * 16;
            if (MK == MK_NONE && kb0 + 15 < g.lk && (!p.causal || kb0 + 15 <= rw0 + g.coff)) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float e = __builtin_amdgcn_exp2f(sv[j] * p.c2 - l2[j]);
                    dsv[j] = from_f32<T>(e * (dpv[j] - drv[j]));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = rw0 + 4 * g4 + j;
                    bool keep = key < g.lk && (!p.causal || key <= row + g.coff);
                    float add = 0.f;
                    if constexpr (MK != MK_NONE) {
                        const float ml = (keep && row < g.lq) ? mask_at<MK>(p, g, h, row, key) : 0.f;
                        keep = keep && (raw[j] || ml > kMaskedLogit);
                        add = raw[j] ? 0.f : ml * kLog2e;
                    }
                    const float e = keep ? __builtin_amdgcn_exp2f(sv[j] * p.c2 + add - l2[j]) : 0.f;
                    dsv[j] = from_f32<T>(e * (dpv[j] - drv[j]));
                }
            }
            // Key kb 16 + l16, rows 4 g4 .. + 3: one 8-byte store.
            *reinterpret_cast<t4*>(dsw + (kb * 16 + l16) * PP + 4 * g4) = dsv;
        }
        // The compiler keeps this LDS read after the stores above (same array); the hardware
        // runs one wavefront's LDS accesses in order.
        __asm__ volatile("" ::: "memory");
        // dS fragments (row l16, keys in tr_frag's order) by transposed reads.
        const v8 da = tr_frag<T>(dsw, PP, 0, g4, l16);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int db = 0; db < DB; ++db) dq[db] = BwdMfma<T>::run(da, tr_frag<T>(ks, RP, 16 * db, g4, l16), dq[db]);
        __builtin_amdgcn_s_setprio(0);
    }
    // Lane (g4, l16) of block db holds rows rw0 + 4 g4 + j, dim db 16 + l16.
    if (p.pdq) {
        float* dst = p.pdq + ((static_cast<int64_t>(h) * p.ksplit + ksp) * p.rows_total + g.row_base) * DP;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = db * 16 + l16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = rw0 + 4 * g4 + j;
                if (row < g.lq && d < p.d) dst[static_cast<int64_t>(row) * DP + d] = dq[db][j] * p.scale;
            }
        }
        return;
    }
    T* dqp = static_cast<T*>(p.dq) + g.dqb + h * p.dqs[1] + static_cast<int64_t>(g.q0) * p.dqs[2];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const int d = db * 16 + l16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = rw0 + 4 * g4 + j;
            if (row < g.lq && d < p.d) dqp[static_cast<int64_t>(row) * p.dqs[2] + d] = from_f32<T>(dq[db][j] * p.scale);
        }
    }
}

// Both gradient passes in one launch (they read the same inputs and the row dots, and
// neither reads the other's output), their workgroups interleaved in proportion (block b
// is dQ workgroup floor(b n_dq / n) when that count steps at b, else a dK / dV workgroup),
// so that the two kinds share every CU from the start.
// Workgroups per CU the fused kernel keeps resident (the register budget it compiles to,
// without spills): those of the dK / dV kernel alone at head dims 64 and 128 for the
// unmasked equal-dim variants, one fewer for masked or value-dim ones.
constexpr int bwd_min_blocks(int dp, bool plain) {
    return dp <= 64 ? (plain ? 4 : 3) : (dp <= 128 ? (plain ? 3 : 2) : 1);
}

template <typename T, int DP, int MK, bool DV>
__global__ __launch_bounds__(BWD_THREADS, bwd_min_blocks(DP, MK == MK_NONE && !DV)) void attn_bwd_grads(
    const BwdParams p, const int kv_blocks, const int dq_blocks) {
    const int64_t b = blockIdx.x, n = static_cast<int64_t>(kv_blocks) + dq_blocks;
    const int q0 = static_cast<int>(b * dq_blocks / n), q1 = static_cast<int>((b + 1) * dq_blocks / n);
    if (q1 > q0)
        attn_bwd_dq<T, DP, MK, DV>(p, q0);
    else
        attn_bwd_dkdv<T, DP, MK, DV>(p, static_cast<int>(b) - q0);
}

// dQ rows from the key splits' fp32 partials, in split order.  One item per (query head,
// query row, 4 head-dim columns).
template <typename T, int DP>
__device__ __forceinline__ void dq_sum_item(const BwdParams& p, const int64_t item) {
    const int nq = p.d / 4;
    const int64_t items = static_cast<int64_t>(p.hq) * p.rows_total * nq;
    if (item >= items) return;
    const int c = static_cast<int>(item % nq);
    const int64_t row = (item / nq) % p.rows_total;
    const int h = static_cast<int>(item / (static_cast<int64_t>(nq) * p.rows_total));
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    auto at = [&](int k) { return ((static_cast<int64_t>(h) * p.ksplit + k) * p.rows_total + row) * DP + 4 * c; };
    // As in kv_sum_item: a batch of loads, then the adds in split order.
    int k = 0;
    for (; k + kSumBatch <= p.ksplit; k += kSumBatch) {
        f32x4 b[kSumBatch];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j) b[j] = *reinterpret_cast<const f32x4*>(p.pdq + at(k + j));
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j) acc += b[j];
    }
    for (; k < p.ksplit; ++k) acc += *reinterpret_cast<const f32x4*>(p.pdq + at(k));
    int64_t off;
    if (p.cu_q) {
        off = row * p.dqs[2];
    } else {
        const int64_t b = row / p.seq_q, i = row - b * p.seq_q;
        off = b * p.dqs[0] + i * p.dqs[2];
    }
    T* dst = static_cast<T*>(p.dq) + off + h * p.dqs[1] + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(acc[e]);
}

// Both sums in one launch (after the gradient launch; neither reads the other's output): blocks
// [0, dq_blocks) take dQ items (the key-split dQ partials), the rest dK / dV items.
template <typename T, int DP>
__global__ __launch_bounds__(256) void attn_bwd_sums(const BwdParams p, const int64_t dq_blocks) {
    const int64_t b = blockIdx.x;
    if (b < dq_blocks) {
        dq_sum_item<T, DP>(p, b * 256 + threadIdx.x);
    } else {
        kv_sum_item<T, DP>(p, (b - dq_blocks) * 256 + threadIdx.x);
    }
}

// The value / output head dim (head_dim_v, or head_dim when 0).
int64_t bwd_value_dim(const kmi_attn_bwd_args* a) { return a->head_dim_v > 0 ? a->head_dim_v : a->head_dim; }

const char* check_bwd(const kmi_attn_bwd_args* a) {
    if (!a) return "null args";
    if (a->dtype != KMI_BF16 && a->dtype != KMI_F16) return "dtype must be BF16 or F16";
    if (!head_dim_supported(a->head_dim)) return "head_dim must be a multiple of 8 up to 256";
    if (a->head_dim_v != 0 && !head_dim_supported(a->head_dim_v))
        return "head_dim_v must be 0 or a multiple of 8 up to 256";
    if (a->batch <= 0 || a->heads_q <= 0 || a->heads_kv <= 0 || a->seq_q <= 0 || a->seq_k <= 0)
        return "sizes must be positive";
    if (a->heads_q % a->heads_kv != 0) return "heads_kv must divide heads_q";
    const bool varlen = a->cu_seqlens_q != nullptr;
    if (varlen != (a->cu_seqlens_k != nullptr)) return "cu_seqlens_q and cu_seqlens_k go together";
    const int64_t rows = varlen ? a->total_q : a->batch * a->seq_q;
    const int64_t keys = varlen ? a->total_k : a->batch * a->seq_k;
    if (varlen && (a->total_q <= 0 || a->total_k <= 0)) return "varlen totals must be positive";
    if (rows * a->heads_q > (int64_t{1} << 31) || keys * a->heads_q > (int64_t{1} << 31) || a->seq_q > (1 << 30) ||
        a->seq_k > (1 << 30))
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
    // The staging loads address a 32-row tile with 32-bit byte offsets.
    for (const int64_t* s : strides)
        if (s[2] >= (int64_t{1} << 25)) return "q, k, v, out and grad_out row strides must be below 2^25 elements";
    const int64_t* ostrides[] = {a->dq_stride, a->dk_stride, a->dv_stride};
    for (const int64_t* s : ostrides)
        for (int i = 0; i < 3; ++i)
            if (s[i] % 4) return "grad_q, grad_k and grad_v strides must be multiples of 4";
    if (a->mask_mode != KMI_MASK_NONE) {
        if (!a->mask) return "mask_mode set without a mask";
        if (a->mask_dtype < KMI_BF16 || a->mask_dtype > KMI_BOOL) return "bad mask dtype";
        if (a->mask_mode != KMI_MASK_STRIDED && a->mask_mode != KMI_MASK_PACKED) return "bad mask mode";
        if (a->mask_mode == KMI_MASK_PACKED && (!varlen || a->mask_numel <= 0 || a->mask_stride[1] != 0))
            return "packed masks are varlen only, need mask_numel and are shared by the heads";
    }
    return nullptr;
}

int64_t rows_total_of(const kmi_attn_bwd_args* a) { return a->cu_seqlens_q ? a->total_q : a->batch * a->seq_q; }
int64_t keys_total_of(const kmi_attn_bwd_args* a) { return a->cu_seqlens_q ? a->total_k : a->batch * a->seq_k; }

// Split rules.  dK / dV and dQ workgroups run interleaved in one launch, so each kind
// needs enough work per workgroup to amortise its set-up and few enough splits to keep
// the fp32 partials small, rather than a grid that fills the chip alone.  A dK / dV
// workgroup takes at most kBwdItemsPerWg64 (query head, 32-row block) items up to head
// dim 64 and kBwdItemsPerWg128 at 128 (in proportion fewer past it) when splitting allows
// it, a dQ workgroup at most kBwdTilesPerWg 32-key tiles; below kBwdMinWgs workgroups of a
// kind, splits go down to kBwdMinItems items (or tiles) each.  Measured on C1 / C4 varlen
// (us): items per workgroup 20 / 24 / 32 / 40 / 48 at every head dim gave 101 / 96 / 92 /
// 88 / 95 on C1 (19 / 19 / 14 / 12 / 10 splits) and 225 / 180 / 205 / 204 / 204 on C4 (4 /
// 3 / 2 / 2 / 2 splits); 43 scaled by 64 / head dim gave 90.3 (11 splits) / 179.0 (3).
// dQ tiles per workgroup 16 / 24 / 32 / 48: C1 94 / 93 / 91 / 92, C4 249 / 248 / 205 / 205.
constexpr int64_t kBwdItemsPerWg64 = 40;
constexpr int64_t kBwdItemsPerWg128 = 22;
constexpr int64_t kBwdTilesPerWg = 32;
constexpr int64_t kBwdMinWgs = 512;
constexpr int64_t kBwdMinItems = 8;
constexpr int64_t kBwdMaxSplits = 32;
constexpr int64_t kBwdMaxKsplit = 8;

// Splits of `units` workgroups of `work` items (or tiles) each under the rules above,
// `per_wg` the kind's bound.
int64_t bwd_split_count(int64_t units, int64_t work, int64_t per_wg, int64_t cap) {
    const int64_t by_work = ceil_div(work, per_wg);
    const int64_t by_fill = std::min(ceil_div(kBwdMinWgs, std::max<int64_t>(1, units)), ceil_div(work, kBwdMinItems));
    return std::max<int64_t>(1, std::min<int64_t>({cap, std::max(by_work, by_fill), std::max<int64_t>(1, work)}));
}

// dK / dV splits over the (query head of the group, 32-row block) items of a key tile.
int bwd_splits(const kmi_attn_bwd_args* a) {
    const int64_t wgs = a->batch * a->heads_kv * ceil_div(a->seq_k, KW);
    const int64_t items = (a->heads_q / a->heads_kv) * ceil_div(a->seq_q, BT);
    const int64_t dp = padded_head_dim(std::max(a->head_dim, bwd_value_dim(a)));
    const int64_t per_wg = dp <= 64 ? kBwdItemsPerWg64 : ceil_div(kBwdItemsPerWg128 * 128, dp);
    return static_cast<int>(bwd_split_count(wgs, items, per_wg, kBwdMaxSplits));
}

// KMI_BWD_KSPLIT=n (read once; tuning): pins the dQ key splits.
int bwd_ksplit_override() {
    static const int v = [] {
        const char* e = std::getenv("KMI_BWD_KSPLIT");
        return e ? std::atoi(e) : 0;
    }();
    return v;
}

// dQ key splits over the 32-key tiles of a (query head, 64-row block).
int bwd_ksplit(const kmi_attn_bwd_args* a) {
    const int64_t tiles = ceil_div(a->seq_k, BT);
    if (bwd_ksplit_override() > 0)
        return static_cast<int>(std::min<int64_t>({bwd_ksplit_override(), kBwdMaxKsplit, tiles}));
    const int64_t wgs = a->batch * a->heads_q * ceil_div(a->seq_q, QW);
    return static_cast<int>(bwd_split_count(wgs, tiles, kBwdTilesPerWg, kBwdMaxKsplit));
}

// Workspace floats: row dot products (padded to 16 bytes); with GQA or splits the dK / dV
// partials; with key splits the dQ partials.
struct BwdLayout {
    size_t dr, part, pdq;
};

BwdLayout bwd_layout(const kmi_attn_bwd_args* a) {
    BwdLayout l{};
    const int64_t dp = padded_head_dim(std::max(a->head_dim, bwd_value_dim(a)));
    l.dr = static_cast<size_t>(ceil_div(a->heads_q * rows_total_of(a), 4) * 4);
    // One split sums the query heads of a K/V head in its registers and writes dK / dV.
    const int s = bwd_splits(a);
    if (s > 1) l.part = static_cast<size_t>(a->heads_kv * s * keys_total_of(a) * dp);
    const int ks = bwd_ksplit(a);
    if (ks > 1) l.pdq = static_cast<size_t>(a->heads_q * ks * rows_total_of(a) * dp);
    return l;
}

size_t bwd_ws_bytes(const kmi_attn_bwd_args* a) {
    const BwdLayout l = bwd_layout(a);
    return (l.dr + 2 * l.part + l.pdq) * sizeof(float);
}

template <typename T, int DP, int MK>
hipError_t launch_bwd(const BwdParams& p, hipStream_t s) {
    const int64_t ntk = ceil_div(p.seq_k, KW), nqb = ceil_div(p.seq_q, QW);
    // The row dots first (both gradient passes read them), then dK / dV and dQ in one grid.
    const dim3 grd(static_cast<unsigned>(static_cast<int64_t>(p.batch) * p.hq * nqb));
    const int64_t ndq = static_cast<int64_t>(p.batch) * p.hq * nqb * p.ksplit;
    const int64_t nkv = static_cast<int64_t>(p.batch) * p.hkv * ntk * p.splits;
    const dim3 grid(static_cast<unsigned>(nkv + ndq));
    if (p.dval != p.d) {
        hipLaunchKernelGGL((attn_bwd_rowdot<T, DP, true>), grd, dim3(BWD_THREADS), 0, s, p);
        hipLaunchKernelGGL((attn_bwd_grads<T, DP, MK, true>), grid, dim3(BWD_THREADS), 0, s, p, static_cast<int>(nkv),
                           static_cast<int>(ndq));
    } else {
        hipLaunchKernelGGL((attn_bwd_rowdot<T, DP, false>), grd, dim3(BWD_THREADS), 0, s, p);
        hipLaunchKernelGGL((attn_bwd_grads<T, DP, MK, false>), grid, dim3(BWD_THREADS), 0, s, p, static_cast<int>(nkv),
                           static_cast<int>(ndq));
    }
    const int64_t dq_blocks = p.pdq ? ceil_div(static_cast<int64_t>(p.hq) * p.rows_total * (p.d / 4), 256) : 0;
    const int64_t kv_blocks =
        p.pdk ? ceil_div(static_cast<int64_t>(p.hkv) * p.keys_total * (std::max(p.d, p.dval) / 4), 256) : 0;
    if (dq_blocks + kv_blocks > 0)
        hipLaunchKernelGGL((attn_bwd_sums<T, DP>), dim3(static_cast<unsigned>(dq_blocks + kv_blocks)), dim3(256), 0, s,
                           p, dq_blocks);
    return hipGetLastError();
}

template <typename T, int DP>
hipError_t launch_bwd_mask(const BwdParams& p, int mk, hipStream_t s) {
    switch (mk) {
        case MK_NONE: return launch_bwd<T, DP, MK_NONE>(p, s);
        case MK_BOOL: return launch_bwd<T, DP, MK_BOOL>(p, s);
        case MK_BF16: return launch_bwd<T, DP, MK_BF16>(p, s);
        case MK_F16: return launch_bwd<T, DP, MK_F16>(p, s);
        default: return launch_bwd<T, DP, MK_F32>(p, s);
    }
}

template <typename T>
hipError_t launch_bwd_dim(const BwdParams& p, int mk, hipStream_t s) {
    switch (padded_head_dim(std::max(p.d, p.dval))) {
        case 32: return launch_bwd_mask<T, 32>(p, mk, s);
        case 64: return launch_bwd_mask<T, 64>(p, mk, s);
        case 96: return launch_bwd_mask<T, 96>(p, mk, s);
        case 128: return launch_bwd_mask<T, 128>(p, mk, s);
        case 192: return launch_bwd_mask<T, 192>(p, mk, s);
        default: return launch_bwd_mask<T, 256>(p, mk, s);
    }
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
    p.splits = bwd_splits(a);
    p.ksplit = bwd_ksplit(a);
    {
        // Partials start 16-byte aligned after the row dot products (DP is a multiple of 4).
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
    const int mk = mask_kind_of(a->mask_mode, a->mask_dtype);
    p.mask = mk == MK_NONE ? nullptr : a->mask;
    p.mask_mode = mk == MK_NONE ? KMI_MASK_NONE : a->mask_mode;
    for (int i = 0; i < 4; ++i) p.ms[i] = a->mask_stride[i];
    p.mask_numel = a->mask_numel;
    p.mask_off = a->mask_mode == KMI_MASK_PACKED ? a->mask_offsets : nullptr;
    p.cu_q = a->cu_seqlens_q;
    p.cu_k = a->cu_seqlens_k;
    p.klen = a->cu_seqlens_q ? nullptr : a->key_lengths;
    p.total_q = static_cast<int>(a->total_q);
    p.total_k = static_cast<int>(a->total_k);
    p.batch = static_cast<int>(a->batch);
    p.hq = static_cast<int>(a->heads_q);
    p.hkv = static_cast<int>(a->heads_kv);
    p.group = p.hq / p.hkv;
    p.seq_q = static_cast<int>(a->seq_q);
    p.seq_k = static_cast<int>(a->seq_k);
    p.causal = a->causal ? 1 : 0;
    p.d = static_cast<int>(a->head_dim);
    p.dval = static_cast<int>(bwd_value_dim(a));
    p.rows_total = rows_total_of(a);
    p.keys_total = keys_total_of(a);
    p.scale = static_cast<float>(a->scale);
    p.c2 = static_cast<float>(a->scale * 1.4426950408889634);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const hipError_t err = a->dtype == KMI_BF16 ? launch_bwd_dim<bf16>(p, mk, s) : launch_bwd_dim<f16>(p, mk, s);
    return hip_status(err, "kmi_attn_bwd");
}
