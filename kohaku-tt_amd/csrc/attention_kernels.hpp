// Flash-attention forward for gfx950: dense / GQA / MQA, causal, bool and additive masks,
// packed variable-length sequences, and split-KV with an fp32 merge pass for short query
// tiles over long key ranges (decode).
//
// Reference semantics (src/kohakutt_native/csrc/aten/attention):
//   - logits = scale * q.k + max(mask, -5e5) (ktt_flash/program.cpp:912-919 mask_operand;
//     varlen_plan.hpp:17 kMaskedLogit); bool masks keep nonzero keys and drop the rest to
//     -5e5 (aten_attention.cpp:223-238).  A masked key therefore has exactly zero weight
//     when its row keeps a key, and a fully-masked row is the softmax over its raw scores.
//   - online softmax in base 2 with scale * log2(e) folded into the logits, P rounded to
//     the operand type for the PV product, O and l in fp32, O / l rounded once
//     (ktt_flash/compute.cpp:193-500 computes the same recurrence on Tensix tiles).
//   - dense causal is top-left (aten_attention.cpp:106-107); varlen causal is bottom-right:
//     query r sees min(Lk, r + 1 + Lk - Lq) keys (varlen_plan.hpp:43-82).
//
// MI355X design (not the reference's Tensix reader/compute/writer split):
//   - a 256-thread workgroup (4 wavefronts) owns 16 * NQB "virtual rows" of one
//     (sequence, K/V head): row r is query position r / G of query head kvh * G + r % G,
//     so the G query heads of a GQA group share every K/V tile;
//   - the four wavefronts hold the same rows and split the key range (every fourth 32-key
//     tile), each staging its own tiles global -> registers -> its own LDS region one tile
//     ahead, so no block-wide barrier runs per tile; their online-softmax states are merged
//     once at the end, in LDS, in a fixed order (deterministic);
//   - S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_{bf16,f16}: with that
//     orientation the S accumulator of a lane is already the B operand of the PV product
//     (no cross-lane shuffles), and each lane owns one query row for the softmax state;
//   - K and V tiles sit in LDS in their natural row layout (padded against bank conflicts);
//     the V^T operand comes from gfx950's transposed LDS read;
//   - the softmax runs on the raw accumulators (scale folded into the exponent's FMA),
//     reduces rows with permlane swaps, and rescales O lazily;
//   - causal work skips key tiles past the tile's last query and issues the heaviest
//     query tiles first; causal / tail masking runs only on the tiles that need it;
//   - decode-shaped calls split the key range across workgroups (fp32 partials merged by
//     a second kernel);
//   - head dims are multiples of 8 up to 256, padded to D (a multiple of 32) with zeros in
//     registers and LDS; each padded D is instantiated in its own attention_d<D>.hip.
//
// Kernels and their launch templates; the host side (argument checks, plan, C ABI) is
// attention.hip.
#pragma once

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "attention_params.hpp"

namespace kmi {
namespace fwd {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazy = 8.f;  // log2 units a row max may grow before O is rescaled


template <typename T>
struct Mfma;
template <>
struct Mfma<bf16> {
    typedef bf16x8 v8;
    static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<f16> {
    typedef f16x8 v8;
    static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// V^T fragments come from V tiles kept in their natural [key][dim] layout through the
// gfx950 transposed LDS read: within each 16-lane group, output lane j, slot s receives
// element j % 4 of the 4-element chunk that source lane 4 s + j / 4 addressed.  Source lane
// k of group g pointing at V[key(g, k / 4)][dim0 + 4 (k % 4)] therefore delivers
// V[key(g, s)][dim0 + j] to lane j, slot s: the A operand of O^T = V^T P^T.
template <typename T>
__device__ __forceinline__ u32x2 lds_read_tr(const T* p) {
    if constexpr (std::is_same<T, bf16>::value) {
        typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
        const auto v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) bf16x4_t*)(const_cast<T*>(p)));
        return __builtin_bit_cast(u32x2, v);
    } else {
        typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 f16x4_t;
        const auto v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (__attribute__((address_space(3))) f16x4_t*)(const_cast<T*>(p)));
        return __builtin_bit_cast(u32x2, v);
    }
}

// A 16-byte head-dim fragment of a row at element column `col`: columns past the head dim
// d (a multiple of 8) read the row's last fragment (in range) and come back as zeros.
template <typename V, typename T>
__device__ __forceinline__ V head_frag(const T* row, int col, int d) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(row + min(col, d - 8));
    return __builtin_bit_cast(V, col < d ? x : u32x4{0u, 0u, 0u, 0u});
}

// Where sequence `seq`'s block of a block-packed mask starts (host-computed offsets when
// given, else the block sizes of the sequences before it added up).
__device__ __forceinline__ int64_t packed_block_offset(const AttnParams& p, int seq) {
    if (p.mask_off) return p.mask_off[seq];
    int64_t off = 0;
    for (int s = 0; s < seq; ++s) {
        const int a0 = min(max(p.cu_q[s], 0), p.total_q);
        const int a1 = min(max(p.cu_q[s + 1], a0), p.total_q);
        const int b0 = min(max(p.cu_k[s], 0), p.total_k);
        const int b1 = min(max(p.cu_k[s + 1], b0), p.total_k);
        off += static_cast<int64_t>(a1 - a0) * (b1 - b0);
    }
    return off;
}


// D: the padded head dim (a multiple of 32; the call's own head dim, a multiple of 8, is
// AttnParams::d and the columns past it are zeros in registers and LDS).
// Unmasked, head-dim-64 tiles of 32 keys and 32 or 64 rows take K and V from global memory
// straight into LDS (buffer loads with the lds modifier).
template <typename T, int D, int NQB, int MK, bool RS, int TWIDTH>
constexpr bool fwd_dma() {
    return MK == MK_NONE && D == 64 && (NQB == 2 || (NQB == 4 && !RS)) && TWIDTH == 32 && sizeof(T) == 2;
}

template <int D, int NQB, int TWIDTH = WN, int NW = NWAVES, bool DMA = false>
struct Shape {
    static constexpr int TW = TWIDTH;    // keys per wavefront tile
    static constexpr int BM = 16 * NQB;  // rows of a workgroup (shared by its wavefronts)
    static constexpr int VP = D + 16;    // V row pitch (elements): transposed b64 reads of 8 rows hit distinct banks
    static constexpr int KP = D + 8;     // K row pitch (elements): b128 reads of 16 rows hit distinct banks
    // Staging of a tile: 16-byte chunks, VPS lanes per row (the chunk count rounded up to
    // a power of two; lanes past the last chunk idle), RPP rows per pass, KIT passes.
    static constexpr int NCH = D / 8;
    static constexpr int VPS = NCH <= 4 ? 4 : (NCH <= 8 ? 8 : (NCH <= 16 ? 16 : 32));
    static constexpr int RPP = kWave / VPS;
    static constexpr int KIT = TW / RPP;
    // The next tile's K / V are loaded during this tile's compute where the registers
    // allow it (D <= 128); wider heads load each tile at the top of its iteration.
    static constexpr bool PREFETCH = D <= 128;
    // K fragments straight from memory into registers (KD) where the wavefront's 64 rows
    // give each loaded fragment the most use; otherwise K is staged in LDS too.
    static constexpr bool KD = D == 64 && NQB == 4 && !DMA;
    static constexpr int TILE = (KD ? 0 : TW * KP) + TW * VP;  // elements of one wavefront's tile
    static constexpr int CP = D + 4;     // merge buffer row pitch (floats)
    // The merge runs over groups of MB row blocks whose buffer fits in the tile area
    // (the buffer must not set the workgroup's LDS size, which bounds workgroups per CU).
    template <typename T>
    static constexpr int merge_blocks() {
        const size_t tiles = static_cast<size_t>(NW) * TILE * sizeof(T);
        const size_t per = static_cast<size_t>(NW) * 16 * CP * sizeof(float);
        const int mb = static_cast<int>(tiles / per);
        return mb < 1 ? 1 : (mb > NQB ? NQB : mb);
    }
    template <typename T>
    static constexpr size_t lds_bytes() {
        const size_t tiles = static_cast<size_t>(NW) * TILE * sizeof(T);
        const size_t comb = static_cast<size_t>(NW) * 16 * merge_blocks<T>() * CP * sizeof(float);
        return (tiles > comb ? tiles : comb) + static_cast<size_t>(NW) * BM * 4 * sizeof(float);
    }
};

// Reductions over the four lanes that hold one query row (l, l^16, l^32, l^48): the
// gfx950 row swaps exchange 16-lane rows (permlane16) and 32-lane halves (permlane32) in
// registers, without the LDS crossbar a generic shuffle uses.
__device__ __forceinline__ float row_max4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float row_sum4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Whether any of the four lanes of this lane's query row has `pred` set.
__device__ __forceinline__ bool row_any4(bool pred, int l16) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(pred) >> l16;
    return (m & 0x0001000100010001ull) != 0;
}

// Four consecutive mask values: one 4-, 8- or 16-byte load at element alignment (gfx950
// global loads take unaligned addresses; the copy tells the compiler the alignment).
template <typename MRaw>
struct Mask4 {
    struct E {
        MRaw e[4];
    };
    static __device__ __forceinline__ void load(const MRaw* at, MRaw (&out)[4]) {
        E x;
        __builtin_memcpy(&x, at, sizeof(E));
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = x.e[i];
    }
};

// Mask value of key `key` of the mask row at `mrow` (zero when the key is out of range),
// read from a clamped, always-valid index: every lane loads, and a group of such loads
// shares one round trip (a per-lane branch around each load can make each wait in turn).
// Used where the loads are few (the decode skip scan); needs lk >= 1 and m_end >= 1.
template <typename MRaw>
__device__ __forceinline__ MRaw mask_load(const MRaw* mp, int64_t mrow, int key, int lk, int64_t m_key, int64_t m_end) {
    const int kc = min(max(key, 0), lk - 1);
    const int64_t mi = min(mrow + static_cast<int64_t>(kc) * m_key, m_end - 1);
    const bool ok = key >= 0 && key < lk && mrow + static_cast<int64_t>(key) * m_key < m_end;
    const MRaw v = mp[mi];
    return ok ? v : MRaw{};
}

// RS (row split, short key ranges): each wavefront owns its own 16 NQB rows and runs every
// key tile itself -- no key split, no merge, no barrier; the workgroup holds 4 row blocks.
template <typename T, int D, int NQB, int MK, bool RS, int TWIDTH, int NW>
__device__ __forceinline__ void attn_block(const AttnParams& p, const int split, const int bh, const int xt) {
    static_assert(!RS || MK == MK_NONE, "row split is for unmasked calls (no block barriers)");
    static_assert(!RS || NW == NWAVES, "row split plans four wavefronts");
    typedef typename Mfma<T>::v8 v8;
    typedef Shape<D, NQB, TWIDTH, NW, fwd_dma<T, D, NQB, MK, RS, TWIDTH>()> S;
    constexpr int TW = S::TW;   // keys per tile
    constexpr int KH = TW / 32;  // 32-key chunks per tile (one PV MFMA each)
    constexpr int BM = S::BM, VP = S::VP, KP = S::KP, CP = S::CP;
    constexpr bool KD = S::KD;
    constexpr int DC = D / 32;  // 32-wide chunks of the head dim
    constexpr int DB = D / 16;  // 16-wide blocks of the head dim
    constexpr int KB = TW / 16;
    constexpr int VPR = S::VPS;          // staging lanes per key row
    constexpr int RPP = S::RPP;          // key rows one wavefront pass covers
    constexpr int KIT = S::KIT;          // passes per tile
    constexpr int NCH = S::NCH;          // 16-byte chunks of a padded row
    static_assert(KIT >= 1 && TW % RPP == 0, "tile shape");
    constexpr bool MASKED = MK != MK_NONE;

    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Uniform per wavefront (readfirstlane tells the compiler so: tile indices and
    // addresses derived from it then live in scalar registers).
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4;
    const int l16 = lane & 15;

    const int seq = fdiv(bh, p.fd_hkv);
    const int kvh = bh - seq * p.hkv;
    const int G = p.group;

    int q0 = 0, lq = p.seq_q, k0 = 0, lk = p.seq_k;
    int64_t qb_off = seq * p.qs[0], kb_off = seq * p.ks[0], vb_off = seq * p.vs[0];
    int64_t ob_off = seq * p.os[0], lb_off = seq * p.ls[0];
    int64_t row_base = static_cast<int64_t>(seq) * p.seq_q;  // partial-row index of query 0
    if (p.cu_q) {
        q0 = min(max(p.cu_q[seq], 0), p.total_q);
        lq = min(max(p.cu_q[seq + 1], q0), p.total_q) - q0;
        k0 = min(max(p.cu_k[seq], 0), p.total_k);
        lk = min(max(p.cu_k[seq + 1], k0), p.total_k) - k0;
        lq = min(lq, p.seq_q);  // the grid covers max_q queries per sequence
        lk = min(lk, p.seq_k);  // and max_k keys (split ranges and LDS are sized from it)
        qb_off = kb_off = vb_off = ob_off = lb_off = 0;
        row_base = q0;
    }
    if (p.klen) lk = min(max(p.klen[seq], 1), p.seq_k);
    const int vrows = lq * G;
    const int r_begin = RS ? (xt * NW + wave) * BM : xt * BM;
    if (lk <= 0) return;
    if constexpr (RS) {
        if (p.rs_shared) {
            // Shared row split: the workgroup stages every key tile of the unit (K rows at
            // pitch KP, then V rows at pitch VP) in one round of loads, then each wavefront
            // runs its own rows over them with no memory traffic in the loop.  Rows past the
            // last key repeat it (finite; their scores are masked).  Every wavefront takes
            // part in the staging and the barrier, rows or not.
            const int nt = (lk + S::TW - 1) / S::TW;
            T* kls = reinterpret_cast<T*>(smem);
            T* vls = kls + nt * S::TW * S::KP;
            const T* kg = static_cast<const T*>(p.k) + kb_off + kvh * p.ks[1] + static_cast<int64_t>(k0) * p.ks[2];
            const T* vg = static_cast<const T*>(p.v) + vb_off + kvh * p.vs[1] + static_cast<int64_t>(k0) * p.vs[2];
            constexpr int VPR_ = D / 8;
            const int nvec = nt * S::TW * VPR_;
            constexpr int MAXV = (kRsTiles * 32 * VPR_ + (NW * kWave) - 1) / (NW * kWave);  // up to kRsTiles tiles (host bound)
            u32x4 kv[MAXV], vv[MAXV];
#pragma unroll
            for (int j = 0; j < MAXV; ++j) {
                const int v = min(tid + (NW * kWave) * j, nvec - 1);
                const int row = min(v / VPR_, lk - 1), ch = v % VPR_;
                // Columns past the head dims read in range and are zeroed.
                const int colk = min(8 * ch, p.d - 8), colv = min(8 * ch, p.dv - 8);
                const u32x4 kx = *reinterpret_cast<const u32x4*>(kg + static_cast<int64_t>(row) * p.ks[2] + colk);
                const u32x4 vx = *reinterpret_cast<const u32x4*>(vg + static_cast<int64_t>(row) * p.vs[2] + colv);
                kv[j] = 8 * ch < p.d ? kx : u32x4{0u, 0u, 0u, 0u};
                vv[j] = 8 * ch < p.dv ? vx : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < MAXV; ++j) {
                const int v = min(tid + (NW * kWave) * j, nvec - 1);
                const int row = v / VPR_, ch = v % VPR_;
                *reinterpret_cast<u32x4*>(kls + row * S::KP + 8 * ch) = kv[j];
                *reinterpret_cast<u32x4*>(vls + row * S::VP + 8 * ch) = vv[j];
            }
            __syncthreads();
        }
    }
    if (r_begin >= vrows) return;
    constexpr int TS = RS ? 1 : NW;  // tile stride of one wavefront
    const int r_end = min(vrows, r_begin + BM);
    const int coff = p.cu_q ? (lk - lq) : 0;  // causal: position i sees keys <= i + coff
    int kend = lk;
    if (p.causal) kend = max(0, min(lk, fdiv(r_end - 1, p.fd_group) + 1 + coff));
    const int ntiles = (kend + TW - 1) / TW;
    // Keys below lim_min are visible to every row of the workgroup: tiles past it need the
    // per-element causal / tail test, the rest do not.
    const int lim_min = p.causal ? min(lk, fdiv(r_begin, p.fd_group) + coff + 1) : lk;
    int t_begin = 0, t_end = ntiles;
    if (p.splits > 1) {
        t_begin = split * p.tiles_per_split;
        t_end = min(ntiles, t_begin + p.tiles_per_split);
    }

    // This lane's rows (the same for every wavefront): Q fragments (B operand of
    // S^T = K Q^T) and row metadata.
    const T* qp = static_cast<const T*>(p.q);
    v8 qf[NQB][DC];
    int lim[NQB];
    int64_t mrow[NQB];
    int64_t m_key = 0, m_end = 0;
    const void* mptr = p.mask;
    bool mvec = false;  // uniform: full tiles read their mask values four keys per load
    int64_t m_seq_packed = 0;  // packed masks: the first value of this sequence's block
    if constexpr (MASKED) {
        // Packed masks are bounded by their element count; strided ones by their shape.
        m_end = p.mask_mode == KMI_MASK_PACKED ? p.mask_numel : INT64_MAX;
        m_key = p.mask_mode == KMI_MASK_PACKED ? 1 : p.ms[3];
        if (p.mask_mode == KMI_MASK_PACKED) m_seq_packed = packed_block_offset(p, seq);
        // A packed block must lie within the mask for the unchecked vector loads.
        mvec = p.mask_vec4 && (p.mask_mode != KMI_MASK_PACKED || m_seq_packed + static_cast<int64_t>(lq) * lk <= m_end);
    }
#pragma unroll
    for (int b = 0; b < NQB; ++b) {
        const int r = r_begin + 16 * b + l16;
        const bool valid = r < r_end;
        const int rr = valid ? r : r_begin;
        const int pos = fdiv(rr, p.fd_group);
        const int head = kvh * G + (rr - pos * G);
        lim[b] = p.causal ? min(lk, pos + coff + 1) : lk;  // keys [0, lim) are visible
        const T* src = qp + qb_off + head * p.qs[1] + static_cast<int64_t>(q0 + pos) * p.qs[2];
        // Rows past the end read row r_begin (in range) and are never written; columns past
        // the head dim read in range and are zeroed below (a uniform fix-up, so that the
        // common case waits for these loads only where the loop first uses them).
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[b][c] = *reinterpret_cast<const v8*>(src + min(32 * c + 8 * g4, p.d - 8));
        if constexpr (MASKED) {
            if (p.mask_mode == KMI_MASK_PACKED) {
                mrow[b] = m_seq_packed + static_cast<int64_t>(pos) * lk;
            } else {
                const int64_t m_seq = p.cu_q ? (static_cast<int64_t>(q0) * p.ms[2] + static_cast<int64_t>(k0) * p.ms[3])
                                             : seq * p.ms[0];
                mrow[b] = m_seq + head * p.ms[1] + static_cast<int64_t>(pos) * p.ms[2];
            }
        }
    }

    // KD: K fragments come straight from memory into MFMA A-operand registers: lane
    // (g4, l16) holds key 16 kb + l16, dims 32 c + 8 g4 .. + 7 of S^T = K Q^T.  Otherwise
    // K rows are staged through the wavefront's LDS tile like V (key row `krow` + RPP
    // per pass); V always is, for the transposed reads.
    //
    // Tiles load through a buffer resource per tile, based at its first key and ending at
    // the unit's last key (at most one tile of rows): rows past the end read as zeros, with
    // no tail branches.  Row strides are at most 2^24 elements (checked on the host), so the
    // in-tile byte offsets fit 32 bits.
    const int krow = lane / VPR, dg = lane - (lane / VPR) * VPR;
    // Staging lanes past the padded row idle; chunks past the head dim stage zeros (their
    // loads stay within the row's range).
    const bool stage_lane = dg < NCH;
    const bool stage_live = 8 * dg < p.d;  // (K's chunks; V's past dv need not be zero)
    const int dgc = min(dg, (p.d - 1) / 8), dgcv = min(dg, (p.dv - 1) / 8);
    // Padded head dims: K's columns past d must be zeros (they meet Q's zero columns in
    // S, and a finite value of another row there could still be inf); V's need not be
    // (they only reach output columns past d, which are never written).  Uniform.
    const bool kpad = p.d < D;
    const int64_t kstride = p.ks[2] * static_cast<int64_t>(sizeof(T)), vstride = p.vs[2] * static_cast<int64_t>(sizeof(T));
    const char* kunit = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + kb_off + kvh * p.ks[1] +
                                                      static_cast<int64_t>(k0) * p.ks[2]);
    const char* vunit = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + vb_off + kvh * p.vs[1] +
                                                      static_cast<int64_t>(k0) * p.vs[2]);
    const uint32_t k_lane = KD ? static_cast<uint32_t>(l16 * kstride + 16 * g4) : static_cast<uint32_t>(krow * kstride + 16 * dgc);
    const uint32_t v_lane = static_cast<uint32_t>(krow * vstride + 16 * dgcv);
    // Bytes per key of the DMA variants' ranges (rows x span; the host keeps rows that
    // overlap off them; a zero row stride repeats one row).  The other tile loads' ranges
    // end with the last row's data (rows_extent), so rows that overlap, as in an
    // as_strided view with a row stride below the head dim, are read in full.
    const uint32_t kspan = static_cast<uint32_t>(kstride > 0 ? kstride : p.d * static_cast<int64_t>(sizeof(T)));
    const uint32_t vspan = static_cast<uint32_t>(vstride > 0 ? vstride : p.dv * static_cast<int64_t>(sizeof(T)));
    T* kl = reinterpret_cast<T*>(smem) + wave * S::TILE;
    T* vl = kl + (KD ? 0 : TW * KP);

    // DMA2 (32- and 64-row tiles at D = 64, unmasked): K and V tiles go from global memory
    // straight into the wavefront's LDS tile (buffer loads with the lds modifier: no
    // staging registers, no LDS store instructions).  A step reads all of its tile's K and
    // V fragments first, then requests the next tile into the same buffer, so the wait
    // before the next step's reads is for loads issued a whole step earlier.  Rows sit at
    // pitch D with 16-byte chunks XOR-swizzled (K: chunk c of row r at c ^ kswz(r); V at
    // c ^ vswz(r)) so that K's row reads and V's transposed reads hit distinct banks.  DMA
    // instruction i fills rows 8 i .. 8 i + 7; lane q the slot of row 8 i + q / 8,
    // physical chunk q % 8.
    constexpr bool DMA2 = fwd_dma<T, D, NQB, MK, RS, TWIDTH>();
    // 32-row DMA tiles raise the wavefront's issue priority over its S and PV MFMA
    // sections (s_setprio 1, back to 0 for the softmax and the loads): of the three or four
    // wavefronts on a SIMD, one in an MFMA section then wins the arbitration while the
    // others run their softmax, which keeps the matrix unit fed (C1 23.3 -> 22.1 us; 64-row
    // tiles measured 2-5% slower with it, head dim 128 no change).
    constexpr bool PRIO = DMA2 && NQB == 2;
    // Swizzles chosen so that rows r and r + 16 share one (the fragment reads of the second
    // 16-key block are an immediate offset away) and, within a DMA instruction's eight rows
    // 8 i + a, depend on a and the parity of i only (the row term 8 i * stride goes to the
    // scalar offset; two lane offsets per operand).
    auto kswz = [](int r) { return (r & 7) ^ ((r >> 3) & 1); };
    auto vswz = [](int r) { return 2 * ((r ^ (r >> 2)) & 3); };
    T* const kd2 = kl;
    T* const vd2 = kl + TW * D;
    uint32_t dk_b[DMA2 ? 2 : 1], dv_b[DMA2 ? 2 : 1];  // DMA lane offsets for even / odd i
    int kfo[DMA2 ? DC : 1];                          // K fragment element offsets (keys 0..15)
    int vtro[DMA2 ? DB : 1];                         // V transposed-read element offsets (first 16 keys)
    if constexpr (DMA2) {
        // Padded head dims: chunks past d (K) / dv (V) repeat the last.
        const int cmax = (p.d - 1) / 8, cmaxv = (p.dv - 1) / 8;
        const int a = lane >> 3, q7 = lane & 7;
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            dk_b[par] = static_cast<uint32_t>(a) * static_cast<uint32_t>(kstride) +
                        16u * static_cast<uint32_t>(min(q7 ^ kswz(8 * par + a), cmax));
            dv_b[par] = static_cast<uint32_t>(a) * static_cast<uint32_t>(vstride) +
                        16u * static_cast<uint32_t>(min(q7 ^ vswz(8 * par + a), cmaxv));
        }
#pragma unroll
        for (int c = 0; c < DC; ++c) kfo[c] = l16 * D + 8 * ((4 * c + g4) ^ kswz(l16));
        const int r = 4 * g4 + (l16 >> 2);
#pragma unroll
        for (int d = 0; d < DB; ++d) vtro[d] = r * D + 8 * (((2 * d) ^ vswz(r)) | ((l16 >> 1) & 1)) + 4 * (l16 & 1);
    }
    // One operand's tile: K (V = false) or V into its half of the wavefront's buffer.
    auto dma_half = [&](int tt, bool V) {
        if constexpr (DMA2) {
            const int key0 = tt * TW;
            const int rows_here = min(lk - key0, TW);
            const int64_t stride = V ? vstride : kstride;
            // Rows of `stride` bytes (the host keeps rows that overlap off these variants).
            const auto rs = buffer_rsrc((V ? vunit : kunit) + key0 * stride,
                                        static_cast<uint32_t>(rows_here) * (V ? vspan : kspan));
            T* const dst = V ? vd2 : kd2;
            if (rows_here == TW) {
#pragma unroll
                for (int i = 0; i < TW / 8; ++i)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + i * 512),
                                                             16, V ? dv_b[i & 1] : dk_b[i & 1],
                                                             static_cast<int>(8 * i * static_cast<uint32_t>(stride)), 0, 0);
            } else {
                // Last tile: rows past the unit's last key repeat it (finite; their scores
                // are masked), so every lane reads in range and every slot is written.
                const int cmax = ((V ? p.dv : p.d) - 1) / 8;
#pragma unroll
                for (int i = 0; i < TW / 8; ++i) {
                    const int r = 8 * i + (lane >> 3);
                    const uint32_t rr = static_cast<uint32_t>(min(r, rows_here - 1));
                    const uint32_t off = rr * static_cast<uint32_t>(stride) +
                                         16u * static_cast<uint32_t>(min((lane & 7) ^ (V ? vswz(r) : kswz(r)), cmax));
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + i * 512),
                                                             16, off, 0, 0, 0);
                }
            }
        } else {
            (void)tt;
            (void)V;
        }
    };
    auto dma_tile = [&](int tt) {
        dma_half(tt, false);
        dma_half(tt, true);
    };
    v8 vpre[DMA2 ? DB : 1];  // DMA2: this tile's V fragments, read at the top of its step

    // Mask values of the staged tile, loaded with its K / V (raw element type; converted
    // when the tile is computed, so the loads stay in flight meanwhile).
    typedef typename std::conditional<MK == MK_BOOL, uint8_t,
            typename std::conditional<MK == MK_BF16 || MK == MK_F16, uint16_t, float>::type>::type MRaw;
    MRaw mpre[MASKED ? NQB : 1][KB][4];

    typedef v8 KRegs[KD ? KB : 1][KD ? DC : 1];
    KRegs kreg;  // KD: the next tile's K, loaded as soon as the S MFMAs consumed this tile's
    u32x4 kst[KD ? 1 : KIT];
    u32x4 vreg[KIT];
    // The row shifts of a tile's passes are uniform; the compiler barrier on them keeps the
    // per-lane offsets from being precomputed into registers held across the loop.
    auto load_k = [&](int t, KRegs& kr) {
        const int key0 = t * TW;
        const auto rs = buffer_rsrc(kunit + key0 * kstride, rows_extent(min(lk - key0, TW), static_cast<uint32_t>(kstride), static_cast<uint32_t>(p.d * sizeof(T))));
        uint32_t step = static_cast<uint32_t>(kstride);
        __asm__ volatile("" : "+s"(step));
        if constexpr (KD) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int c = 0; c < DC; ++c) {
                    kr[kb][c] = __builtin_bit_cast(v8, buffer_load16(rs, k_lane + 16 * kb * step + 64 * c));
                }
            }
            if (kpad) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int c = 0; c < DC; ++c)
                        if (32 * c + 8 * g4 >= p.d) kr[kb][c] = v8{};
            }
        } else {
#pragma unroll
            for (int i = 0; i < KIT; ++i) kst[i] = buffer_load16(rs, k_lane + i * RPP * step);
            if (kpad && !stage_live) {
#pragma unroll
                for (int i = 0; i < KIT; ++i) kst[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    // V rows and mask values of tile t.
    auto load_v = [&](int t) {
        const int key0 = t * TW;
        const auto rs = buffer_rsrc(vunit + key0 * vstride, rows_extent(min(lk - key0, TW), static_cast<uint32_t>(vstride), static_cast<uint32_t>(p.dv * sizeof(T))));
        uint32_t step = static_cast<uint32_t>(vstride);
        __asm__ volatile("" : "+s"(step));
#pragma unroll
        for (int i = 0; i < KIT; ++i) vreg[i] = buffer_load16(rs, v_lane + i * RPP * step);
        if constexpr (MASKED) {
            const MRaw* mp = static_cast<const MRaw*>(mptr);
            if (mvec && key0 + TW <= lk) {
                // Whole tile in range: four keys per load.
#pragma unroll
                for (int b = 0; b < NQB; ++b)
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) Mask4<MRaw>::load(mp + mrow[b] + key0 + 16 * kb + 4 * g4, mpre[b][kb]);
            } else {
#pragma unroll
                for (int b = 0; b < NQB; ++b) {
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int kk = key0 + 16 * kb + 4 * g4 + i;
                            const int64_t mi = mrow[b] + kk * m_key;
                            mpre[b][kb][i] = (kk < lk && mi < m_end) ? mp[mi] : MRaw{};
                        }
                    }
                }
            }
        }
    };
    auto load_tile = [&](int t) {
        load_k(t, kreg);
        load_v(t);
    };
    // V (and staged K) rows as loaded.
    auto store_k = [&]() {
        if constexpr (!KD) {
            if (!stage_lane) return;
#pragma unroll
            for (int i = 0; i < KIT; ++i) *reinterpret_cast<u32x4*>(kl + (krow + i * RPP) * KP + 8 * dg) = kst[i];
        }
    };
    auto store_v = [&]() {
        if (!stage_lane) return;
#pragma unroll
        for (int i = 0; i < KIT; ++i) *reinterpret_cast<u32x4*>(vl + (krow + i * RPP) * VP + 8 * dg) = vreg[i];
    };
    auto store_tile = [&]() {
        store_k();
        store_v();
    };

    // Running state per row block: O^T accumulators, the row sums as MFMA accumulators
    // (every element of lacc[b] holds lane l16's row sum), the reference point m (base-2
    // logit units), m + 8 (the lazy-rescale threshold) and -m for the exponent.
    f32x4 o[DB][NQB];
    // Row sums as MFMA columns (P times a column of ones: one MFMA per 32 keys and row
    // block, where fp32 adds would take eight VALU instructions).
    f32x4 lacc[NQB];
    float m_run[NQB], m_thr[NQB], neg_m[NQB];
    bool raw[NQB];
#pragma unroll
    for (int b = 0; b < NQB; ++b) {
        raw[b] = MASKED;
        m_run[b] = -INFINITY;
        m_thr[b] = -INFINITY;
        neg_m[b] = 0.f;
        lacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < DB; ++d) o[d][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    v8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = static_cast<T>(1.f);
    // A negative scale flips the sign of Q (exact) so that the exponent's multiplier is
    // positive and a larger score is a larger logit.
    // Each wavefront's first tile is requested before anything else waits on memory (its
    // loads share one round trip with the Q fragments and the mask-row scan below).
    const int t_spec = t_begin + (RS ? 0 : wave);
    const bool rs_shared = RS && p.rs_shared;
    if constexpr (DMA2) {
        if (t_spec < t_end && !rs_shared) dma_tile(t_spec);
    } else if (S::PREFETCH && t_spec < t_end && !rs_shared) {
        load_tile(t_spec);
    }
    // Padded head dims zero Q's columns past d; a negative scale flips Q's sign.  Both are
    // uniform, and only they wait for the Q loads here.
    float c2 = p.scale_log2;
    const bool qneg = c2 < 0.f;
    if (qneg) c2 = -c2;
    if (kpad || qneg) {
        const uint32_t flip = qneg ? 0x80008000u : 0u;
#pragma unroll
        for (int b = 0; b < NQB; ++b)
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const u32x4 x = __builtin_bit_cast(u32x4, qf[b][c]) ^ flip;
                qf[b][c] = __builtin_bit_cast(v8, 32 * c + 8 * g4 < p.d ? x : u32x4{0u, 0u, 0u, 0u});
            }
    }

    // Key-mask tile skipping: with a mask that depends only on the key (a padding mask),
    // tiles whose every key is masked contribute exactly nothing once the row is known to
    // keep a key somewhere, so they are neither loaded nor computed.  A scan of the whole
    // mask row establishes that first (a row with no kept key needs every raw score).
    constexpr int FLAG_CAP = NW * BM * 4 * static_cast<int>(sizeof(float));
    uint8_t* tflag = smem + S::template lds_bytes<T>() - FLAG_CAP;
    bool skip = false;
    if constexpr (MASKED) {
        constexpr int EPV = 16 / static_cast<int>(sizeof(MRaw));
        const int ntl = t_end - t_begin;
        const MRaw* mrow0 = static_cast<const MRaw*>(mptr) + mrow[0];
        // Uniform across the workgroup: with zero head and query strides every row of the
        // workgroup reads the same mask row.
        const bool eligible = p.mask_mode == KMI_MASK_STRIDED && p.ms[1] == 0 && p.ms[2] == 0 &&
                              m_key == 1 && ntl > 0 && ntl <= FLAG_CAP && lk % EPV == 0 &&
                              (reinterpret_cast<uintptr_t>(mrow0) & 15) == 0;
        if (eligible) {
            for (int i = tid; i < ntl; i += (NW * kWave)) tflag[i] = 0;
            __syncthreads();
            bool keeps = false;
            const int nv = lk / EPV;
            for (int v0 = tid; v0 < nv; v0 += 2 * (NW * kWave)) {
                u32x4 raw2[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int v = v0 + u * (NW * kWave);
                    raw2[u] = v < nv ? *reinterpret_cast<const u32x4*>(mrow0 + static_cast<int64_t>(v) * EPV)
                                     : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int v = v0 + u * (NW * kWave);
                    if (v >= nv) continue;
                    const MRaw* e = reinterpret_cast<const MRaw*>(&raw2[u]);
#pragma unroll
                    for (int j = 0; j < EPV; ++j) {
                        if (mask_logit_of<MK>(e[j]) > kMaskedLogit) {
                            keeps = true;
                            const int tile = (v * EPV + j) / TW;
                            if (tile >= t_begin && tile < t_end) tflag[tile - t_begin] = 1;
                        }
                    }
                }
            }
            skip = __syncthreads_or(keeps);
        }
    }
    auto next_tile = [&](int t) {
        if (skip) {
            while (t < t_end && !tflag[t - t_begin]) t += TS;
        }
        return t;
    };

    // Softmax and PV of tile t from its S^T accumulators (and mask values).
    typedef MRaw MCur[MASKED ? NQB : 1][KB][4];
    auto consume = [&](const int t, const f32x4 (&s)[KB][NQB], const MCur& mcur) {
        const int key0 = t * TW;
        const bool edge = key0 + TW > lim_min;
        // x: logits in base-2 units times 1 / xs.  Mask-free rows keep the raw accumulators
        // (the scale is folded into the exponent's FMA below), -inf where not visible.
        float x[NQB][KB][4];
        float xs = c2;  // multiplier of x in the exponent (positive)
#pragma unroll
        for (int b = 0; b < NQB; ++b) {
            const int rel = lim[b] - key0 - 4 * g4;  // element (kb, i) is visible iff 16 kb + i < rel
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) x[b][kb][i] = s[kb][b][i];
            }
            if constexpr (MASKED) {
                xs = 1.f;
                bool keep_any = false;
                float xm[KB][4];
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool vis = 16 * kb + i < rel;
                        float val = x[b][kb][i] * c2;
                        float vm = -INFINITY;
                        if (vis) {
                            const float ml = mask_logit_of<MK>(mcur[b][kb][i]);
                            if (ml > kMaskedLogit) {
                                vm = val + kLog2e * ml;
                                keep_any = true;
                            }
                        } else {
                            val = -INFINITY;
                        }
                        x[b][kb][i] = val;
                        xm[kb][i] = vm;
                    }
                }
                // A row runs over its raw scores (mask ignored: the reference's result for
                // a row whose every key is masked) until its first kept key; then it drops
                // that state and masked keys get exactly zero weight.
                if (raw[b] && row_any4(keep_any, l16)) {
                    raw[b] = false;
                    m_run[b] = -INFINITY;
                    m_thr[b] = -INFINITY;
                    neg_m[b] = 0.f;
                }
                if (!raw[b]) {
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) x[b][kb][i] = xm[kb][i];
                    }
                }
            } else if (edge) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[b][kb][i] = 16 * kb + i < rel ? x[b][kb][i] : -INFINITY;
                }
            }
        }
        // Lazy rescale: the reference point m moves only when a score would exceed it by
        // more than 2^8 (P stays <= 256, exact in bf16's exponent range).  Each lane checks
        // its own scores against that threshold; only a row block where some lane crosses
        // it pays for the row reduction, the move and the O / l rescale.
#pragma unroll
        for (int b = 0; b < NQB; ++b) {
            // A chain of three-way maxima (v_max3): 4 instructions per 8 scores.
            float lmax = fmaxf(x[b][0][0], x[b][0][1]);
#pragma unroll
            for (int j = 2; j < 4 * KB; j += 2) {
                const float a0 = x[b][j / 4][j % 4], a1 = x[b][(j + 1) / 4][(j + 1) % 4];
                lmax = fmaxf(fmaxf(lmax, a0), a1);
            }
            if (__builtin_amdgcn_ballot_w64(lmax * xs > m_thr[b])) {
                const float mt = row_max4(lmax) * xs;
                const bool move = mt > m_thr[b];
                float alpha = 1.f;
                if (move) {
                    alpha = __builtin_amdgcn_exp2f(m_run[b] - mt);  // 0 while m was -inf
                    m_run[b] = mt;
                    m_thr[b] = mt + kLazy;
                    neg_m[b] = -mt;
                }
                if (__builtin_amdgcn_ballot_w64(move)) {
                    lacc[b] *= alpha;
#pragma unroll
                    for (int d = 0; d < DB; ++d) o[d][b] *= alpha;
                }
            }
        }
        // O^T += V^T P^T, and l += P 1 (the row sums of the bf16 weights, as MFMA columns).
        // The V fragments are requested first; the MFMAs of row block b then interleave
        // with the exponentials of row block b + 1 (scheduling groups below).
        v8 vf[KH][DB];
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
        if (DMA2 && !rs_shared) {
#pragma unroll
            for (int d = 0; d < DB; ++d) vf[0][d] = vpre[d];
        } else
#pragma unroll
        for (int h = 0; h < KH; ++h) {
            const T* vsrc = vl + (32 * h + 4 * g4 + (l16 >> 2)) * VP + 4 * (l16 & 3);
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const u32x2 lo = lds_read_tr(vsrc + 16 * d);            // keys 32 h + 4 g + s
                const u32x2 hi = lds_read_tr(vsrc + 16 * VP + 16 * d);  // keys 32 h + 16 + 4 g + s
                vf[h][d] = __builtin_bit_cast(v8, u32x4{lo[0], lo[1], hi[0], hi[1]});
            }
        }
#pragma unroll
        for (int b = 0; b < NQB; ++b) {
#pragma unroll
            for (int h = 0; h < KH; ++h) {
                // The 32 keys of chunk h: S accumulator blocks 2 h and 2 h + 1.
                v8 pf;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[b][2 * h][i], xs, neg_m[b]));
                    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[b][2 * h + 1][i], xs, neg_m[b]));
                    pf[i] = static_cast<T>(e0);
                    pf[4 + i] = static_cast<T>(e1);
                }
                lacc[b] = Mfma<T>::run(ones, pf, lacc[b]);
#pragma unroll
                for (int d = 0; d < DB; ++d) o[d][b] = Mfma<T>::run(vf[h][d], pf, o[d][b]);
            }
        }
        __builtin_amdgcn_iglp_opt(2);
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    };
    auto take_mask = [&](MCur& mcur) {
        if constexpr (MASKED) {
#pragma unroll
            for (int b = 0; b < NQB; ++b)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mcur[b][kb][i] = mpre[b][kb][i];
        }
    };

    int t = next_tile(t_spec);
    if (!DMA2 && S::PREFETCH && t != t_spec && t < t_end && !rs_shared) load_tile(t);
    if (DMA2 && !rs_shared) {
        // A tile's K loads are requested before its V loads.  32-row tiles (row split or
        // not): a step waits for its K alone (the four V loads after it may still be in
        // flight; an explicit wait, as the compiler's own covers the transposed reads but
        // not the plain ones), reads the K fragments and issues the S MFMAs, then waits for
        // its V and reads V^T while they run (C2 B=32 17.1 -> 16.5 us; C1, with the MFMA
        // priority above, 22.2 -> 21.9 us).  64-row key-split tiles read K and V^T first,
        // then issue the S MFMAs (the split order measured 3% slower on C5 self).  Either
        // way the next tile is requested (K, then V) once every read of this one is done.
        static_assert(TW / 8 == 4, "four DMA loads per operand (the vmcnt(4) waits)");
        constexpr bool KFIRST = RS || NQB == 2;
        auto read_v = [&]() {
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const u32x2 lo = lds_read_tr(vd2 + vtro[d]);           // keys 4 g + s
                const u32x2 hi = lds_read_tr(vd2 + 16 * D + vtro[d]);  // keys 16 + 4 g + s (same swizzle)
                vpre[d] = __builtin_bit_cast(v8, u32x4{lo[0], lo[1], hi[0], hi[1]});
            }
        };
        while (t < t_end) {
            const int t_next = next_tile(t + TS);
            if constexpr (KFIRST) {
                __asm__ volatile("s_waitcnt vmcnt(4)" ::: "memory");
            } else {
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            v8 kf[KB][DC];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int c = 0; c < DC; ++c) kf[kb][c] = *reinterpret_cast<const v8*>(kd2 + 16 * kb * D + kfo[c]);
            if (kpad) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int c = 0; c < DC; ++c)
                        if (32 * c + 8 * g4 >= p.d) kf[kb][c] = v8{};
            }
            if constexpr (!KFIRST) read_v();
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            f32x4 s[KB][NQB];
            if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int b = 0; b < NQB; ++b) {
                    s[kb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < DC; ++c) s[kb][b] = Mfma<T>::run(kf[kb][c], qf[b][c], s[kb][b]);
                }
            }
            if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
            if constexpr (KFIRST) {
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile's V landed
                read_v();
                // The V reads are done before the next tile lands in the same buffer.
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            if (t_next < t_end) dma_tile(t_next);
            const MCur mnone{};
            consume(t, s, mnone);
            t = t_next;
        }
    } else if (rs_shared) {
        // Every key tile is in LDS: S, softmax and PV per tile, nothing else.
        T* const kls = reinterpret_cast<T*>(smem);
        T* const vls = kls + ((lk + TW - 1) / TW) * TW * KP;
        for (; t < t_end; ++t) {
            kl = kls + t * TW * KP;
            vl = vls + t * TW * VP;
            v8 kf[KB][DC];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int c = 0; c < DC; ++c)
                    kf[kb][c] = *reinterpret_cast<const v8*>(kl + (16 * kb + l16) * KP + 32 * c + 8 * g4);
            }
            f32x4 s[KB][NQB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int b = 0; b < NQB; ++b) {
                    s[kb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < DC; ++c) s[kb][b] = Mfma<T>::run(kf[kb][c], qf[b][c], s[kb][b]);
                }
            }
            const MCur mnone{};
            consume(t, s, mnone);
        }
    } else if constexpr (KD) {
        // K fragments in registers (64-row workgroups): the next tile's K loads into the set
        // the S MFMAs just consumed; V is one tile ahead through LDS.
        int t1 = next_tile(t + TS);
        auto step = [&](KRegs& kc) {
            // LDS keeps one wavefront's accesses in order (the previous tile's reads,
            // these writes, this tile's reads): only the compiler must keep it.
            __asm__ volatile("" ::: "memory");
            store_tile();
            MCur mcur;
            take_mask(mcur);
            const int t_next = t1;
            if (t_next < t_end) load_v(t_next);
            f32x4 s[KB][NQB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int b = 0; b < NQB; ++b) {
                    s[kb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < DC; ++c) s[kb][b] = Mfma<T>::run(kc[kb][c], qf[b][c], s[kb][b]);
                }
            }
            const int t_nn = t_next < t_end ? next_tile(t_next + TS) : t_end;
            if (t_next < t_end) load_k(t_next, kc);
            consume(t, s, mcur);
            t = t_next;
            t1 = t_nn;
        };
        while (t < t_end) step(kreg);
    } else {
        while (t < t_end) {
            // LDS keeps one wavefront's accesses in order (the previous tile's reads,
            // these writes, this tile's reads): only the compiler must keep it.
            __asm__ volatile("" ::: "memory");
            if constexpr (S::PREFETCH) {
                store_tile();
            } else {
                // Wide heads: this tile's K, then its V, loaded and staged here.
                load_k(t, kreg);
                store_k();
                load_v(t);
                store_v();
            }
            MCur mcur;
            take_mask(mcur);
            const int t_next = next_tile(t + TS);
            // S^T = K Q^T from the LDS tile, with the whole next tile requested first.
            if (S::PREFETCH && t_next < t_end) load_tile(t_next);
            v8 kf[KB][DC];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int c = 0; c < DC; ++c)
                    kf[kb][c] = *reinterpret_cast<const v8*>(kl + (16 * kb + l16) * KP + 32 * c + 8 * g4);
            }
            f32x4 s[KB][NQB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int b = 0; b < NQB; ++b) {
                    s[kb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < DC; ++c) s[kb][b] = Mfma<T>::run(kf[kb][c], qf[b][c], s[kb][b]);
                }
            }
            consume(t, s, mcur);
            t = t_next;
        }
    }

    if constexpr (RS) {
        // The wavefront's rows are complete: normalise and write them (lane (g4, l16) holds
        // dims 16 d + 4 g4 .. + 3 of row 16 b + l16).
#pragma unroll
        for (int b = 0; b < NQB; ++b) {
            const int r = r_begin + 16 * b + l16;
            const float l = lacc[b][0];
            if (r >= r_end) continue;
            const int pos = fdiv(r, p.fd_group);
            const int head = kvh * G + (r - pos * G);
            const float inv = l > 0.f ? 1.f / l : 0.f;
            T* dst = static_cast<T*>(p.out) + ob_off + head * p.os[1] + static_cast<int64_t>(q0 + pos) * p.os[2];
            typedef T v4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                v4 w;
#pragma unroll
                for (int i = 0; i < 4; ++i) w[i] = static_cast<T>(o[d][b][i] * inv);
                if (16 * d + 4 * g4 < p.dv) *reinterpret_cast<v4*>(dst + 16 * d + 4 * g4) = w;
            }
            if (p.lse && g4 == 0)
                p.lse[lb_off + head * p.ls[1] + static_cast<int64_t>(q0 + pos) * p.ls[2]] =
                    l > 0.f ? (m_run[b] + log2f(l)) * kLn2 : -INFINITY;
        }
        return;
    }
    // Merge the wavefronts' states: (m, l, raw) per wavefront and row as 16-byte records
    // (read back with one load per wavefront, combined without branches) and the O
    // accumulators.  Wavefronts in masked mode (they met a kept key) win; a row none of
    // them kept a key for merges every wavefront's raw-score state.  The sums run in a
    // fixed wavefront order.
    f32x4* stats = reinterpret_cast<f32x4*>(smem + S::template lds_bytes<T>() - NW * BM * sizeof(f32x4));
    float l_run[NQB];
#pragma unroll
    for (int b = 0; b < NQB; ++b) {
        l_run[b] = lacc[b][0];
    }
    auto combine = [&](const f32x4 (&sw)[NW], float (&wt)[NW], float& m, float& lt, bool& any_masked) {
        any_masked = false;
#pragma unroll
        for (int w = 0; w < NW; ++w) any_masked = any_masked || (sw[w][2] == 0.f && sw[w][1] > 0.f);
        m = -INFINITY;
        bool sel[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            sel[w] = (!any_masked || sw[w][2] == 0.f) && sw[w][1] > 0.f;
            m = fmaxf(m, sel[w] ? sw[w][0] : -INFINITY);
        }
        lt = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            wt[w] = sel[w] ? __builtin_amdgcn_exp2f(sw[w][0] - m) : 0.f;
            lt += wt[w] * sw[w][1];
        }
    };
    auto write_row = [&](int r, int col, const f32x4& acc) {
        if (col >= p.dv) return;  // padded head-dim columns
        const int pos = fdiv(r, p.fd_group);
        const int head = kvh * G + (r - pos * G);
        if (p.splits > 1) {
            const int64_t prow = (static_cast<int64_t>(split) * p.rows_total + row_base + pos) * p.hq + head;
            *reinterpret_cast<f32x4*>(p.part_o + prow * D + col) = acc;
        } else {
            typedef T v4 __attribute__((ext_vector_type(4)));
            v4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = static_cast<T>(acc[i]);
            T* dst = static_cast<T*>(p.out) + ob_off + head * p.os[1] + static_cast<int64_t>(q0 + pos) * p.os[2];
            *reinterpret_cast<v4*>(dst + col) = w;
        }
    };
    auto write_lse = [&](int r, float row_lse, bool row_raw) {
        const int pos = fdiv(r, p.fd_group);
        const int head = kvh * G + (r - pos * G);
        if (p.splits > 1) {
            const int64_t prow = (static_cast<int64_t>(split) * p.rows_total + row_base + pos) * p.hq + head;
            p.part_lse[2 * prow] = row_lse;
            p.part_lse[2 * prow + 1] = row_raw ? 1.f : 0.f;
        } else if (p.lse) {
            // A row without a kept key: its logits all carry the -5e5 clamp.
            p.lse[lb_off + head * p.ls[1] + static_cast<int64_t>(q0 + pos) * p.ls[2]] =
                row_lse * kLn2 + (row_raw ? kMaskedLogit : 0.f);
        }
    };
    constexpr int VPRO = D / 4;  // float4 columns per row
    // OWN (head dim 64): each wavefront's O over its own tile area, one barrier, the
    // combine per output item.  Head dim 128 measured 2-4% faster with the grouped merge
    // below (each wavefront scales its own O once per row; the final pass only sums).
    constexpr bool OWN = D == 64 && static_cast<size_t>(S::TILE) * sizeof(T) >= static_cast<size_t>(NQB) * 16 * CP * sizeof(float);
    if constexpr (OWN) {
        // Each wavefront's O fits over its own tile area, which no other wavefront reads:
        // one barrier (the mask-skip flags share the statistics area, so a skipping
        // workgroup waits for every wavefront's loop first).
        if (skip) __syncthreads();
        float* mine = reinterpret_cast<float*>(smem + static_cast<size_t>(wave) * S::TILE * sizeof(T));
#pragma unroll
        for (int b = 0; b < NQB; ++b) {
#pragma unroll
            for (int d = 0; d < DB; ++d)
                *reinterpret_cast<f32x4*>(mine + (16 * b + l16) * CP + 16 * d + 4 * g4) = o[d][b];
            if (g4 == 0) stats[wave * BM + 16 * b + l16] = f32x4{m_run[b], l_run[b], raw[b] ? 1.f : 0.f, 0.f};
        }
        __syncthreads();
        // thread -> (row, 8 consecutive head-dim columns): weights of the wavefronts, their
        // O sum, the normalised row (one combine per thread at 32 rows).
        constexpr int CG = D / 8;  // 8-column groups of a row
        for (int idx = tid; idx < BM * CG; idx += (NW * kWave)) {
            const int row = idx / CG, col = 8 * (idx % CG);
            const int r = r_begin + row;
            if (r >= r_end) continue;
            f32x4 sw[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) sw[w] = stats[w * BM + row];
            float wt[NW], m, lt;
            bool any_masked;
            combine(sw, wt, m, lt, any_masked);
            f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float* ow =
                    reinterpret_cast<const float*>(smem + static_cast<size_t>(w) * S::TILE * sizeof(T)) + row * CP + col;
                lo += *reinterpret_cast<const f32x4*>(ow) * wt[w];
                hi += *reinterpret_cast<const f32x4*>(ow + 4) * wt[w];
            }
            const float inv = lt > 0.f ? 1.f / lt : 0.f;
            write_row(r, col, lo * inv);
            write_row(r, col + 4, hi * inv);
            if (col == 0) write_lse(r, lt > 0.f ? m + log2f(lt) : -INFINITY, !any_masked && MASKED);
        }
    } else {
        __syncthreads();  // every wavefront is done with its tile buffer
        float* comb = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int b = 0; b < NQB; ++b)
            if (g4 == 0) stats[wave * BM + 16 * b + l16] = f32x4{m_run[b], l_run[b], raw[b] ? 1.f : 0.f, 0.f};
        __syncthreads();
        // Each wavefront scales its O by 2^(m_w - m) / l and writes it.
        float row_lse[NQB];
        bool row_raw[NQB];
        float fscale[NQB];
#pragma unroll
        for (int b = 0; b < NQB; ++b) {
            f32x4 sw[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) sw[w] = stats[w * BM + 16 * b + l16];
            float wt[NW], m, lt;
            bool any_masked;
            combine(sw, wt, m, lt, any_masked);
            fscale[b] = lt > 0.f ? wt[wave] / lt : 0.f;
            row_lse[b] = lt > 0.f ? m + log2f(lt) : -INFINITY;
            row_raw[b] = !any_masked && MASKED;
        }
        // Groups of MB row blocks: each wavefront writes its scaled O, then
        // thread -> (row, 4 consecutive head-dim columns) sums the wavefronts.
        constexpr int MB = S::template merge_blocks<T>();
        constexpr int MROWS = 16 * MB;
#pragma unroll
        for (int b0 = 0; b0 < NQB; b0 += MB) {
            if (b0 > 0) __syncthreads();  // the previous group's sums are read
#pragma unroll
            for (int b = b0; b < b0 + MB && b < NQB; ++b) {
#pragma unroll
                for (int d = 0; d < DB; ++d)
                    *reinterpret_cast<f32x4*>(comb + (wave * MROWS + 16 * (b - b0) + l16) * CP + 16 * d + 4 * g4) =
                        o[d][b] * fscale[b];
            }
            __syncthreads();
            for (int idx = tid; idx < MROWS * VPRO; idx += (NW * kWave)) {
                const int row = idx / VPRO, col = 4 * (idx - (idx / VPRO) * VPRO);
                const int r = r_begin + 16 * b0 + row;
                if (16 * b0 + row >= BM || r >= r_end) continue;
                f32x4 acc = *reinterpret_cast<const f32x4*>(comb + row * CP + col);
#pragma unroll
                for (int w = 1; w < NW; ++w) acc += *reinterpret_cast<const f32x4*>(comb + (w * MROWS + row) * CP + col);
                write_row(r, col, acc);
            }
        }
        // Row statistics: the lanes of group 0 of wavefront 0 own rows 16 b + l16.
        if (wave == 0 && g4 == 0) {
#pragma unroll
            for (int b = 0; b < NQB; ++b) {
                const int r = r_begin + 16 * b + l16;
                if (r < r_end) write_lse(r, row_lse[b], row_raw[b]);
            }
        }
    }
}

// Work items: heaviest query tiles first (causal), then (sequence, K/V head), split.  The
// 2 npair shortest causal query tiles of each unit run two to a workgroup (shortest with
// longest of that set, so no pair outlasts the heaviest tile), which keeps the grid within
// one round of resident workgroups.
// The 32-row D = 64 unmasked variant (K and V by DMA, no staging registers) is held to
// four wavefronts per SIMD (128 VGPRs), its row-split form to three (168 VGPRs: at 128 it
// spilled, and a spill reload between a tile's DMA and its fixed vmcnt wait would release
// the wait early; the build checks that no DMA variant spills).
template <typename T, int D, int NQB, int MK, bool RS, int TWIDTH>
constexpr int fwd_waves_per_simd() {
    return fwd_dma<T, D, NQB, MK, RS, TWIDTH>() ? (NQB == 2 ? (RS ? 3 : 4) : 2) : 1;
}

template <typename T, int D, int NQB, int MK, bool RS, int TWIDTH, int NW>
__global__ __launch_bounds__(NW * kWave, (fwd_waves_per_simd<T, D, NQB, MK, RS, TWIDTH>()))
void attn_fwd_kernel(const AttnParams p) {
    int lin = blockIdx.x;
    const int units = p.batch * p.hkv;
    if (p.xcd_map != 0) {
        // XCD-aware order (one split, no pairs): the dispatcher deals workgroups to the
        // eight XCDs in turn, so block b runs on XCD b % 8; each XCD takes its own units,
        // whose K/V then stay in its L2 instead of every XCD streaming every unit.
        const int x = lin & 7, s = lin >> 3;
        int bh, xi;
        if (p.xcd_map == 1 || p.xcd_map == 3) {
            // Unit u on XCD u % 8; within an XCD the query tile rows go heaviest first
            // (mode 3: the units of a row rotated by the row, as the plain varlen order).
            const int nxu = (units - x + 7) >> 3;
            if (nxu <= 0) return;
            const int rank = s / nxu;
            if (rank >= p.nx) return;
            int slot = s - rank * nxu;
            if (p.xcd_map == 3) slot = (slot + rank) % nxu;
            bh = x + 8 * slot;
            xi = p.causal ? p.nx - 1 - rank : rank;
        } else {
            // The unit-major query tiles, one contiguous chunk per XCD.
            const int total = p.nx * units, per = (total + 7) >> 3;
            const int item = x * per + s;
            if (s >= per || item >= total) return;
            bh = item / p.nx;
            const int r = item - bh * p.nx;
            xi = p.causal ? p.nx - 1 - r : r;
        }
        attn_block<T, D, NQB, MK, RS, TWIDTH, NW>(p, 0, bh, xi);
        return;
    }
    const int lsp = fdiv(lin, p.fd_splits);
    const int split = lin - lsp * p.splits;
    lin = lsp;
    if (p.snake > 0) {
        // One resident round: the rank order alternates direction per round of CU count
        // blocks (C1: the most key tiles on one CU 148 -> 121, mean 114).
        const int round = fdiv(lin, p.fd_snake), pos = lin - round * p.snake;
        const int in_round = min(p.snake, p.nx * units - round * p.snake);
        if (round & 1) lin = round * p.snake + (in_round - 1 - pos);
    }
    const int xi = fdiv(lin, p.fd_units);
    // Varlen: the units of a query tile row are rotated by 9 per row.  Workgroups are dealt
    // to XCDs and then shader engines in fixed rotation, so without it the units that have
    // work at a given row (the long sequences of the batch) land on the same engines row
    // after row, fill them, and stall the in-order dispatch while the rest of the chip
    // idles.  Equal-length batches keep each XCD on few units (their K/V stay in its L2).
    const int bu = lin - xi * units + (p.cu_q ? xi * 9 : 0);
    const int bh = bu - fdiv(bu, p.fd_units) * units;
    if (!p.causal) {
        attn_block<T, D, NQB, MK, RS, TWIDTH, NW>(p, split, bh, xi);
        return;
    }
    const int singles = p.nx - 2 * p.npair;
    if (xi < singles) {
        attn_block<T, D, NQB, MK, RS, TWIDTH, NW>(p, split, bh, p.nx - 1 - xi);
        return;
    }
    const int j = xi - singles;
    attn_block<T, D, NQB, MK, RS, TWIDTH, NW>(p, split, bh, 2 * p.npair - 1 - j);
    __syncthreads();  // the second tile reuses the LDS
    attn_block<T, D, NQB, MK, RS, TWIDTH, NW>(p, split, bh, j);
}

// A decode unit's query side: sequence, K/V head, first query position and count, the
// row of its split partials, and its virtual rows (Sq x G, at most 16).
struct DecodeRows {
    int seq, kvh, q0, lq, vrows;
    int64_t row_base;
};

__device__ __forceinline__ DecodeRows decode_rows(const AttnParams& p, const int bh) {
    DecodeRows u;
    u.seq = fdiv(bh, p.fd_hkv);
    u.kvh = bh - u.seq * p.hkv;
    u.q0 = 0;
    u.lq = p.seq_q;
    u.row_base = static_cast<int64_t>(u.seq) * p.seq_q;
    if (p.cu_q) {
        u.q0 = min(max(p.cu_q[u.seq], 0), p.total_q);
        u.lq = min(min(max(p.cu_q[u.seq + 1], u.q0), p.total_q) - u.q0, p.seq_q);
        u.row_base = u.q0;
    }
    u.vrows = min(u.lq * p.group, 16);
    return u;
}

// Decode partials go through device-scope accesses: the stores write through to the level
// that every XCD reads and the loads read from it (past the reader's own L2), so a
// workgroup's partials are visible to the one that merges them with no L2-wide writeback
// or invalidate (an agent-scope fence costs one of each; with thousands of wavefronts
// they serialise into tens of microseconds).  The order: each wavefront waits for its
// stores (vmcnt(0)) before the workgroup barrier, the barrier precedes the count, and the
// merging workgroup loads only after its count returned the final value.
__device__ __forceinline__ void store_dev(float* p, f32x2 v) {
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), __builtin_bit_cast(unsigned long long, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ f32x2 load_dev(const float* p) {
    return __builtin_bit_cast(f32x2, __hip_atomic_load(reinterpret_cast<unsigned long long*>(const_cast<float*>(p)),
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// The 16-byte forms for the partial outputs, through a buffer resource over the whole
// partial array (the plan keeps it under 2^31 bytes) with the cache policy of those
// device-scope accesses (sc1).  An 8-byte store costs a whole write transaction of its own
// (the C3 partials wrote 4.2 MB for 1 MB of data).
constexpr int kDevScope = 16;  // raw buffer cache-policy bits: sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const AttnParams& p) {
    return buffer_rsrc(p.part_o, 0x7fffffffu);
}
__device__ __forceinline__ void store_dev4(__amdgpu_buffer_rsrc_t r, int64_t elem, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, static_cast<uint32_t>(elem * 4), 0,
                                           kDevScope);
}
__device__ __forceinline__ f32x4 load_dev4(__amdgpu_buffer_rsrc_t r, int64_t elem) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<uint32_t>(elem * 4), 0,
                                                                          kDevScope));
}

// Merge of a decode unit's split partials, in split order (deterministic).  Two running
// merges per row: the splits that met a kept key (masked mode) and the raw-score ones;
// a row that met a kept key in some split takes the first, a fully masked row the second
// (the reference's raw-score result for such rows).  Splits whose partial carries no
// weight for a row add nothing to it, so `live` (bit s: split s carries weight for some
// row) only saves the loads of the others.  Thread t of the workgroup takes columns
// 4 (t % (D / 4)) .. + 3 of virtual row t / (D / 4), then the next 256 (row, columns)
// items.  Reference: the split-KV combine of the decode path (device_attention.cpp:836-907).
template <typename T, int D>
__device__ __forceinline__ void decode_merge_unit(const AttnParams& p, const int bh, const uint32_t live) {
    constexpr int C4 = D / 4;
    constexpr int CH = 16;  // splits per round of loads
    const DecodeRows u = decode_rows(p, bh);
    const int items = u.vrows * C4;
    const int64_t split_rows = p.rows_total * p.hq;
    // Splits that are not live load the first live split's record (no per-split branch;
    // their weight is zero).
    const int s_any = live ? __builtin_ctz(live) : 0;
    const auto pr = part_rsrc(p);
    for (int item = threadIdx.x; item < items; item += NTHREADS) {
        const int rr = item / C4;
        const int c = 4 * (item - rr * C4);
        const int pos = fdiv(rr, p.fd_group);
        const int head = u.kvh * p.group + (rr - pos * p.group);
        const int64_t row0 = (u.row_base + pos) * p.hq + head;
        float mk = -INFINITY, sk = 0.f, mr = -INFINITY, sr = 0.f;
        f32x4 ak = f32x4{0.f, 0.f, 0.f, 0.f}, ar = ak;
        for (int s0 = 0; s0 < p.splits; s0 += CH) {
            f32x2 e[CH];
            f32x4 v[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int s = s0 + j;
                const bool use = s < p.splits && ((live >> s) & 1u);
                const int64_t prow = static_cast<int64_t>(use ? s : s_any) * split_rows + row0;
                e[j] = load_dev(p.part_lse + 2 * prow);
                v[j] = load_dev4(pr, prow * D + c);
                if (!use) e[j] = f32x2{-INFINITY, 0.f};
            }
            float ck = mk, cr = mr;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                if (e[j][1] == 0.f) ck = fmaxf(ck, e[j][0]);
                else cr = fmaxf(cr, e[j][0]);
            }
            // Rescale what the earlier rounds added (exactly 0 while nothing was).
            const float fk = ck == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mk - ck);
            const float fr = cr == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mr - cr);
            sk *= fk;
            ak *= fk;
            sr *= fr;
            ar *= fr;
            mk = ck;
            mr = cr;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const bool raw = e[j][1] != 0.f;
                const float m = raw ? mr : mk;
                const float w = e[j][0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(e[j][0] - m);
                if (w != 0.f) {
                    if (raw) {
                        sr += w;
                        ar += w * v[j];
                    } else {
                        sk += w;
                        ak += w * v[j];
                    }
                }
            }
        }
        const bool masked = sk > 0.f;
        const float m = masked ? mk : mr, l = masked ? sk : sr;
        const f32x4 a = masked ? ak : ar;
        const float inv = l > 0.f ? 1.f / l : 0.f;
        if (c < p.dv) {
            const int64_t ob_off = p.cu_q ? 0 : u.seq * p.os[0];
            T* out = static_cast<T*>(p.out) + ob_off + head * p.os[1] + static_cast<int64_t>(u.q0 + pos) * p.os[2] + c;
            typedef __attribute__((__vector_size__(2 * sizeof(T)))) T t2;
            t2 w0, w1;
            w0[0] = static_cast<T>(a[0] * inv);
            w0[1] = static_cast<T>(a[1] * inv);
            w1[0] = static_cast<T>(a[2] * inv);
            w1[1] = static_cast<T>(a[3] * inv);
            *reinterpret_cast<t2*>(out) = w0;
            *reinterpret_cast<t2*>(out + 2) = w1;
        }
        if (p.lse && c == 0) {
            const int64_t lb_off = p.cu_q ? 0 : u.seq * p.ls[0];
            p.lse[lb_off + head * p.ls[1] + static_cast<int64_t>(u.q0 + pos) * p.ls[2]] =
                l > 0.f ? (m + log2f(l)) * kLn2 + (masked ? 0.f : kMaskedLogit) : -INFINITY;
        }
    }
}

// The merge of decode_merge_unit as a launch of its own (one workgroup per unit), for
// calls without split counters.
template <typename T, int D>
__global__ __launch_bounds__(NTHREADS) void attn_decode_merge_kernel(const AttnParams p) {
    decode_merge_unit<T, D>(p, blockIdx.x, 0xffffffffu);
}

// Decode: at most 16 "virtual rows" (Sq x G) per (sequence, K/V head).  The key tiles of a
// unit are dealt round-robin to its wavefronts (wavefront slot s of S takes tiles s, s + S,
// ...): K goes straight from global memory into MFMA A-operand registers, V through a
// per-wavefront LDS tile read transposed, with the next tile's loads in flight during the
// softmax.  With a mask shared by the rows (a padding mask), tiles whose keys are all
// masked are skipped once a kept key among the first 64 proves that no row is fully
// masked (their keys then carry exactly zero weight).  The four wavefronts of a workgroup
// merge their (m, l, O) in LDS; one workgroup per unit writes the output, several write
// fp32 partials that the last of them to finish merges (split counter), or that
// attn_decode_merge_kernel merges in a launch of its own.
template <typename T, int D, int MK>
__global__ __launch_bounds__(NTHREADS) void attn_decode_kernel(const AttnParams p) {
    typedef typename Mfma<T>::v8 v8;
    constexpr int DC = D / 32;
    constexpr int DB = D / 16;
    constexpr int KB = WN / 16;
    typedef Shape<D, 1, WN> S;
    constexpr int VPR = S::VPS;  // staging lanes per V row (lanes past the row idle)
    constexpr int RPP = S::RPP;
    constexpr int KIT = S::KIT;
    constexpr int NCH = S::NCH;
    constexpr int VP = D + 16;
    constexpr int CP = D + 4;
    constexpr bool MASKED = MK != MK_NONE;
    constexpr int SCAN = 8;  // mask loads per lane of the skip scan: up to 2 * SCAN tiles
    typedef typename std::conditional<MK == MK_BOOL, uint8_t,
            typename std::conditional<MK == MK_BF16 || MK == MK_F16, uint16_t, float>::type>::type MRaw;

    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4;
    const int l16 = lane & 15;

    const int wg_per_unit = p.splits;
    const int bh = fdiv(static_cast<int>(blockIdx.x), p.fd_splits);
    const int split = blockIdx.x - bh * wg_per_unit;
    const int nslots = wg_per_unit * NWAVES;
    // Wavefront-major slots: workgroup `split` takes tiles split, split + wg_per_unit, ...
    // across the whole key range, so every workgroup meets the live keys of a padded row
    // (no workgroup of only masked tiles) and the work spreads evenly.
    const int slot = wave * wg_per_unit + split;
    const DecodeRows u = decode_rows(p, bh);
    const int seq = u.seq, kvh = u.kvh, q0 = u.q0, lq = u.lq, vrows = u.vrows;
    const int64_t row_base = u.row_base;
    const int G = p.group;

    int k0 = 0, lk = p.seq_k;
    int64_t qb_off = seq * p.qs[0], kb_off = seq * p.ks[0], vb_off = seq * p.vs[0];
    if (p.cu_q) {
        k0 = min(max(p.cu_k[seq], 0), p.total_k);
        lk = min(min(max(p.cu_k[seq + 1], k0), p.total_k) - k0, p.seq_k);
        qb_off = kb_off = vb_off = 0;
    }
    if (p.klen) lk = min(max(p.klen[seq], 1), p.seq_k);
    // Uniform over the workgroup: an empty sequence leaves before any barrier.  (With
    // split counters every split of such a unit leaves here and none merges: its rows
    // have no output to write.)
    if (vrows <= 0) return;
    const int coff = p.cu_q ? (lk - lq) : 0;
    int kend = max(lk, 0);
    if (p.causal) kend = max(0, min(lk, fdiv(vrows - 1, p.fd_group) + 1 + coff));
    const int ntiles = (kend + WN - 1) / WN;
    const int n_t = slot < ntiles ? (ntiles - 1 - slot) / nslots + 1 : 0;  // this wavefront's tiles

    // This lane's row.
    const bool valid = l16 < vrows;
    const int rr = valid ? l16 : 0;
    const int pos = fdiv(rr, p.fd_group);
    const int head = kvh * G + (rr - pos * G);
    const int lim = p.causal ? min(lk, pos + coff + 1) : lk;
    v8 qf[DC];
    {
        const T* src = static_cast<const T*>(p.q) + qb_off + head * p.qs[1] + static_cast<int64_t>(q0 + pos) * p.qs[2];
        // Lanes past the last row read row 0 (in range) and are never written.
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[c] = head_frag<v8>(src, 32 * c + 8 * g4, p.d);
    }
    int64_t mrow = 0, m_key = 0, m_end = 0;
    bool shared_row = false;
    bool mvec = false;  // see attn_block
    if constexpr (MASKED) {
        const bool packed = p.mask_mode == KMI_MASK_PACKED;
        m_end = packed ? p.mask_numel : INT64_MAX;
        m_key = packed ? 1 : p.ms[3];
        if (packed) {
            const int64_t m_seq = packed_block_offset(p, seq);
            mrow = m_seq + static_cast<int64_t>(pos) * lk;
            mvec = p.mask_vec4 && m_seq + static_cast<int64_t>(lq) * lk <= m_end;
        } else {
            const int64_t m_seq = p.cu_q ? (static_cast<int64_t>(q0) * p.ms[2] + static_cast<int64_t>(k0) * p.ms[3])
                                         : seq * p.ms[0];
            mrow = m_seq + head * p.ms[1] + static_cast<int64_t>(pos) * p.ms[2];
            mvec = p.mask_vec4;
        }
        // Every row of the wavefront reads the same mask row.
        shared_row = (lq == 1 || (!packed && p.ms[2] == 0)) && (G == 1 || packed || p.ms[1] == 0);
    }

    // K fragments of a tile come straight from memory: lane (g4, l16) holds key
    // 16 kb + l16, dims 32 c + 8 g4 .. + 7 -- the A operand of S^T = K Q^T.  Both K and V
    // load through one buffer resource per tile that ends at the unit's last key (rows past
    // it read as zeros).
    const int64_t kstride = p.ks[2] * static_cast<int64_t>(sizeof(T)), vstride = p.vs[2] * static_cast<int64_t>(sizeof(T));
    const char* kunit = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + kb_off + kvh * p.ks[1] +
                                                      static_cast<int64_t>(k0) * p.ks[2]);
    const char* vunit = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + vb_off + kvh * p.vs[1] +
                                                      static_cast<int64_t>(k0) * p.vs[2]);
    const int krow = lane / VPR, dg = lane - (lane / VPR) * VPR;
    const bool stage_lane = dg < NCH;  // staging lanes past the padded row idle
    const int dgc = min(dg, (p.dv - 1) / 8);  // V's chunk (V's columns past dv repeat the last)
    // Padded head dims: K's columns past d are zeroed (as in the prefill kernel); V's
    // reach only output columns past dv, which are never written.  Uniform.
    const bool kpad = p.d < D;
    const uint32_t k_lane = static_cast<uint32_t>(l16 * kstride + 16 * g4);
    const uint32_t v_lane = static_cast<uint32_t>(krow * vstride + 16 * dgc);
    // Resources end with the last row's data (overlapping rows read in full).
    const uint32_t krow_b = static_cast<uint32_t>(p.d * sizeof(T)), vrow_b = static_cast<uint32_t>(p.dv * sizeof(T));
    T* vl = reinterpret_cast<T*>(smem) + wave * WN * VP;

    // One tile's registers: K fragments, the V rows this lane stages, the mask values.
    v8 kreg[KB][DC];
    u32x4 vreg[KIT];
    MRaw mpre[MASKED ? KB : 1][4];
    auto load_tile = [&](int i) {
        const int key0 = (slot + i * nslots) * WN;
        const int rows = min(lk - key0, WN);
        const auto rk = buffer_rsrc(kunit + key0 * kstride, rows_extent(rows, static_cast<uint32_t>(kstride), krow_b));
        const auto rv = buffer_rsrc(vunit + key0 * vstride, rows_extent(rows, static_cast<uint32_t>(vstride), vrow_b));
        uint32_t kst = static_cast<uint32_t>(kstride), vst = static_cast<uint32_t>(vstride);
        __asm__ volatile("" : "+s"(kst), "+s"(vst));
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int c = 0; c < DC; ++c)
                kreg[kb][c] = __builtin_bit_cast(v8, buffer_load16(rk, k_lane + 16 * kb * kst + 64 * c));
        if (kpad) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int c = 0; c < DC; ++c)
                    if (32 * c + 8 * g4 >= p.d) kreg[kb][c] = v8{};
        }
#pragma unroll
        for (int i2 = 0; i2 < KIT; ++i2) vreg[i2] = buffer_load16(rv, v_lane + i2 * RPP * vst);
        if constexpr (MASKED) {
            const MRaw* mp = static_cast<const MRaw*>(p.mask);
            if (mvec && key0 + WN <= lk) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) Mask4<MRaw>::load(mp + mrow + key0 + 16 * kb + 4 * g4, mpre[kb]);
            } else {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int kk = key0 + 16 * kb + 4 * g4 + j;
                        const int64_t mi = mrow + kk * m_key;
                        mpre[kb][j] = (kk < lk && mi < m_end) ? mp[mi] : MRaw{};
                    }
                }
            }
        }
    };

    // Tiles this wavefront runs: bit i of `live` stands for tile slot + i * nslots.
    uint32_t live = 0xffffffffu;
    const bool use_bits = MASKED && shared_row && n_t > 0 && n_t <= 2 * SCAN;
    if constexpr (MASKED) {
        if (use_bits) {
            const MRaw* mp = static_cast<const MRaw*>(p.mask);
            const int lim0 = p.causal ? min(lk, coff + 1) : lk;
            const int pk = lane;
            const MRaw first = mask_load(mp, mrow, pk < lim0 ? pk : -1, lk, m_key, m_end);
            MRaw sv[SCAN];
#pragma unroll
            for (int j = 0; j < SCAN; ++j) {
                const int i = 2 * j + (lane >> 5);
                const int key = (slot + i * nslots) * WN + (lane & 31);
                sv[j] = mask_load(mp, mrow, i < n_t ? key : -1, lk, m_key, m_end);
            }
            const bool proof = __builtin_amdgcn_ballot_w64(pk < lim0 && mask_logit_of<MK>(first) > kMaskedLogit) != 0;
            if (proof) {
                live = 0;
#pragma unroll
                for (int j = 0; j < SCAN; ++j) {
                    const int i = 2 * j + (lane >> 5);
                    const int key = (slot + i * nslots) * WN + (lane & 31);
                    const uint64_t b = __builtin_amdgcn_ballot_w64(i < n_t && key < lk &&
                                                                   mask_logit_of<MK>(sv[j]) > kMaskedLogit);
                    live |= (static_cast<uint32_t>(b) != 0u ? 1u : 0u) << (2 * j);
                    live |= (static_cast<uint32_t>(b >> 32) != 0u ? 1u : 0u) << (2 * j + 1);
                }
            }
        }
    }
    auto next_i = [&](int i) -> int {  // the first tile index after i that runs
        if (!use_bits) return i + 1;
        const uint32_t rest = live & (0xfffffffeu << i);
        return rest ? __builtin_ctz(rest) : n_t;
    };

    f32x4 o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;
    bool raw = MASKED;

    int i = use_bits ? (live ? __builtin_ctz(live) : n_t) : 0;
    if (i < n_t) load_tile(i);
    // A negative scale flips the sign of Q (exact) so that the exponent's multiplier is
    // positive and the row maximum of the raw scores is the maximum logit.
    float c2 = p.scale_log2;
    if (c2 < 0.f) {
        c2 = -c2;
#pragma unroll
        for (int c = 0; c < DC; ++c) qf[c] = __builtin_bit_cast(v8, __builtin_bit_cast(u32x4, qf[c]) ^ 0x80008000u);
    }
    while (i < n_t) {
        // LDS keeps one wavefront's accesses in order (the previous tile's reads, these
        // writes, this tile's reads): only the compiler must keep it.
        __asm__ volatile("" ::: "memory");
        if (stage_lane) {
#pragma unroll
            for (int i2 = 0; i2 < KIT; ++i2) *reinterpret_cast<u32x4*>(vl + (krow + i2 * RPP) * VP + 8 * dg) = vreg[i2];
        }
        MRaw mcur[MASKED ? KB : 1][4];
        if constexpr (MASKED) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) mcur[kb][j] = mpre[kb][j];
        }
        f32x4 sacc[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            sacc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < DC; ++c) sacc[kb] = Mfma<T>::run(kreg[kb][c], qf[c], sacc[kb]);
        }
        // The K fragments are consumed: the next tile's loads overlap the softmax and PV.
        const int key0 = (slot + i * nslots) * WN;
        i = next_i(i);
        if (i < n_t) load_tile(i);
        const int rel = lim - key0 - 4 * g4;
        float x[KB][4];
        float xs = c2;
        if constexpr (MASKED) {
            xs = 1.f;
            bool keep_any = false;
            float xm[KB][4];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool vis = 16 * kb + j < rel;
                    const float val = vis ? sacc[kb][j] * c2 : -INFINITY;
                    float vm = -INFINITY;
                    if (vis) {
                        const float ml = mask_logit_of<MK>(mcur[kb][j]);
                        if (ml > kMaskedLogit) {
                            vm = val + kLog2e * ml;
                            keep_any = true;
                        }
                    }
                    x[kb][j] = val;
                    xm[kb][j] = vm;
                }
            }
            // Raw scores until the row's first kept key (the reference's fully-masked-row
            // result), then masked keys get exactly zero weight.
            if (raw && row_any4(keep_any, l16)) {
                raw = false;
                m_run = -INFINITY;
                l_run = 0.f;
#pragma unroll
                for (int d = 0; d < DB; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            if (!raw) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) x[kb][j] = xm[kb][j];
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) x[kb][j] = 16 * kb + j < rel ? sacc[kb][j] : -INFINITY;
        }
        float mt = fmaxf(fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3])),
                         fmaxf(fmaxf(x[1][0], x[1][1]), fmaxf(x[1][2], x[1][3])));
        mt = row_max4(mt) * xs;
        const bool move = mt > m_run + kLazy;
        float alpha = 1.f;
        if (move) {
            alpha = __builtin_amdgcn_exp2f(m_run - mt);
            m_run = mt;
        }
        const float neg_m = m_run == -INFINITY ? 0.f : -m_run;
        if (__builtin_amdgcn_ballot_w64(move)) {
            l_run *= alpha;
#pragma unroll
            for (int d = 0; d < DB; ++d) o[d] *= alpha;
        }
        v8 pf;
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kb][j], xs, neg_m));
                ls += e;
                pf[4 * kb + j] = static_cast<T>(e);
            }
        }
        l_run += ls;
        v8 vf[DB];
        {
            const T* vsrc = vl + (4 * g4 + (l16 >> 2)) * VP + 4 * (l16 & 3);
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const u32x2 lo = lds_read_tr(vsrc + 16 * d);
                const u32x2 hi = lds_read_tr(vsrc + 16 * VP + 16 * d);
                vf[d] = __builtin_bit_cast(v8, u32x4{lo[0], lo[1], hi[0], hi[1]});
            }
        }
#pragma unroll
        for (int d = 0; d < DB; ++d) o[d] = Mfma<T>::run(vf[d], pf, o[d]);
    }

    // Merge of the four wavefronts in LDS (their V tiles are done with after the barrier):
    // lane (g4, l16) holds dims 16 d + 4 g4 .. + 3 of row l16.
    const float l = row_sum4(l_run);
    __syncthreads();
    float* comb = reinterpret_cast<float*>(smem);
    float* st = comb + NWAVES * 16 * CP;
#pragma unroll
    for (int d = 0; d < DB; ++d) *reinterpret_cast<f32x4*>(comb + (wave * 16 + l16) * CP + 16 * d + 4 * g4) = o[d];
    if (g4 == 0) {
        st[(wave * 16 + l16) * 3] = m_run;
        st[(wave * 16 + l16) * 3 + 1] = l;
        st[(wave * 16 + l16) * 3 + 2] = raw ? 1.f : 0.f;
    }
    __syncthreads();
    // Wavefront w combines dims [w D / 4, (w + 1) D / 4) of the 16 rows: lane (g4, l16)
    // takes D / 16 of them for row l16.  Rows that met a kept key in some wavefront merge
    // those wavefronts only; the others merge every wavefront's raw-score statistics.
    float mw[NWAVES], lw[NWAVES];
    bool sel_masked = false;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
        mw[w] = st[(w * 16 + l16) * 3];
        lw[w] = st[(w * 16 + l16) * 3 + 1];
        if (st[(w * 16 + l16) * 3 + 2] == 0.f && lw[w] > 0.f) sel_masked = true;
    }
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
        const bool sel = lw[w] > 0.f && ((st[(w * 16 + l16) * 3 + 2] == 0.f) == sel_masked);
        if (!sel) lw[w] = 0.f;
        if (sel) M = fmaxf(M, mw[w]);
    }
    float L = 0.f, wt[NWAVES];
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
        wt[w] = lw[w] > 0.f ? __builtin_amdgcn_exp2f(mw[w] - M) : 0.f;
        L += wt[w] * lw[w];
    }
    // PER (= D / 16, even) columns per lane, in pairs; pairs past the head dim are skipped.
    constexpr int PER = D / 16;
    const int c0 = wave * (D / 4) + g4 * PER;
    float acc[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) acc[j] = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
#pragma unroll
        for (int j = 0; j < PER; j += 2) {
            const f32x2 v = *reinterpret_cast<const f32x2*>(comb + (w * 16 + l16) * CP + c0 + j);
            acc[j] += wt[w] * v[0];
            acc[j + 1] += wt[w] * v[1];
        }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (p.splits == 1) {
        if (!valid) return;
        // One workgroup per unit: the merged rows are the output.
        const int64_t ob_off = p.cu_q ? 0 : seq * p.os[0];
        T* out = static_cast<T*>(p.out) + ob_off + head * p.os[1] + static_cast<int64_t>(q0 + pos) * p.os[2] + c0;
#pragma unroll
        for (int j = 0; j < PER; j += 2) {
            typedef __attribute__((__vector_size__(2 * sizeof(T)))) T t2;
            t2 w2;
            w2[0] = static_cast<T>(acc[j] * inv);
            w2[1] = static_cast<T>(acc[j + 1] * inv);
            if (c0 + j < p.dv) *reinterpret_cast<t2*>(out + j) = w2;
        }
        if (p.lse && wave == 0 && g4 == 0) {
            const int64_t lb_off = p.cu_q ? 0 : seq * p.ls[0];
            p.lse[lb_off + head * p.ls[1] + static_cast<int64_t>(q0 + pos) * p.ls[2]] =
                L > 0.f ? (M + log2f(L)) * kLn2 + ((MASKED && !sel_masked) ? kMaskedLogit : 0.f) : -INFINITY;
        }
        return;
    }
    if (valid) {
        const int64_t prow = (static_cast<int64_t>(split) * p.rows_total + row_base + pos) * p.hq + head;
        const auto pr = part_rsrc(p);
#pragma unroll
        for (int j = 0; j < PER; j += (PER % 4 == 0 ? 4 : 2)) {
            if (c0 + j >= p.dv) continue;  // dv is a multiple of 8: a chunk is in or out
            if constexpr (PER % 4 == 0) {
                store_dev4(pr, prow * D + c0 + j, f32x4{acc[j] * inv, acc[j + 1] * inv, acc[j + 2] * inv, acc[j + 3] * inv});
            } else {
                store_dev(p.part_o + prow * D + c0 + j, f32x2{acc[j] * inv, acc[j + 1] * inv});
            }
        }
        if (wave == 0 && g4 == 0)
            store_dev(p.part_lse + 2 * prow,
                      f32x2{L > 0.f ? M + log2f(L) : -INFINITY, (MASKED && !sel_masked) ? 1.f : 0.f});
    }
    if (!p.ctr) return;
    // Split counter: the workgroup that completes the count merges every split's partials
    // and clears the word for the next call.
    const bool carries = __builtin_amdgcn_ballot_w64(valid && L > 0.f) != 0;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's partials are stored
    __syncthreads();  // ... and every wavefront's; the LDS is free
    uint32_t* flag = reinterpret_cast<uint32_t*>(smem);
    if (threadIdx.x == 0) {
        const unsigned long long add = (1ull << 32) | (carries ? 1ull << split : 0ull);
        const unsigned long long now =
            __hip_atomic_fetch_add(p.ctr + bh, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
        const bool last = static_cast<int>(now >> 32) == wg_per_unit;
        if (last) __hip_atomic_store(p.ctr + bh, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag[0] = last ? 1u : 0u;
        flag[1] = static_cast<uint32_t>(now);
    }
    __syncthreads();
    if (!flag[0]) return;
    decode_merge_unit<T, D>(p, bh, flag[1]);
}

// Merge of split-KV partials: one wavefront per (query row, head); lanes over splits for
// the statistics, over head-dim columns for O (every split's loads independent).
// Splits in masked mode (they met a kept key) win; a row with no kept key in any split
// merges the raw-score partials of every split.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (item >= p.rows_total * p.hq) return;
    const int64_t row = item / p.hq;
    const int h = static_cast<int>(item % p.hq);
    const int64_t stride = p.rows_total * p.hq;
    // Lane l holds columns l + 64 j (reads clamped to the head dim, writes past it skipped).
    constexpr int PER = (D + 63) / 64;
    int colc[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) colc[j] = min(lane + 64 * j, p.dv - 1);
    float acc[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) acc[j] = 0.f;
    float m = -INFINITY, wsum = 0.f;
    bool any_masked = false;  // some split met a kept key: raw-score partials drop out
    if (p.splits <= 32) {
        // Every split's statistics (lane s) and O values in one round of loads.
        // Lanes past the last split read the last split's record (one round of loads, no
        // per-lane branch) and drop it.
        const float* e = p.part_lse + 2 * (min(lane, p.splits - 1) * stride + item);
        const float e0 = e[0], e1 = e[1];
        float lse = lane < p.splits ? e0 : -INFINITY;
        const float flag = lane < p.splits ? e1 : 1.f;
        float v[32][PER];
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float* src = p.part_o + (min(k, p.splits - 1) * stride + item) * D;
#pragma unroll
            for (int j = 0; j < PER; ++j) v[k][j] = src[colc[j]];
        }
        any_masked = __builtin_amdgcn_ballot_w64(lane < p.splits && flag == 0.f && lse != -INFINITY) != 0;
        if (any_masked && flag != 0.f) lse = -INFINITY;
        m = wave_max(lse);
        const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(lse - m);
        wsum = wave_sum(w);
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float wl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), k));
            const float wk = k < p.splits ? wl : 0.f;
#pragma unroll
            for (int j = 0; j < PER; ++j) acc[j] += wk * v[k][j];
        }
    } else {
    // Splits go 64 at a time: lane s holds split s0 + s's statistics (read once).
    for (int s0 = 0; s0 < p.splits; s0 += kWave) {
        const int s = s0 + lane;
        if (s < p.splits) {
            const float* e = p.part_lse + 2 * (s * stride + item);
            if (e[1] == 0.f && e[0] != -INFINITY) any_masked = true;
        }
    }
    any_masked = __builtin_amdgcn_ballot_w64(any_masked) != 0;
    for (int s0 = 0; s0 < p.splits; s0 += kWave) {
        const int s = s0 + lane;
        float lse = -INFINITY;
        if (s < p.splits) {
            const float* e = p.part_lse + 2 * (s * stride + item);
            if (!any_masked || e[1] == 0.f) lse = e[0];
        }
        const float m_chunk = wave_max(lse);
        const float m_new = fmaxf(m, m_chunk);
        if (m_new == -INFINITY) continue;
        const float rescale = __builtin_amdgcn_exp2f(m - m_new);  // 0 while m was -inf
        wsum *= rescale;
#pragma unroll
        for (int j = 0; j < PER; ++j) acc[j] *= rescale;
        m = m_new;
        const float w = __builtin_amdgcn_exp2f(lse - m);
        wsum += wave_sum(w);
        const int n = min(kWave, p.splits - s0);
        // Eight splits' O rows in flight at a time.
        for (int k0 = 0; k0 < n; k0 += 8) {
            float v[8][PER];
            float wk[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int k = min(k0 + u, n - 1);
                wk[u] = k0 + u < n ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), k)) : 0.f;
                const float* src = p.part_o + ((s0 + k) * stride + item) * D;
#pragma unroll
                for (int j = 0; j < PER; ++j) v[u][j] = src[colc[j]];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
#pragma unroll
                for (int j = 0; j < PER; ++j) acc[j] += wk[u] * v[u][j];
            }
        }
    }
    }
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
    int seq = 0, posn = static_cast<int>(row);
    int64_t ob_off = 0, lb_off = 0;
    if (!p.cu_q) {
        seq = static_cast<int>(row / p.seq_q);
        posn = static_cast<int>(row % p.seq_q);
        ob_off = seq * p.os[0];
        lb_off = seq * p.ls[0];
    }
    T* dst = static_cast<T*>(p.out) + ob_off + h * p.os[1] + static_cast<int64_t>(posn) * p.os[2];
#pragma unroll
    for (int j = 0; j < PER; ++j)
        if (lane + 64 * j < p.dv) dst[lane + 64 * j] = static_cast<T>(acc[j] * inv);
    if (p.lse && lane == 0)
        p.lse[lb_off + h * p.ls[1] + static_cast<int64_t>(posn) * p.ls[2]] =
            wsum > 0.f ? (m + log2f(wsum)) * kLn2 + (any_masked ? 0.f : kMaskedLogit) : -INFINITY;
}

// KMI_ATTN_XCD_MAP (read once): 0 keeps the plain workgroup order everywhere; 1 and 3 also
// order dense causal grids by XCD (1 without the per-row unit rotation); unset: by XCD for
// non-causal dense grids (mode 2) and varlen grids (mode 3).
inline int xcd_map_mode() {
    static const int v = [] {
        const char* e = std::getenv("KMI_ATTN_XCD_MAP");
        return e ? std::atoi(e) : 2;
    }();
    return v;
}

template <typename T, int D, int NQB, int MK, bool RS = false, int TWIDTH = WN, int NW = NWAVES>
hipError_t launch_fwd(const AttnParams& p_in, int64_t grid, hipStream_t stream) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    static int per_cu = 0;  // resident workgroups per CU
    typedef Shape<D, NQB, TWIDTH, NW, fwd_dma<T, D, NQB, MK, RS, TWIDTH>()> S;
    // Shared row split: every key tile of a unit (at most four) in LDS, K then V.
    constexpr size_t rs_max = RS ? kRsTiles * TWIDTH * static_cast<size_t>(S::KP + S::VP) * sizeof(T) : 0;
    const size_t lds_tiles = S::template lds_bytes<T>();
    const size_t lds = RS && p_in.rs_shared
                           ? ceil_div(p_in.seq_k, TWIDTH) * TWIDTH * static_cast<size_t>(S::KP + S::VP) * sizeof(T)
                           : lds_tiles;
    const void* fn = reinterpret_cast<const void*>(&attn_fwd_kernel<T, D, NQB, MK, RS, TWIDTH, NW>);
    std::call_once(once, [&] {
        attr_err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(std::max(lds_tiles, rs_max)));
        if (attr_err == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, (NW * kWave), lds_tiles) != hipSuccess)
            per_cu = 0;
    });
    if (attr_err != hipSuccess) return attr_err;
    AttnParams p = p_in;
    p.npair = 0;
    // Causal grids up to twice the resident workgroups pair their shortest query tiles so
    // that every workgroup starts at once (larger grids balance over their many rounds).
    const int64_t units = static_cast<int64_t>(p.batch) * p.hkv;
    const int64_t slots = static_cast<int64_t>(per_cu) * cu_count();
    if (p.causal && p.splits == 1 && slots > 0 && grid > slots && grid <= 2 * slots) {
        const int64_t extra = grid - slots;
        p.npair = static_cast<int>(std::min<int64_t>(ceil_div(extra, units), p.nx / 2));
        grid -= static_cast<int64_t>(p.npair) * units;
    }
    // XCD-aware order for grids whose units' K/V exceed an XCD's 4 MB L2.  Non-causal dense
    // grids: each XCD takes a contiguous chunk of the unit-major query tiles (C5 self: 149
    // -> 47 MB of L2 misses for 42 MB of data, 140 -> 136 us).  Varlen grids: unit u on XCD
    // u % 8, query tile rows heaviest first with each row's units rotated by the row (C4:
    // 61 -> 54 us, masked 127 -> 114 us; without the rotation 71 and 153 us, the in-order
    // dispatch then meets the same few units' work row after row).  Dense causal grids keep
    // the plain (snake) order unless KMI_ATTN_XCD_MAP asks.
    p.xcd_map = 0;
    p.snake = 0;
    if (p.causal && !p.cu_q && p.splits == 1 && p.npair == 0 && slots > 0 && grid <= slots) p.snake = cu_count();
    p.fd_snake = fast_div(static_cast<uint32_t>(p.snake));
    const int64_t kv_bytes = units * static_cast<int64_t>(p.seq_k) * (p.d + p.dv) * static_cast<int64_t>(sizeof(T));
    if (!RS && p.splits == 1 && p.npair == 0 && kv_bytes > (int64_t{4} << 20) && xcd_map_mode() != 0) {
        if (p.cu_q || p.causal) {
            const int mode = xcd_map_mode() == 2 ? (p.cu_q ? 3 : 0) : xcd_map_mode();
            if (units >= 8 && (mode == 1 || mode == 3)) {
                p.xcd_map = mode;
                p.snake = 0;
                grid = 8 * ceil_div(units, 8) * static_cast<int64_t>(p.nx);
            }
        } else {
            p.xcd_map = 2;
            grid = 8 * ceil_div(static_cast<int64_t>(p.nx) * units, 8);
        }
    }
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, NQB, MK, RS, TWIDTH, NW>), dim3(static_cast<unsigned>(grid)), dim3((NW * kWave)), lds,
                       stream, p);
    return hipGetLastError();
}

template <typename T, int D, int NQB>
hipError_t launch_mask(const AttnParams& p, int64_t grid, hipStream_t stream) {
    if (p.mask_mode == KMI_MASK_NONE) return launch_fwd<T, D, NQB, MK_NONE>(p, grid, stream);
    switch (p.mask_dtype) {
        case KMI_BOOL: return launch_fwd<T, D, NQB, MK_BOOL>(p, grid, stream);
        case KMI_BF16: return launch_fwd<T, D, NQB, MK_BF16>(p, grid, stream);
        case KMI_F16: return launch_fwd<T, D, NQB, MK_F16>(p, grid, stream);
        default: return launch_fwd<T, D, NQB, MK_F32>(p, grid, stream);
    }
}

template <typename T, int D, int MK>
hipError_t launch_decode(const AttnParams& p, hipStream_t stream) {
    const int64_t grid = static_cast<int64_t>(p.batch) * p.hkv * p.splits;
    const size_t tiles = static_cast<size_t>(NWAVES) * WN * (D + 16) * sizeof(T);
    const size_t comb = static_cast<size_t>(NWAVES) * 16 * (D + 4) * sizeof(float);
    const size_t lds = std::max(tiles, comb) + static_cast<size_t>(NWAVES) * 16 * 3 * sizeof(float);
    // Wide heads need more than the default 64 KiB of dynamic LDS.
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [&] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_decode_kernel<T, D, MK>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    });
    if (attr_err != hipSuccess) return attr_err;
    hipLaunchKernelGGL((attn_decode_kernel<T, D, MK>), dim3(static_cast<unsigned>(grid)), dim3(NTHREADS), lds, stream,
                       p);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_decode_mask(const AttnParams& p, hipStream_t stream) {
    if (p.mask_mode == KMI_MASK_NONE) return launch_decode<T, D, MK_NONE>(p, stream);
    switch (p.mask_dtype) {
        case KMI_BOOL: return launch_decode<T, D, MK_BOOL>(p, stream);
        case KMI_BF16: return launch_decode<T, D, MK_BF16>(p, stream);
        case KMI_F16: return launch_decode<T, D, MK_F16>(p, stream);
        default: return launch_decode<T, D, MK_F32>(p, stream);
    }
}

template <typename T, int D>
hipError_t launch_all(const AttnParams& p, const Plan& pl, hipStream_t stream) {
    const int64_t grid = static_cast<int64_t>(pl.nx) * p.batch * p.hkv * pl.splits;
    hipError_t err;
    // Variants: 64-row workgroups (and K straight into registers) at D = 64, 32-row ones up
    // to D = 128, 16-row ones everywhere; row split up to D = 128 (the plan keeps to these).
    if (pl.decode) {
        err = launch_decode_mask<T, D>(p, stream);
    } else if (pl.rs) {
        if constexpr (D <= 128) {
            if (pl.nqb == 4 && D == 64) {
                err = launch_fwd<T, D, 4, MK_NONE, true>(p, grid, stream);
            } else if (pl.nqb == 2) {
                err = launch_fwd<T, D, 2, MK_NONE, true>(p, grid, stream);
            } else {
                err = launch_fwd<T, D, 1, MK_NONE, true>(p, grid, stream);
            }
        } else {
            err = hipErrorInvalidValue;  // not planned
        }
    } else if (D == 64 && pl.nqb == 4) {
        // 64-row workgroups are planned for unmasked calls only.
        err = p.mask_mode == KMI_MASK_NONE ? launch_fwd<T, D, (D == 64 ? 4 : 1), MK_NONE>(p, grid, stream)
                                           : hipErrorInvalidValue;
    } else if (D <= 128 && pl.nqb >= 2) {
        err = launch_mask<T, D, (D <= 128 ? 2 : 1)>(p, grid, stream);
    } else {
        err = launch_mask<T, D, 1>(p, grid, stream);
    }
    if (err != hipSuccess || pl.splits <= 1) return err;
    if (pl.decode) {
        if (p.ctr) return hipSuccess;  // merged by the last workgroup of each unit
        hipLaunchKernelGGL((attn_decode_merge_kernel<T, D>), dim3(static_cast<unsigned>(p.batch * p.hkv)),
                           dim3(NTHREADS), 0, stream, p);
        return hipGetLastError();
    }
    const int64_t items = p.rows_total * p.hq;
    hipLaunchKernelGGL((attn_merge_kernel<T, D>), dim3(static_cast<unsigned>(ceil_div(items, 4))), dim3(256), 0,
                       stream, p);
    return hipGetLastError();
}

}  // namespace fwd
}  // namespace kmi
