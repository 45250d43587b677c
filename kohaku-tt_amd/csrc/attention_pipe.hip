// Attention forward for head dim 64, unmasked dense causal calls (top-left): the prefill
// shape of BASELINE config 1 (causal GQA 1x14/2x2048x64), the headline row.
//
// What it computes is what attn_fwd_kernel computes for these calls (attention_kernels.hpp:
// logits scale * q.k in base 2, online softmax with a lazy rescale, P rounded to the
// operand type, O and l in fp32, O / l rounded once; reference aten_attention.cpp:389-713
// and ktt_flash/compute.cpp:193-500).  Layout: a 256-thread workgroup (four wavefronts)
// owns 32 "virtual rows" of one (sequence, K/V head): row r is query position r / G of
// query head kvh * G + r % G (GQA heads share every K/V tile).  The four wavefronts hold
// the same rows and split the key range; their online-softmax states merge once in LDS,
// in a fixed order (deterministic).  Where it differs from attn_fwd_kernel:
//   - a wavefront's key tiles are a contiguous run of full tiles (no per-element mask)
//     then at most a few edge tiles (the causal diagonal, the key tail); the tiles with
//     most keys' worth of work go to the wavefronts with fewer;
//   - K / V tiles arrive by LDS DMA through one buffer resource per operand and unit,
//     the tile's offset in the scalar offset (one scalar multiply per operand and one M0
//     write per instruction a step; the per-tile resource of attn_fwd_kernel took about
//     fifty scalar instructions), with one s_waitcnt vmcnt(0) per step (correct whatever
//     else is in flight);
//   - the first tile sets the row reference points from its own maxima and starts O and
//     l from its products (no zero fill, no first-tile rescale of zeros);
//   - 128 VGPRs, four wavefronts per SIMD, no spills.
// Two variants stay selectable for measurement (KMI_ATTN_PIPE_NW, KMI_ATTN_PIPE_MODE): a
// software-pipelined step (the next tile's S MFMAs interleaved with this tile's softmax;
// ~150 VGPRs, three wavefronts per SIMD) and eight-wavefront workgroups that give the
// heaviest causal tiles eight wavefronts and pair the rest heaviest-with-lightest.  On
// gfx950 MFMA and FMA issue overlap almost fully and MFMA and exp by about 60%, yet both
// measured slower on C1 (the table above launch_pipe_c).
#include <algorithm>
#include <mutex>

#include "attention_kernels.hpp"

namespace kmi {
namespace fwd {
namespace {

constexpr int PD = 64;         // head dim
constexpr int PT = 32;         // keys per tile
constexpr int PB = 32;         // rows per query tile
constexpr int PKT = PT * PD;   // elements of one K or V tile (4 KiB in 16-bit)
constexpr int PCP = PD;        // merge row pitch (floats; the chunks are XOR-swizzled per row)
// Per-wavefront LDS: its K tile and V tile, which its O (32 x 64 floats) later overlays.
constexpr int PWAVE_BYTES = std::max<int>(2 * PKT * 2, PB * PCP * 4);
template <int NW>
constexpr size_t pipe_lds_bytes() { return static_cast<size_t>(NW) * (PWAVE_BYTES + PB * 8); }

// Maximum of a lane's eight scores of one row block, shaped for three v_max3_f32 and one
// v_max_f32 (the kernels never see NaN scores).
__device__ __forceinline__ float lane_max8(const f32x4& a, const f32x4& b) {
    const float t0 = fmaxf(fmaxf(a[0], a[1]), a[2]);
    const float t1 = fmaxf(fmaxf(a[3], b[0]), b[1]);
    return fmaxf(fmaxf(fmaxf(t0, t1), b[2]), b[3]);
}

// Key tiles of query tile xt of a unit: (ntiles, nfull); [0, nfull) are visible to every
// row (no mask), [nfull, ntiles) need the per-element causal / key-tail test.
template <bool CAUSAL>
__device__ __forceinline__ int2 tile_keys(const AttnParams& p, int xt) {
    const int vrows = p.seq_q * p.group;
    const int r_begin = xt * PB;
    const int r_end = min(vrows, r_begin + PB);
    const int lk = p.seq_k;
    const int kend = CAUSAL ? min(lk, fdiv(r_end - 1, p.fd_group) + 1) : lk;
    const int lim_min = CAUSAL ? min(lk, fdiv(r_begin, p.fd_group) + 1) : lk;
    return int2{(kend + PT - 1) / PT, lim_min / PT};
}

// One wavefront's share of query tile xt of unit bh: wavefront wv of the nw that split
// the tile's key range.  Leaves its O in its LDS area (16-byte chunk c of row r at chunk
// c ^ (r & 15)) and (m, l) per row in `stats`.
//
// PIPE: the MFMAs of the next key tile (S = K Q^T) are issued interleaved with the
// softmax of the current one (two score register sets, ~150 VGPRs); otherwise a step
// issues its own S MFMAs, reads V^T meanwhile, then runs the softmax and the PV MFMAs
// (fits 128 VGPRs: four wavefronts per SIMD).  Either way the PV MFMAs of row block 0
// interleave with the exponentials of row block 1.
template <typename T, bool CAUSAL, bool PIPE, int NWC>
__device__ __forceinline__ void pipe_tile(const AttnParams& p, const int bh, const int xt, const int wv, const int nw_rt,
                                          unsigned char* const wbase, float* const stats) {
    const int nw = NWC > 0 ? NWC : nw_rt;  // wavefronts sharing the tile (a constant where known)
    typedef typename Mfma<T>::v8 v8;
    const int lane = threadIdx.x & 63;
    const int g4 = lane >> 4;
    const int l16 = lane & 15;

    const int seq = fdiv(bh, p.fd_hkv);
    const int kvh = bh - seq * p.hkv;
    const int G = p.group;
    const int lk = p.seq_k;
    const int vrows = p.seq_q * G;
    const int r_begin = xt * PB;
    const int r_end = min(vrows, r_begin + PB);

    const int2 tk = tile_keys<CAUSAL>(p, xt);
    const int ntiles = __builtin_amdgcn_readfirstlane(tk.x), nfull = __builtin_amdgcn_readfirstlane(tk.y);
    // Full tiles in contiguous runs (the first rem wavefronts one more); edge tile e goes
    // to wavefront (rem + e) % nw, one of those with one fewer.  Wavefront-uniform.
    const int base = __builtin_amdgcn_readfirstlane(nfull / nw), rem = nfull - base * nw;
    const int fa = wv * base + min(wv, rem);
    const int nf_w = base + (wv < rem ? 1 : 0);
    const int ne = ntiles - nfull;
    const int e0 = wv >= rem ? wv - rem : wv - rem + nw;
    const int ne_w = __builtin_amdgcn_readfirstlane(e0 < ne ? (ne - e0 + nw - 1) / nw : 0);
    const int nt_w = nf_w + ne_w;
    auto tile_of = [&](int j) { return j < nf_w ? fa + j : nfull + e0 + nw * (j - nf_w); };

    // Q fragments (B operand of S^T = K Q^T): lane (g4, l16) holds dims 32 c + 8 g4 .. + 7
    // of row 16 b + l16.  Rows past the end read row r_begin and are never written.
    const T* qp = static_cast<const T*>(p.q);
    v8 qf[2][2];
    // Keys [0, lim) are visible to row block b's row of this lane (recomputed where edge
    // tiles need it, so that nothing is held across the loop for it).
    auto row_lim = [&](int b) {
        const int r = r_begin + 16 * b + l16;
        const int rr = r < r_end ? r : r_begin;
        return CAUSAL ? min(lk, fdiv(rr, p.fd_group) + 1) : lk;
    };
    // Issued after the first tile's K / V loads (which need only scalar set-up and two
    // lane offsets), so that those go out first.
    auto load_q = [&] {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int r = r_begin + 16 * b + l16;
            const int rr = r < r_end ? r : r_begin;
            const int pos = fdiv(rr, p.fd_group);
            const int head = kvh * G + (rr - pos * G);
            const T* src = qp + seq * p.qs[0] + head * p.qs[1] + static_cast<int64_t>(pos) * p.qs[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) qf[b][c] = *reinterpret_cast<const v8*>(src + 32 * c + 8 * g4);
        }
    };

    // K / V tiles by LDS DMA (buffer loads with the lds modifier), 16-byte chunks
    // XOR-swizzled per row so that K's fragment reads and V's transposed reads hit
    // distinct banks: K chunk c of row r at c ^ kswz(r), V at c ^ vswz(r).  One buffer
    // resource per operand spans the unit's keys (the host bounds seq_k * stride below
    // 2^31 bytes); DMA instruction i of a tile fills rows 8 i .. 8 i + 7 (lane q: row
    // 8 i + q / 8, physical chunk q % 8) from per-lane offsets fixed for the call, and
    // the tile's own offset rides in the scalar offset: a step's loads cost one scalar
    // multiply per operand and one M0 write per instruction.
    auto kswz = [](int r) { return (r & 7) ^ ((r >> 3) & 1); };
    auto vswz = [](int r) { return 2 * ((r ^ (r >> 2)) & 3); };
    const uint32_t kstride = static_cast<uint32_t>(p.ks[2] * static_cast<int64_t>(sizeof(T)));
    const uint32_t vstride = static_cast<uint32_t>(p.vs[2] * static_cast<int64_t>(sizeof(T)));
    const char* kunit = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + seq * p.ks[0] + kvh * p.ks[1]);
    const char* vunit = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + seq * p.vs[0] + kvh * p.vs[1]);
    // A resource's range ends with the unit's last key row, so the rows of a partial last
    // tile past it read as zeros (their keys are masked on edge tiles and their P is 0);
    // a zero row stride repeats one row.
    const uint32_t row_bytes = PD * static_cast<uint32_t>(sizeof(T));
    const auto krs = buffer_rsrc(kunit, rows_extent(lk, kstride, row_bytes));
    const auto vrs = buffer_rsrc(vunit, rows_extent(lk, vstride, row_bytes));
    // Lane offsets of DMA instruction i depend on the parity of i only (the swizzles of rows
    // 8 i + a do); the row term 8 i * stride is added to the scalar offset.
    uint32_t dko[2], dvo[2];
    {
        const int a = lane >> 3, q7 = lane & 7;
#pragma unroll
        for (int par = 0; par < 2; ++par) {
            dko[par] = static_cast<uint32_t>(a) * kstride + 16u * static_cast<uint32_t>(q7 ^ kswz(8 * par + a));
            dvo[par] = static_cast<uint32_t>(a) * vstride + 16u * static_cast<uint32_t>(q7 ^ vswz(8 * par + a));
        }
    }
    T* const kl = reinterpret_cast<T*>(wbase);
    T* const vl = kl + PKT;
    // K fragment offsets: chunk 4 c + g4 of row l16 (the second is the first with bit 5 of
    // the element offset flipped: (4 + g4) ^ k = 4 ^ (g4 ^ k) for g4 < 4).
    const int kfo0 = l16 * PD + 8 * (g4 ^ kswz(l16));
    int vtro[4];
    {
        const int r = 4 * g4 + (l16 >> 2);
#pragma unroll
        for (int d = 0; d < 4; ++d) vtro[d] = r * PD + 8 * (((2 * d) ^ vswz(r)) | ((l16 >> 1) & 1)) + 4 * (l16 & 1);
    }
    // One operand of tile tt into its LDS tile.  Full tiles carry their row offsets in the
    // scalar offset.  The last, partial tile carries them in the lane offset, to which the
    // hardware's range check applies: its rows past the last key read as zeros (those keys
    // are masked and their P is 0).
    auto dma = [&](int tt, bool V) {
        const uint32_t stride = V ? vstride : kstride;
        const auto rs = V ? vrs : krs;
        T* const dst = V ? vl : kl;
        const int soff = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(tt * PT) * stride));
        if ((tt + 1) * PT <= lk) {
#pragma unroll
            for (int i = 0; i < PT / 8; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + i * 512), 16,
                                                         V ? dvo[i & 1] : dko[i & 1], soff + static_cast<int>(8 * i * stride),
                                                         0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < PT / 8; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void*)(dst + i * 512), 16,
                    (V ? dvo[i & 1] : dko[i & 1]) + static_cast<uint32_t>(soff) + 8u * i * stride, 0, 0, 0);
        }
    };

    // Running state: O^T accumulators, row sums as MFMA columns (P times a column of
    // ones), the reference point m (base-2 logit units), its lazy-rescale threshold m + 8
    // and -m.  The scale multiplies the raw scores inside the exponent's FMA.
    f32x4 o[4][2];
    f32x4 lacc[2];
    float m_run[2], m_thr[2], neg_m[2];  // m_thr: the threshold in raw-score units
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        m_run[b] = -INFINITY;
        m_thr[b] = -INFINITY;
        neg_m[b] = 0.f;
        if constexpr (PIPE) {
            lacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < 4; ++d) o[d][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    float c2 = p.scale_log2;
    // A negative scale flips Q's sign (exact), so the multiplier is positive and a larger
    // score is a larger logit.  Applied once the first tile's loads are out: the test waits
    // for the scale's scalar load, which then overlaps their flight.
    // The lazy-rescale margin in raw-score units (a hardware reciprocal: any margin near
    // kLazy / c2 keeps the exponents bounded).
    float lazy_raw = 0.f;
    auto fix_sign = [&] {
        if (c2 < 0.f) {
            c2 = -c2;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int c = 0; c < 2; ++c) qf[b][c] = __builtin_bit_cast(v8, __builtin_bit_cast(u32x4, qf[b][c]) ^ 0x80008000u);
        }
        lazy_raw = kLazy * __builtin_amdgcn_rcpf(c2);
    };

    auto read_k = [&](v8 (&kf)[2][2]) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int c = 0; c < 2; ++c) kf[kb][c] = *reinterpret_cast<const v8*>(kl + 16 * kb * PD + (kfo0 ^ (32 * c)));
    };
    auto read_v = [&](v8 (&vf)[4]) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const u32x2 lo = lds_read_tr(vl + vtro[d]);            // keys 4 g4 + s
            const u32x2 hi = lds_read_tr(vl + 16 * PD + vtro[d]);  // keys 16 + 4 g4 + s
            vf[d] = __builtin_bit_cast(v8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        }
    };
    auto s_mfma = [&](const v8 (&kf)[2][2], f32x4 (&s)[2][2]) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                s[kb][b] = Mfma<T>::run(kf[kb][0], qf[b][0], f32x4{0.f, 0.f, 0.f, 0.f});
                s[kb][b] = Mfma<T>::run(kf[kb][1], qf[b][1], s[kb][b]);
            }
    };
    // Edge tiles: keys at or past a row's limit get -inf.
    auto mask_edge = [&](const int t, f32x4 (&s)[2][2]) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int rel = row_lim(b) - t * PT - 4 * g4;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[kb][b][i] = 16 * kb + i < rel ? s[kb][b][i] : -INFINITY;
        }
    };
    // Lazy rescale: m moves only when a score would pass it by more than 2^8; each lane
    // checks its own scores, and only a wavefront where one does pays for the row maximum
    // and the O / l rescale.
    auto rescale = [&](const f32x4 (&s)[2][2]) -> bool {
        float lmax[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) lmax[b] = lane_max8(s[0][b], s[1][b]);
        if (__builtin_amdgcn_ballot_w64((lmax[0] > m_thr[0]) | (lmax[1] > m_thr[1]))) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const float rmax = row_max4(lmax[b]);
                const bool move = rmax > m_thr[b];
                const float mt = rmax * c2;
                const float alpha = move ? __builtin_amdgcn_exp2f(m_run[b] - mt) : 1.f;  // 0 while m was -inf
                if (move) {
                    m_run[b] = mt;
                    m_thr[b] = rmax + lazy_raw;
                    neg_m[b] = -mt;
                }
                lacc[b] *= alpha;
#pragma unroll
                for (int d = 0; d < 4; ++d) o[d][b] *= alpha;
            }
            return true;
        }
        return false;
    };
    auto probs = [&](const f32x4 (&s)[2][2], int b, v8& pf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[0][b][i], c2, neg_m[b]));
            const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[1][b][i], c2, neg_m[b]));
            pf[i] = static_cast<T>(e0);
            pf[4 + i] = static_cast<T>(e1);
        }
    };
    // The row-sum MFMA's column of ones, held in four VGPRs across the loop (the empty asm
    // keeps the compiler from rebuilding it from scalar constants at every use).
    v8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = static_cast<T>(1.f);
    __asm__ volatile("" : "+v"(ones));
    auto pv = [&](const v8 (&vf)[4], int b, const v8& pf) {
        lacc[b] = Mfma<T>::run(ones, pf, lacc[b]);
#pragma unroll
        for (int d = 0; d < 4; ++d) o[d][b] = Mfma<T>::run(vf[d], pf, o[d][b]);
    };

    if constexpr (PIPE) {
        // Prologue: tile 0's K and V, then S of tile 0.
        f32x4 s_cur[2][2];
        if (nt_w > 0) {
            dma(tile_of(0), false);
            dma(tile_of(0), true);
        }
        load_q();
        fix_sign();
        if (nt_w > 0) {
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            v8 kf[2][2];
            read_k(kf);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            s_mfma(kf, s_cur);
            if (nt_w > 1) dma(tile_of(1), false);
        }
        // One step: tile t = tile_of(j) with S in s_cur; NEXT: tile_of(j + 1) exists, its
        // K is in the LDS tile (V of tile t is in the V tile).
        auto step = [&](const int j, auto next_tag) {
            constexpr bool NEXT = decltype(next_tag)::value;
            const int t = tile_of(j);
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            v8 kf[2][2], vf[4];
            if constexpr (NEXT) read_k(kf);
            read_v(vf);
            if (t >= nfull) mask_edge(t, s_cur);
            rescale(s_cur);
            // This step's fragments are in registers: the next step's loads go out now.
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if constexpr (NEXT) {
                if (j + 2 < nt_w) dma(tile_of(j + 2), false);
                dma(tile_of(j + 1), true);
            }
            v8 pf[2];
            f32x4 s_nxt[2][2];
            if constexpr (NEXT) s_mfma(kf, s_nxt);
            probs(s_cur, 0, pf[0]);
            pv(vf, 0, pf[0]);
            probs(s_cur, 1, pf[1]);
            pv(vf, 1, pf[1]);
            // Issue pattern (one basic block): the 8 S MFMAs of the next tile each followed
            // by about three of row block 0's 20 softmax instructions (8 FMA, 8 exp, 4
            // packs); row block 0's 5 PV MFMAs each followed by 4 of row block 1's; then
            // row block 1's PV MFMAs.  MFMA (mask 0x008) and VALU (0x002) groups.
            if constexpr (NEXT) {
#pragma unroll
                for (int i = 0; i < 6; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            } else {
                __builtin_amdgcn_sched_group_barrier(0x002, 20, 0);
            }
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
            if constexpr (NEXT) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int b = 0; b < 2; ++b) s_cur[kb][b] = s_nxt[kb][b];
            }
        };
        int j = 0;
        for (; j + 1 < nt_w; ++j) step(j, std::true_type{});
        if (j < nt_w) step(j, std::false_type{});
    } else {
        // A step: wait for tile t's K and V (requested one step earlier), S = K Q^T with
        // V^T read meanwhile, the next tile's loads, then softmax and PV.
        if (nt_w > 0) {
            dma(tile_of(0), false);
            dma(tile_of(0), true);
        }
        load_q();
        fix_sign();
        auto load_step = [&](const int j, f32x4 (&s)[2][2], v8 (&vf)[4]) {
            const int t = tile_of(j);
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            {
                v8 kf[2][2];
                read_k(kf);
                s_mfma(kf, s);
            }
            read_v(vf);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (j + 1 < nt_w) {
                dma(tile_of(j + 1), false);
                dma(tile_of(j + 1), true);
            }
            if (t >= nfull) mask_edge(t, s);
        };
        if (nt_w > 0) {
            // First tile: its row maxima are the reference points, and O and l start from
            // its products (no zero fill, no rescale).  A row with no visible key here keeps
            // m = -inf and weight 0 until one comes.
            f32x4 s[2][2];
            v8 vf[4];
            load_step(0, s, vf);
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const float rmax = row_max4(lane_max8(s[0][b], s[1][b]));
                const bool seen = rmax > -INFINITY;
                m_run[b] = seen ? rmax * c2 : -INFINITY;
                m_thr[b] = seen ? rmax + lazy_raw : -INFINITY;
                neg_m[b] = seen ? -m_run[b] : 0.f;
            }
            v8 pf[2];
            probs(s, 0, pf[0]);
            probs(s, 1, pf[1]);
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                lacc[b] = Mfma<T>::run(ones, pf[b], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int d = 0; d < 4; ++d) o[d][b] = Mfma<T>::run(vf[d], pf[b], f32x4{0.f, 0.f, 0.f, 0.f});
            }
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                lacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int d = 0; d < 4; ++d) o[d][b] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        for (int j = 1; j < nt_w; ++j) {
            f32x4 s[2][2];
            v8 vf[4];
            load_step(j, s, vf);
            rescale(s);
            v8 pf[2];
            probs(s, 0, pf[0]);
            pv(vf, 0, pf[0]);
            probs(s, 1, pf[1]);
            pv(vf, 1, pf[1]);
            // Row block 0's PV MFMAs interleave with row block 1's exponentials.
            __builtin_amdgcn_sched_group_barrier(0x002, 20, 0);
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
        }
    }

    float* const mine = reinterpret_cast<float*>(wbase);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int row = 16 * b + l16;
#pragma unroll
        for (int d = 0; d < 4; ++d)
            *reinterpret_cast<f32x4*>(mine + row * PCP + 4 * ((4 * d + g4) ^ l16)) = o[d][b];
        if (g4 == 0) *reinterpret_cast<float2*>(stats + 2 * row) = float2{m_run[b], lacc[b][0]};
    }
}

// The combine of query tile xt of unit bh over the nw wavefronts from w0 (their O areas
// and statistics in LDS): thread i of 256 -> row i / 8, columns 8 (i % 8) .. + 7; the
// wavefronts are added in order (deterministic).
template <typename T>
__device__ __forceinline__ void pipe_combine(const AttnParams& p, const int bh, const int xt, const int w0,
                                             const int nw, const int i, unsigned char* const smem, const int nw_all) {
    const int seq = fdiv(bh, p.fd_hkv);
    const int kvh = bh - seq * p.hkv;
    const int G = p.group;
    const int vrows = p.seq_q * G;
    const int row = i >> 3, cg = i & 7;
    const int r = xt * PB + row;
    const float* stats = reinterpret_cast<const float*>(smem + static_cast<size_t>(nw_all) * PWAVE_BYTES);
    float m = -INFINITY;
    for (int w = w0; w < w0 + nw; ++w) {
        const float2 sw = *reinterpret_cast<const float2*>(stats + 2 * (w * PB + row));
        m = fmaxf(m, sw.y > 0.f ? sw.x : -INFINITY);
    }
    float lt = 0.f;
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
    for (int w = w0; w < w0 + nw; ++w) {
        const float2 sw = *reinterpret_cast<const float2*>(stats + 2 * (w * PB + row));
        const float wt = sw.y > 0.f ? __builtin_amdgcn_exp2f(sw.x - m) : 0.f;
        lt += wt * sw.y;
        const float* ow = reinterpret_cast<const float*>(smem + static_cast<size_t>(w) * PWAVE_BYTES) + row * PCP;
        lo += *reinterpret_cast<const f32x4*>(ow + 4 * ((2 * cg) ^ (row & 15))) * wt;
        hi += *reinterpret_cast<const f32x4*>(ow + 4 * ((2 * cg + 1) ^ (row & 15))) * wt;
    }
    if (r >= vrows) return;
    // lt >= 1 when a row saw a key (the wavefront whose reference point is the row's
    // maximum contributes exp2(0) = 1 at weight 1): the hardware reciprocal and log2 are
    // used without range reduction (the output is rounded to 16 bits).
    const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;
    const int pos = fdiv(r, p.fd_group);
    const int head = kvh * G + (r - pos * G);
    typedef T v8o __attribute__((ext_vector_type(8)));
    v8o w8;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w8[k] = static_cast<T>(lo[k] * inv);
        w8[4 + k] = static_cast<T>(hi[k] * inv);
    }
    // The host takes this kernel only for 16-byte aligned output rows.
    T* dst = static_cast<T*>(p.out) + seq * p.os[0] + head * p.os[1] + static_cast<int64_t>(pos) * p.os[2] + 8 * cg;
    *reinterpret_cast<v8o*>(dst) = w8;
    if (p.lse && cg == 0)
        p.lse[seq * p.ls[0] + head * p.ls[1] + static_cast<int64_t>(pos) * p.ls[2]] =
            lt > 0.f ? (m + __builtin_amdgcn_logf(lt)) * kLn2 : -INFINITY;
}

// Workgroup -> group of query tiles.  Four wavefronts: one query tile per workgroup, in
// the orders of attn_fwd_kernel (causal: heaviest first, alternating direction per round
// of CU-count blocks when the grid is resident in one round; non-causal grids over large
// K/V: one contiguous chunk of the unit-major tiles per XCD).  Eight wavefronts (causal):
// the tiles ranked heaviest first (rank r: unit r % units, tile nx - 1 - r / units); the
// grp_single heaviest run alone, the rest in pairs (rank grp_single + j with the
// lightest unpaired rank), the wavefronts split between a pair's tiles in proportion to
// their key tiles, so that every workgroup carries about the same work.
template <typename T, bool CAUSAL, int NW, bool PIPE>
__global__ __launch_bounds__(NW * kWave, PIPE ? 3 : 4) void attn_pipe_kernel(const AttnParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    // Read one word of each 64-byte argument line the kernel uses, all in one batch: the
    // compiler splits the argument loads into batches by use (the workgroup mapping, then
    // the tile's pointers and strides, then the scale), each a round trip before the first
    // K / V loads go out; with the lines in the scalar cache the later batches hit it.
    __asm__ volatile("" ::"s"(p.q), "s"(p.ks[0]), "s"(p.os[0]), "s"(p.batch), "s"(p.fd_units.m));
    const int units = p.batch * p.hkv;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    int lin = blockIdx.x;
    int bh[2] = {0, 0}, xt[2] = {0, 0}, nwv[2] = {NW, 0};
    int ntile = 1;
    if constexpr (NW == 4) {
        if (p.xcd_map == 2) {
            const int x = lin & 7, s = lin >> 3;
            const int total = p.nx * units, per = (total + 7) >> 3;
            const int item = x * per + s;
            if (s >= per || item >= total) return;
            bh[0] = item / p.nx;
            const int r = item - bh[0] * p.nx;
            xt[0] = CAUSAL ? p.nx - 1 - r : r;
        } else {
            if (p.snake > 0) {
                const int round = fdiv(lin, p.fd_snake), pos = lin - round * p.snake;
                const int in_round = min(p.snake, p.nx * units - round * p.snake);
                if (round & 1) lin = round * p.snake + (in_round - 1 - pos);
            }
            const int xi = fdiv(lin, p.fd_units);
            bh[0] = lin - xi * units;
            xt[0] = CAUSAL ? p.nx - 1 - xi : xi;
        }
        nwv[0] = 4;
    } else {
        const int total = p.nx * units;
        int ra, rb = -1;
        if (lin < p.grp_single) {
            ra = lin;
        } else if (lin - p.grp_single < p.grp_pair) {
            const int j = lin - p.grp_single;
            ra = p.grp_single + j;
            rb = total - 1 - j;
        } else {
            ra = p.grp_single + p.grp_pair;
            if (ra >= total - p.grp_pair) return;
        }
        auto unrank = [&](int r, int& u, int& x) {
            const int q = fdiv(r, p.fd_units);
            u = r - q * units;
            x = CAUSAL ? p.nx - 1 - q : q;
        };
        unrank(ra, bh[0], xt[0]);
        nwv[0] = NW;
        if (rb >= 0) {
            unrank(rb, bh[1], xt[1]);
            const int na = tile_keys<CAUSAL>(p, xt[0]).x, nb = tile_keys<CAUSAL>(p, xt[1]).x;
            const int wa = min(NW - 1, max(1, (NW * na + (na + nb) / 2) / max(1, na + nb)));
            nwv[0] = wa;
            nwv[1] = NW - wa;
            ntile = 2;
        }
    }
    // This wavefront's tile (selects, not indexing: the pair stays in scalar registers).
    const bool second = ntile == 2 && wave >= nwv[0];
    const int w0 = second ? nwv[0] : 0;
    float* const stats = reinterpret_cast<float*>(smem + static_cast<size_t>(NW) * PWAVE_BYTES) + 2 * PB * wave;
    const int my_bh = __builtin_amdgcn_readfirstlane(second ? bh[1] : bh[0]);
    const int my_xt = __builtin_amdgcn_readfirstlane(second ? xt[1] : xt[0]);
    const int my_nw = __builtin_amdgcn_readfirstlane(second ? nwv[1] : nwv[0]);
    if (my_xt * PB < p.seq_q * p.group)
        pipe_tile<T, CAUSAL, PIPE, (NW == 4 ? 4 : 0)>(p, my_bh, my_xt, wave - w0, my_nw,
                                                       smem + static_cast<size_t>(wave) * PWAVE_BYTES, stats);
    __syncthreads();
    const int i = threadIdx.x & 255;
    const bool tg = static_cast<int>(threadIdx.x) >= 256;
    const int c_bh = tg ? bh[1] : bh[0], c_xt = tg ? xt[1] : xt[0];
    if ((!tg || ntile == 2) && c_xt * PB < p.seq_q * p.group)
        pipe_combine<T>(p, c_bh, c_xt, tg ? nwv[0] : 0, tg ? nwv[1] : nwv[0], i, smem, NW);
}

// KMI_ATTN_PIPE_NW=4|8 and KMI_ATTN_PIPE_MODE=0|1 (read once) pin the wavefronts per
// workgroup and the pipelined step for experiments.
int pipe_env(const char* name, int dflt) {
    const char* e = std::getenv(name);
    return e ? std::atoi(e) : dflt;
}

template <typename T, bool CAUSAL, int NW, bool PIPE>
hipError_t launch_pipe_t(const AttnParams& p_in, hipStream_t stream) {
    static std::once_flag once;
    static int per_cu = 0;
    static hipError_t attr_err = hipSuccess;
    const void* fn = reinterpret_cast<const void*>(&attn_pipe_kernel<T, CAUSAL, NW, PIPE>);
    constexpr size_t lds = pipe_lds_bytes<NW>();
    std::call_once(once, [&] {
        attr_err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (attr_err == hipSuccess &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, NW * kWave, lds) != hipSuccess)
            per_cu = 0;
    });
    if (attr_err != hipSuccess) return attr_err;
    AttnParams p = p_in;
    const int64_t units = static_cast<int64_t>(p.batch) * p.hkv;
    p.nx = static_cast<int>(ceil_div(static_cast<int64_t>(p.seq_q) * p.group, PB));
    const int64_t total = static_cast<int64_t>(p.nx) * units;
    int64_t grid = total;
    const int64_t slots = static_cast<int64_t>(per_cu) * cu_count();
    p.xcd_map = 0;
    p.snake = 0;
    p.grp_single = 0;
    p.grp_pair = 0;
    if constexpr (NW == 4) {
        const int64_t kv_bytes = units * static_cast<int64_t>(p.seq_k) * PD * 2 * static_cast<int64_t>(sizeof(T));
        if (CAUSAL && slots > 0 && grid <= slots) p.snake = cu_count();
        if (!CAUSAL && kv_bytes > (int64_t{4} << 20) && xcd_map_mode() != 0) {
            p.xcd_map = 2;
            grid = 8 * ceil_div(grid, int64_t{8});
        }
    } else {
        // Groups: as many as the resident workgroups when the tiles allow it (the heaviest
        // alone, the rest paired), otherwise every tile paired.
        const int64_t target = std::max<int64_t>(1, slots);
        const int64_t singles = std::min<int64_t>(total, std::max<int64_t>(0, 2 * target - total));
        const int64_t pairs = (total - singles) / 2;
        p.grp_single = static_cast<int>(singles);
        p.grp_pair = static_cast<int>(pairs);
        grid = singles + pairs + ((total - singles) & 1);
    }
    p.fd_snake = fast_div(static_cast<uint32_t>(p.snake));
    p.fd_units = fast_div(static_cast<uint32_t>(units));
    hipLaunchKernelGGL((attn_pipe_kernel<T, CAUSAL, NW, PIPE>), dim3(static_cast<unsigned>(grid)), dim3(NW * kWave),
                       lds, stream, p);
    return hipGetLastError();
}

// Defaults, from same-box A/B runs on C1 (causal GQA 1x14/2x2048x64): four wavefronts and
// the plain step, 20.8 us; pipelined step 21.7 us; eight wavefronts 22.9 / 26.8 us;
// attn_fwd_kernel 22.2 us.
template <typename T, bool CAUSAL>
hipError_t launch_pipe_c(const AttnParams& p, hipStream_t stream) {
    static const int nw = pipe_env("KMI_ATTN_PIPE_NW", 4);
    static const int mode = pipe_env("KMI_ATTN_PIPE_MODE", 0);
    if (nw == 8 && CAUSAL) {
        return mode ? launch_pipe_t<T, CAUSAL, 8, true>(p, stream) : launch_pipe_t<T, CAUSAL, 8, false>(p, stream);
    }
    return mode ? launch_pipe_t<T, CAUSAL, 4, true>(p, stream) : launch_pipe_t<T, CAUSAL, 4, false>(p, stream);
}

}  // namespace

template <typename T>
hipError_t launch_pipe(const AttnParams& p, hipStream_t stream) {
    return p.causal ? launch_pipe_c<T, true>(p, stream) : launch_pipe_c<T, false>(p, stream);
}
template hipError_t launch_pipe<bf16>(const AttnParams&, hipStream_t);
template hipError_t launch_pipe<f16>(const AttnParams&, hipStream_t);

}  // namespace fwd
}  // namespace kmi
