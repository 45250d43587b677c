// Parameters shared by the host side of the attention forward (attention.hip) and its
// kernels (attention_kernels.hpp, instantiated per padded head dim in attention_d*.hip).
#pragma once

#include "common.hpp"

namespace kmi {
namespace fwd {

constexpr int NWAVES = 4;  // wavefronts per workgroup
constexpr int NTHREADS = NWAVES * kWave;
// Keys per wavefront tile.
constexpr int WN = 32;
// Row split stages a unit's whole key range in LDS up to this many tiles (eight measured
// slower: fewer workgroups fit per CU).
constexpr int kRsTiles = 4;

// n / d for 0 <= n < 2^31 by a multiply-high (the round-up method of Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994): with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, m) + n) >> l
// (the sum stays below 2^32 since mulhi(n, m) <= n).  The kernels' tile and row indices
// divide by a few per-call values (the split count, the unit count, the K/V heads, the
// GQA group); a runtime integer division is a ~30-instruction sequence through the
// reciprocal unit, this is three.
struct FastDiv {
    uint32_t m, l;
};

inline FastDiv fast_div(uint32_t d) {
    if (d == 0) d = 1;
    uint32_t l = 0;
    while ((uint64_t{1} << l) < d) ++l;
    const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1;
    return FastDiv{static_cast<uint32_t>(m), l};
}

__device__ __forceinline__ int fdiv(int n, FastDiv f) {
    const uint32_t u = static_cast<uint32_t>(n);
    return static_cast<int>((__umulhi(u, f.m) + u) >> f.l);
}

struct AttnParams {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    float* lse;
    float* part_o;    // [splits][rows_total][hq][D] fp32 (normalised partial outputs)
    float* part_lse;  // [splits][rows_total][hq][2] fp32: base-2 log-sum-exp, raw-mode flag
    int64_t qs[3], ks[3], vs[3], os[3], ls[3];
    const void* mask;
    int64_t ms[4];
    int64_t mask_numel;
    const int32_t* cu_q;
    const int32_t* cu_k;
    // Dense key lengths [batch] (or null): sequence b sees keys [0, clamp(klen[b], 1, seq_k)).
    const int32_t* klen;
    int mask_dtype, mask_mode;
    // Mask rows with unit key stride (every packed mask; strided masks with key stride 1):
    // whole tiles read their mask values four keys per load (element-aligned vector loads).
    int mask_vec4;
    // Row split with the unit's whole key range staged once in the workgroup's LDS
    // (rs_shared: the dynamic LDS holds every key tile, K then V).
    int rs_shared;
    // Packed masks: device int64 [batch + 1] block offsets (or null: added up in-kernel).
    const int64_t* mask_off;
    int batch, hq, hkv, group, seq_q, seq_k;
    int d;   // q / k head dim
    int dv;  // v / out head dim (the kernels' D template argument is the larger, padded to a multiple of 32)
    int causal;
    float scale_log2;
    int splits, tiles_per_split;
    int nx;  // query tiles per (sequence, K/V head)
    int npair;  // causal: the 2 npair shortest query tiles of a unit run two per workgroup
    // Workgroup order across the XCDs (block b runs on XCD b % 8): 0 the plain order; 1
    // unit u on XCD u % 8, query tiles heaviest first; 3 the same with each tile row's units
    // rotated by the row; 2 the unit-major query tiles in one contiguous chunk per XCD.
    // Each keeps a unit's K/V in the L2 of one or two XCDs.
    int xcd_map;
    // Causal grids resident in one round: the CU count n (0: off).  Blocks b, b + n, b + 2n
    // ... run on one CU, so the heaviest-first rank order runs forward in even rounds of n
    // blocks and backward in odd ones, which evens out the work each CU gets.
    int snake;
    // Divisors of the index arithmetic (see FastDiv): splits, batch * hkv, hkv, group, snake.
    FastDiv fd_splits, fd_units, fd_hkv, fd_group, fd_snake;
    int total_q, total_k;  // varlen packed token counts
    int64_t rows_total;
    // attn_pipe_kernel with eight wavefronts: the heaviest grp_single query tiles run
    // alone, the next 2 grp_pair in pairs (attention_pipe.hip).
    int grp_single, grp_pair;
    // Decode split counters (or null: a separate merge launch): one 64-bit word per
    // (sequence, K/V head), zero between calls.  Each workgroup adds 2^32 plus bit `split`
    // when its partial carries weight; the one that brings the count to `splits` merges
    // the unit's partials and clears the word.
    unsigned long long* ctr;
};

struct Plan {
    bool decode;  // attn_decode_kernel: per-wavefront key ranges, fp32 partials + merge
    bool rs;      // row split: short key ranges, one row block per wavefront
    bool rs_shared;  // row split with the unit's key tiles (at most four) staged in LDS once
    bool pipe;       // attn_pipe_kernel: head dim 64, unmasked, dense, one split (attention_pipe.hip)
    int nqb, nx, splits, tiles_per_split;
    int64_t rows_total;
    size_t ws_bytes;
};

// Compute units of the current device (cached per device id).
int cu_count();

// Enqueues the forward of a planned call for element type T and padded head dim D
// (explicit instantiations in attention_d<D>.hip).
template <typename T, int D>
hipError_t launch_all(const AttnParams& p, const Plan& pl, hipStream_t stream);

// The current device's decode split counters for calls on `stream` (zero-initialised
// device memory that every merge leaves zero; one slab per stream so that calls on
// different streams never share a word), or null when a call over `units` units must
// merge in a separate launch.
unsigned long long* decode_counters(hipStream_t stream, int64_t units);

// Enqueues attn_pipe_kernel for a call the plan gave it (instantiated in attention_pipe.hip).
template <typename T>
hipError_t launch_pipe(const AttnParams& p, hipStream_t stream);

}  // namespace fwd
}  // namespace kmi
