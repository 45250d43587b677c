// LayerNorm / RMSNorm forward for gfx950 with fp32 statistics.
//
// Reference semantics: src/kohakutt_native/csrc/aten/nn/aten_norm.cpp:65-127 (layer_norm:
// y = (x - mean) * rstd * weight + bias, fp32 mean / rstd), :604-652 (rms_norm), and
// aten_fused.cpp:13-28 (rms_norm with bias); statistics as ktt_norm/fwd_compute.cpp:
// 275-358: two passes (mean, then the centred sum of squares), var = relu(M2 / W),
// rstd = 1 / sqrt(var + eps).  The reference splits a tile row of 32 rows over a group of
// Tensix cores and merges partial statistics (Chan); here a 64-lane wavefront owns one
// row, keeps it in registers (one HBM read, one HBM write) and reduces across lanes.
//
// Vector paths (rows whose width is a multiple of one 16-byte vector, 16-byte aligned
// pointers): one wavefront per row holding up to 4 vectors per lane, or for wider rows
// one 256-thread block per row holding up to 8 vectors per thread.  Generic path: one
// 256-thread block per row with element loads (any width and alignment).
#include "common.hpp"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace kmi {
namespace fwd {
// Split counters shared with the decode merge (attention.hip): zero-initialised device
// words, one slab per stream, left zero by every use (null: none free).
unsigned long long* decode_counters(hipStream_t stream, int64_t units);
}  // namespace fwd
namespace {

// Row-block grids.  HIP bounds each grid dimension at 2^32 - 1 work-items, which one
// 256-thread block per row passes at 2^24 rows (and one wavefront per row at 2^26): a
// launch of more blocks than kGridX spreads them over y, and a block finds its index as
// y * gridDim.x + x (blocks past the last row return before any barrier).
constexpr int64_t kGridX = int64_t{1} << 20;

dim3 block_grid(int64_t blocks) {
    if (blocks <= kGridX) return dim3(static_cast<unsigned>(blocks));
    return dim3(static_cast<unsigned>(kGridX), static_cast<unsigned>(ceil_div(blocks, kGridX)));
}

__device__ __forceinline__ int64_t block_index() {
    return static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
}

// Compute units of the current device (cached per device id; 0 when unknown).
int device_cus() {
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

template <typename T, int E>
struct alignas(E * sizeof(T)) Pack {
    T e[E];
};

template <typename T, int E>
__device__ __forceinline__ void store_pack(T* p, const float* in) {
    Pack<T, E> v;
#pragma unroll
    for (int j = 0; j < E; ++j) v.e[j] = from_f32<T>(in[j]);
    *reinterpret_cast<Pack<T, E>*>(p) = v;
}

// Weight or bias values for one vector of E elements of x, loaded raw (so that every load
// of a row is issued before the first one is waited for) and widened when used.
template <typename W, int E>
struct Param {
    Pack<W, E> v;
    __device__ __forceinline__ void load(const W* p, int vi) { v = *reinterpret_cast<const Pack<W, E>*>(p + vi * E); }
    __device__ __forceinline__ float at(int j) const { return to_f32(v.e[j]); }
};

// The E = 16 / sizeof(T) elements of one 16-byte vector as fp32 (bf16: the high half of
// an fp32; f16: converted; f32: as is).
template <typename T>
__device__ __forceinline__ void unpack(const u32x4& raw, float* out) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int k = 0; k < 4; ++k) out[k] = __uint_as_float(raw[k]);
    } else if constexpr (std::is_same<T, bf16>::value) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            out[2 * k] = __uint_as_float(raw[k] << 16);
            out[2 * k + 1] = __uint_as_float(raw[k] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            out[2 * k] = to_f32(__builtin_bit_cast(f16, static_cast<uint16_t>(raw[k] & 0xffffu)));
            out[2 * k + 1] = to_f32(__builtin_bit_cast(f16, static_cast<uint16_t>(raw[k] >> 16)));
        }
    }
}

// Sum over a wavefront's 64 lanes without LDS round trips: a butterfly within each row of
// 16 lanes through DPP (xor 1 and xor 2 by quad permutes, then the half-row and row
// mirrors), the four row sums read from lanes 0, 16, 32, 48 and added in that order; every
// lane gets the result.  (The lane-shuffle butterfly takes six dependent LDS-crossbar
// round trips.)
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f32<0xb1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f32<0x4e>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    const int iv = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
    return (r0 + r1) + (r2 + r3);
}

// LayerNorm statistics of a set of values: count, mean and centred sum of squares.  A
// wavefront forms them exactly over its values (a sum for the mean, then the centred
// squares, both plain cross-lane sums); sets held by different wavefronts merge by Chan,
// Golub and LeVeque's pairwise update -- the reference's merge of per-core partial
// statistics (ktt_norm/fwd_compute.cpp:317-346).
struct RowStats {
    float n, mean, m2;
};

__device__ __forceinline__ RowStats chan_merge(const RowStats& a, const RowStats& b) {
    const float n = a.n + b.n;
    const float fb = n > 0.f ? b.n / n : 0.f;
    const float d = b.mean - a.mean;
    return RowStats{n, a.mean + d * fb, a.m2 + b.m2 + d * d * a.n * fb};
}

// A wavefront's statistics over the n values of its lanes' valid vectors (vector i of a
// lane is valid when valid(i); invalid ones hold zeros).
template <typename T, int NV, typename Valid>
__device__ __forceinline__ RowStats wave_row_stats(const u32x4 (&raw)[NV], Valid valid, float n) {
    constexpr int E = 16 / sizeof(T);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float v[E];
        unpack<T>(raw[i], v);
#pragma unroll
        for (int j = 0; j < E; ++j) sum += v[j];
    }
    sum = wave_sum(sum);
    const float mean = n > 0.f ? sum / n : 0.f;
    float m2 = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (!valid(i)) continue;
        float v[E];
        unpack<T>(raw[i], v);
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float c = v[j] - mean;
            m2 += c * c;
        }
    }
    return RowStats{n, mean, wave_sum(m2)};
}

// One wavefront per row, blockDim / 64 rows per block.  T: x / y; W: weight and bias.  The
// row stays in registers as loaded (packed) and is widened to fp32 in each pass, which
// keeps the register count, and so the wavefronts in flight per SIMD, up.  Every load of
// the row (x, weight, bias) is issued at once from clamped in-range indices: per-lane
// branches around them made each wait for the previous one (five round trips for a
// LayerNorm row instead of one).
template <typename T, typename W, int VPL, bool LAYER, int PRM>
__global__ __launch_bounds__(1024) void norm_rows_wave(
    const T* x, const W* weight, const W* bias,
    T* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out,
    int64_t rows, int width, float eps) {
    constexpr int E = 16 / sizeof(T);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = block_index() * (blockDim.x / kWave) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int nvec = width / E;
    const T* xr = x + row * width;
    // PRM bit 0: a weight, bit 1: a bias (compile-time, so that the loads form one
    // straight-line group).
    constexpr bool HW = PRM & 1, HB = PRM & 2;
    u32x4 raw[VPL];
    Param<W, E> g[VPL], bb[VPL];
    // Weight and bias first, then the row: the row's values are used first, and the
    // compiler waits for them where they are used (after every load is issued).
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vc = min(lane + kWave * i, nvec - 1);
        if constexpr (HW) g[i].load(weight, vc);
        if constexpr (HB) bb[i].load(bias, vc);
    }
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < VPL; ++i) raw[i] = *reinterpret_cast<const u32x4*>(xr + min(lane + kWave * i, nvec - 1) * E);
#pragma unroll
    for (int i = 0; i < VPL; ++i)
        if (lane + kWave * i >= nvec) raw[i] = u32x4{0u, 0u, 0u, 0u};
    const float inv_w = 1.f / static_cast<float>(width);
    float mean = 0.f, rstd;
    if constexpr (LAYER) {
        const RowStats st = wave_row_stats<T, VPL>(raw, [&](int i) { return lane + kWave * i < nvec; },
                                                   static_cast<float>(width));
        mean = st.mean;
        rstd = 1.f / sqrtf(fmaxf(st.m2 * inv_w, 0.f) + eps);
    } else {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            float v[E];
            unpack<T>(raw[i], v);
#pragma unroll
            for (int j = 0; j < E; ++j) sum += v[j] * v[j];
        }
        sum = wave_sum(sum);
        rstd = 1.f / sqrtf(sum * inv_w + eps);
    }
    T* yr = y + row * width;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + kWave * i;
        if (vi < nvec) {
            float v[E], o[E];
            unpack<T>(raw[i], v);
#pragma unroll
            for (int j = 0; j < E; ++j) {
                o[j] = (v[j] - mean) * rstd;
                if constexpr (HW) o[j] *= g[i].at(j);
                if constexpr (HB) o[j] += bb[i].at(j);
            }
            store_pack<T, E>(yr + vi * E, o);
        }
    }
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
}

// Wide rows: 256-thread blocks that stride over the rows (grid sized to the resident
// blocks), each thread holding VPT vectors of a row; the weight and bias vectors are loaded
// once per block, not once per row (at width 8192 that re-read was as many bytes as the
// rows themselves).  The four wavefronts' partial statistics meet in LDS in a fixed order,
// in a buffer that alternates with the row's parity (one barrier per row).
template <typename T, typename W, int VPT, bool LAYER, int PRM>
__global__ __launch_bounds__(256) void norm_rows_block(
    const T* x, const W* weight, const W* bias,
    T* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out,
    int64_t rows, int width, float eps) {
    constexpr int E = 16 / sizeof(T);
    constexpr int NW = 4;
    __shared__ float red[2][3][NW];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wave = tid >> 6;
    const int64_t row0 = block_index();
    const int64_t rstep = static_cast<int64_t>(gridDim.x) * gridDim.y;
    if (row0 >= rows) return;
    const int nvec = width / E;
    constexpr bool HW = PRM & 1, HB = PRM & 2;  // weight, bias (see norm_rows_wave)
    Param<W, E> g[VPT], bb[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int vc = min(tid + 256 * i, nvec - 1);
        if constexpr (HW) g[i].load(weight, vc);
        if constexpr (HB) bb[i].load(bias, vc);
    }
    const float inv_w = 1.f / static_cast<float>(width);
    int nv_w = 0;  // this wavefront's valid vectors
#pragma unroll
    for (int i = 0; i < VPT; ++i) nv_w += min(max(nvec - 256 * i - kWave * wave, 0), kWave);
    // The next row's vectors are requested before this row is reduced and written, so a
    // block always has a row in flight.
    auto load_row = [&](int64_t r, u32x4 (&dst)[VPT]) {
        const T* xr = x + min(r, rows - 1) * width;
#pragma unroll
        for (int i = 0; i < VPT; ++i) dst[i] = *reinterpret_cast<const u32x4*>(xr + min(tid + 256 * i, nvec - 1) * E);
    };
    u32x4 nxt[VPT];
    load_row(row0, nxt);
    int par = 0;
    for (int64_t row = row0; row < rows; row += rstep, par ^= 1) {
        u32x4 raw[VPT];
#pragma unroll
        for (int i = 0; i < VPT; ++i) raw[i] = nxt[i];
        if (row + rstep < rows) load_row(row + rstep, nxt);
#pragma unroll
        for (int i = 0; i < VPT; ++i)
            if (tid + 256 * i >= nvec) raw[i] = u32x4{0u, 0u, 0u, 0u};
        float mean = 0.f, rstd;
        if constexpr (LAYER) {
            const RowStats st = wave_row_stats<T, VPT>(raw, [&](int i) { return tid + 256 * i < nvec; },
                                                       static_cast<float>(nv_w * E));
            if (lane == 0) {
                red[par][0][wave] = st.n;
                red[par][1][wave] = st.mean;
                red[par][2][wave] = st.m2;
            }
            __syncthreads();
            // Every thread merges the four wavefronts' statistics in wavefront order.
            RowStats all{red[par][0][0], red[par][1][0], red[par][2][0]};
#pragma unroll
            for (int w = 1; w < NW; ++w) all = chan_merge(all, RowStats{red[par][0][w], red[par][1][w], red[par][2][w]});
            mean = all.mean;
            rstd = 1.f / sqrtf(fmaxf(all.m2 * inv_w, 0.f) + eps);
        } else {
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < VPT; ++i) {
                float v[E];
                unpack<T>(raw[i], v);
#pragma unroll
                for (int j = 0; j < E; ++j) sum += v[j] * v[j];
            }
            sum = wave_sum(sum);
            if (lane == 0) red[par][0][wave] = sum;
            __syncthreads();
            sum = (red[par][0][0] + red[par][0][1]) + (red[par][0][2] + red[par][0][3]);
            rstd = 1.f / sqrtf(sum * inv_w + eps);
        }
        T* yr = y + row * width;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int vi = tid + 256 * i;
            if (vi < nvec) {
                float v[E], o[E];
                unpack<T>(raw[i], v);
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    o[j] = (v[j] - mean) * rstd;
                    if constexpr (HW) o[j] *= g[i].at(j);
                    if constexpr (HB) o[j] += bb[i].at(j);
                }
                store_pack<T, E>(yr + vi * E, o);
            }
        }
        if (tid == 0) {
            if (mean_out) mean_out[row] = mean;
            if (rstd_out) rstd_out[row] = rstd;
        }
    }
}

__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t i) {
    switch (dtype) {
        case KMI_BF16: return to_f32(static_cast<const bf16*>(p)[i]);
        case KMI_F16: return to_f32(static_cast<const f16*>(p)[i]);
        default: return static_cast<const float*>(p)[i];
    }
}

__device__ __forceinline__ void store_any(void* p, int dtype, int64_t i, float v) {
    switch (dtype) {
        case KMI_BF16: static_cast<bf16*>(p)[i] = from_f32<bf16>(v); break;
        case KMI_F16: static_cast<f16*>(p)[i] = from_f32<f16>(v); break;
        default: static_cast<float*>(p)[i] = v;
    }
}

__device__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) t += scratch[i];
    return t;
}

// One 256-thread block per row; any width, any alignment; x read three times.
template <bool LAYER>
__global__ __launch_bounds__(256) void norm_rows_generic(
    const void* x, const void* weight, const void* bias, void* y, float* mean_out,
    float* rstd_out, int64_t rows, int64_t width, int x_dtype, int w_dtype, int b_dtype, float eps) {
    __shared__ float scratch[4];
    const int64_t row = block_index();
    if (row >= rows) return;
    const int64_t base = row * width;
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
        const float a = load_any(x, x_dtype, base + i);
        s += LAYER ? a : a * a;
    }
    s = block_sum(s, scratch);
    const float inv_w = 1.f / static_cast<float>(width);
    float mean = 0.f, rstd;
    if (LAYER) {
        mean = s * inv_w;
        float m2 = 0.f;
        for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
            const float c = load_any(x, x_dtype, base + i) - mean;
            m2 += c * c;
        }
        m2 = block_sum(m2, scratch);
        rstd = 1.f / sqrtf(fmaxf(m2 * inv_w, 0.f) + eps);
    } else {
        rstd = 1.f / sqrtf(s * inv_w + eps);
    }
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
        float o = (load_any(x, x_dtype, base + i) - mean) * rstd;
        if (weight) o *= load_any(weight, w_dtype, i);
        if (bias) o += load_any(bias, b_dtype, i);
        store_any(y, x_dtype, base + i, o);
    }
    if (threadIdx.x == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
}

template <typename T, typename W, bool LAYER>
hipError_t launch_wave(const void* x, const void* w, const void* b, void* y, float* mean,
                       float* rstd, int64_t rows, int width, float eps, int vpl,
                       hipStream_t stream) {
    // 16 rows per block once there are enough rows to fill the chip that way (fewer
    // workgroups to dispatch), 4 rows per block otherwise.
    const int rpb = rows >= 16 * 512 ? 16 : 4;
    const dim3 grid = block_grid(ceil_div(rows, rpb)), block(kWave * rpb);
    auto* xp = static_cast<const T*>(x);
    auto* wp = static_cast<const W*>(w);
    auto* bp = static_cast<const W*>(b);
    auto* yp = static_cast<T*>(y);
    const int prm = (w ? 1 : 0) | (b ? 2 : 0);
#define KMI_NORM_CASE(N)                                                                           \
    case N:                                                                                        \
        switch (prm) {                                                                             \
            case 0: hipLaunchKernelGGL((norm_rows_wave<T, W, N, LAYER, 0>), grid, block, 0, stream, \
                                       xp, wp, bp, yp, mean, rstd, rows, width, eps); break;       \
            case 1: hipLaunchKernelGGL((norm_rows_wave<T, W, N, LAYER, 1>), grid, block, 0, stream, \
                                       xp, wp, bp, yp, mean, rstd, rows, width, eps); break;       \
            case 2: hipLaunchKernelGGL((norm_rows_wave<T, W, N, LAYER, 2>), grid, block, 0, stream, \
                                       xp, wp, bp, yp, mean, rstd, rows, width, eps); break;       \
            default: hipLaunchKernelGGL((norm_rows_wave<T, W, N, LAYER, 3>), grid, block, 0, stream, \
                                        xp, wp, bp, yp, mean, rstd, rows, width, eps);             \
        }                                                                                          \
        break;
    switch (vpl) {
        KMI_NORM_CASE(1)
        KMI_NORM_CASE(2)
        KMI_NORM_CASE(4)
        default: return hipErrorInvalidValue;
    }
#undef KMI_NORM_CASE
    return hipGetLastError();
}

template <typename T, typename W, bool LAYER>
hipError_t launch_block(const void* x, const void* w, const void* b, void* y, float* mean,
                        float* rstd, int64_t rows, int width, float eps, int vpt,
                        hipStream_t stream) {
    // LayerNorm: eight blocks per CU, the rows striding over them (its weight and bias are
    // then read once per block; sweep [8192 x 8192] 48.4 -> 47.4 us).  RMSNorm: one block
    // per row (42.4 us; striding measured 44.1 us, its single weight re-read costing less
    // than the lost overlap).
    const int64_t nblocks = LAYER ? std::min<int64_t>(rows, 8 * std::max(1, device_cus())) : rows;
    const dim3 grid = block_grid(nblocks), block(256);
    auto* xp = static_cast<const T*>(x);
    auto* wp = static_cast<const W*>(w);
    auto* bp = static_cast<const W*>(b);
    auto* yp = static_cast<T*>(y);
    const int prm = (w ? 1 : 0) | (b ? 2 : 0);
#define KMI_NORM_CASE(N)                                                                            \
    case N:                                                                                         \
        switch (prm) {                                                                              \
            case 0: hipLaunchKernelGGL((norm_rows_block<T, W, N, LAYER, 0>), grid, block, 0, stream, \
                                       xp, wp, bp, yp, mean, rstd, rows, width, eps); break;        \
            case 1: hipLaunchKernelGGL((norm_rows_block<T, W, N, LAYER, 1>), grid, block, 0, stream, \
                                       xp, wp, bp, yp, mean, rstd, rows, width, eps); break;        \
            case 2: hipLaunchKernelGGL((norm_rows_block<T, W, N, LAYER, 2>), grid, block, 0, stream, \
                                       xp, wp, bp, yp, mean, rstd, rows, width, eps); break;        \
            default: hipLaunchKernelGGL((norm_rows_block<T, W, N, LAYER, 3>), grid, block, 0, stream, \
                                        xp, wp, bp, yp, mean, rstd, rows, width, eps);              \
        }                                                                                           \
        break;
    switch (vpt) {
        KMI_NORM_CASE(1)
        KMI_NORM_CASE(2)
        KMI_NORM_CASE(4)
        KMI_NORM_CASE(8)
        default: return hipErrorInvalidValue;
    }
#undef KMI_NORM_CASE
    return hipGetLastError();
}

int dtype_size(int dt) {
    switch (dt) {
        case KMI_BF16:
        case KMI_F16: return 2;
        case KMI_F32: return 4;
        default: return 0;
    }
}

bool aligned(const void* p, int64_t bytes) {
    return p == nullptr || (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// RMSNorm backward (the reference's ktt_norm backward programs, ktt_norm/bwd_*.cpp, with
// its column sum for the weight, colsum_*; layernorm.md:90-102).  y = x r w with
// r = rstd of the row: dx = r (g w) - x r^3 mean(g w x), dw = sum over rows of g x r.
// dx: one 256-thread block per row, fp32 sums; any width and alignment.
template <typename T>
__global__ __launch_bounds__(256) void rms_bwd_rows(const T* dy, const T* x, const void* weight, const float* rstd,
                                                    T* dx, int64_t rows, int64_t width, int w_dtype) {
    __shared__ float scratch[4];
    const int64_t row = block_index();
    if (row >= rows) return;
    const int64_t base = row * width;
    float s = 0.f;
#pragma unroll 4
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
        float gw = to_f32(dy[base + i]);
        if (weight) gw *= load_any(weight, w_dtype, i);
        s += gw * to_f32(x[base + i]);
    }
    s = block_sum(s, scratch);
    const float r = rstd[row];
    const float c = r * r * r * s / static_cast<float>(width);
#pragma unroll 4
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
        float gw = to_f32(dy[base + i]);
        if (weight) gw *= load_any(weight, w_dtype, i);
        dx[base + i] = from_f32<T>(r * gw - to_f32(x[base + i]) * c);
    }
}

// dw, first stage: block (column group, chunk) sums g x r over the chunk's rows for 256
// consecutive columns (coalesced across the threads) into fp32 partials [chunk][width].
template <typename T>
__global__ __launch_bounds__(256) void rms_bwd_dw_partial(const T* dy, const T* x, const float* rstd, float* part,
                                                          int64_t rows, int64_t width, int64_t rows_per_chunk) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (col >= width) return;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < rows ? r0 + rows_per_chunk : rows;
    float acc = 0.f;
#pragma unroll 8
    for (int64_t r = r0; r < r1; ++r) acc += to_f32(dy[r * width + col]) * to_f32(x[r * width + col]) * rstd[r];
    part[static_cast<int64_t>(blockIdx.y) * width + col] = acc;
}

// dw, second stage: the chunks' partials added in chunk order.
__global__ __launch_bounds__(256) void rms_bwd_dw_final(const float* part, void* dw, int64_t chunks, int64_t width,
                                                        int w_dtype) {
    const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (col >= width) return;
    float acc = 0.f;
#pragma unroll 8
    for (int64_t c = 0; c < chunks; ++c) acc += part[c * width + col];
    store_any(dw, w_dtype, col, acc);
}

constexpr int64_t kRmsBwdRowsPerChunk = 16;
constexpr int64_t kRmsBwdMaxChunks = 4096;

template <typename T>
hipError_t launch_rms_bwd(const void* dy, const void* x, const void* weight, const float* rstd, void* dx,
                          void* dweight, int64_t rows, int64_t width, int w_dtype, float* part, int64_t chunks,
                          hipStream_t s) {
    hipLaunchKernelGGL((rms_bwd_rows<T>), block_grid(rows), dim3(256), 0, s,
                       static_cast<const T*>(dy), static_cast<const T*>(x), weight, rstd, static_cast<T*>(dx), rows,
                       width, w_dtype);
    if (dweight) {
        const unsigned gx = static_cast<unsigned>(ceil_div(width, 256));
        hipLaunchKernelGGL((rms_bwd_dw_partial<T>), dim3(gx, static_cast<unsigned>(chunks)), dim3(256), 0, s,
                           static_cast<const T*>(dy), static_cast<const T*>(x), rstd, part, rows, width,
                           ceil_div(rows, chunks));
        hipLaunchKernelGGL(rms_bwd_dw_final, dim3(gx), dim3(256), 0, s, part, dweight, chunks, width, w_dtype);
    }
    return hipGetLastError();
}

int64_t rms_bwd_chunks(int64_t rows) {
    return std::min<int64_t>(kRmsBwdMaxChunks, std::max<int64_t>(1, ceil_div(rows, kRmsBwdRowsPerChunk)));
}

// Norm backward in one pass over dy and x (LayerNorm y = (x - m) r w + b; RMSNorm m = 0):
//   xh = (x - m) r, g = dy w, dx = r (g - mean(g) [LayerNorm only] - xh mean(g xh)),
//   dw = sum over rows of dy xh, db = sum over rows of dy
// (the reference's ktt_norm backward and column-sum programs, layernorm.md:90-102; torch's
// native_layer_norm_backward computes the same).  A block of four wavefronts takes a run of
// consecutive rows; wavefront w takes rows w, w + 4, ... of it (the next one's loads
// issued before the current one is worked on), holds a row in registers as
// VPL 16-byte vectors per lane, reduces mean(g) and mean(g xh) across its lanes, writes dx
// and adds dy xh (and dy) into per-lane column sums.  The wavefronts' column sums
// meet in LDS in wavefront order and the block writes one partial row pair;
// norm_bwd_colsum_parts adds the blocks' partials in a fixed order (deterministic).
// Wavefronts per block of the one-pass backward (eight measured slower: C5 LayerNorm's
// row pass 14.9 -> 23 us).
constexpr int kNormBwdWaves = 4;

template <typename T, typename W, bool LAYER, int VPL, bool HW, bool HB>
__global__ __launch_bounds__(kNormBwdWaves * kWave) void norm_bwd_rows(const T* dy, const T* x, const float* mean, const float* rstd,
                                                     const W* weight, T* __restrict__ dx, float* __restrict__ part,
                                                     int64_t rows, int width, int64_t rows_per_block) {
    constexpr int E = 16 / sizeof(T);
    extern __shared__ float colsum[];  // [2][width]: dw, db
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
    const int nvec = width / E;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
    const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
    Param<W, E> gw[HW ? VPL : 1];
    if constexpr (HW) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) gw[i].load(weight, min(lane + kWave * i, nvec - 1));
    }
    float aw[VPL][E], ab[HB ? VPL : 1][E];
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int j = 0; j < E; ++j) {
            aw[i][j] = 0.f;
            if constexpr (HB) ab[i][j] = 0.f;
        }
    const float inv_w = 1.f / static_cast<float>(width);
    // This wavefront's rows r0 + wave, r0 + wave + kNormBwdWaves, ...: the next row's dy, x and
    // statistics are requested before the current row is worked on (the statistics read in
    // the row's own iteration cost every row a round trip).
    int voff[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) voff[i] = min(lane + kWave * i, nvec - 1) * E;
    u32x4 nx_x[VPL], nx_g[VPL];
    float nx_m = 0.f, nx_r = 0.f;
    if (r0 + wave < r1) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            nx_x[i] = *reinterpret_cast<const u32x4*>(x + (r0 + wave) * width + voff[i]);
            nx_g[i] = *reinterpret_cast<const u32x4*>(dy + (r0 + wave) * width + voff[i]);
        }
        if constexpr (LAYER) nx_m = mean[r0 + wave];
        nx_r = rstd[r0 + wave];
    }
    for (int64_t row = r0 + wave; row < r1; row += kNormBwdWaves) {
        u32x4 rx[VPL], rg[VPL];
        for (int i = 0; i < VPL; ++i) {
            rx[i] = nx_x[i];
            rg[i] = nx_g[i];
        }
        const float m = nx_m, r = nx_r;
        if (row + kNormBwdWaves < r1) {
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                nx_x[i] = *reinterpret_cast<const u32x4*>(x + (row + kNormBwdWaves) * width + voff[i]);
                nx_g[i] = *reinterpret_cast<const u32x4*>(dy + (row + kNormBwdWaves) * width + voff[i]);
            }
            if constexpr (LAYER) nx_m = mean[row + kNormBwdWaves];
            nx_r = rstd[row + kNormBwdWaves];
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i)
            if (lane + kWave * i >= nvec) rx[i] = rg[i] = u32x4{0u, 0u, 0u, 0u};
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            float xv[E], gv[E];
            unpack<T>(rx[i], xv);
            unpack<T>(rg[i], gv);
#pragma unroll
            for (int j = 0; j < E; ++j) {
                const float xh = (xv[j] - m) * r;
                const float g = HW ? gv[j] * gw[i].at(j) : gv[j];
                sg += g;
                sgx += g * xh;
                aw[i][j] += gv[j] * xh;
                if constexpr (HB) ab[i][j] += gv[j];
            }
        }
        sgx = wave_sum_dpp(sgx);
        const float b = sgx * inv_w;
        const float a = LAYER ? wave_sum_dpp(sg) * inv_w : 0.f;
        T* dr = dx + row * width;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = lane + kWave * i;
            if (vi < nvec) {
                float xv[E], gv[E], o[E];
                unpack<T>(rx[i], xv);
                unpack<T>(rg[i], gv);
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const float xh = (xv[j] - m) * r;
                    const float g = HW ? gv[j] * gw[i].at(j) : gv[j];
                    o[j] = r * (g - a - xh * b);
                }
                store_pack<T, E>(dr + vi * E, o);
            }
        }
    }
    // The wavefronts' column sums, added in wavefront order; the last wavefront writes the block's
    // partial rows [blockIdx.x][2][width].  part is null when neither dw nor db is asked for
    // (the same for the whole grid, so every wavefront leaves here together).
    if (part == nullptr) return;
    float* pw = part + static_cast<int64_t>(blockIdx.x) * 2 * width;
    for (int w = 0; w < kNormBwdWaves; ++w) {
        if (wave == w) {
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                const int vi = lane + kWave * i;
                if (vi >= nvec) continue;
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const int col = vi * E + j;
                    const float vw = aw[i][j] + (w > 0 ? colsum[col] : 0.f);
                    const float vb = HB ? ab[i][j] + (w > 0 ? colsum[width + col] : 0.f) : 0.f;
                    if (w < kNormBwdWaves - 1) {
                        colsum[col] = vw;
                        if (HB) colsum[width + col] = vb;
                    } else {
                        pw[col] = vw;
                        if (HB) pw[width + col] = vb;
                    }
                }
            }
        }
        __syncthreads();
    }
}

// dw (and db) from the blocks' partial rows, in two levels in one launch: workgroup
// (chunk of 64 columns, part p) adds the blocks of its part (blocks p * per .. + per - 1):
// 16 lanes per column over them (lane l takes blocks l, l + 16, ..., all loaded in one
// round: a loop of dependent rounds made one-level sums as long as the row pass), their
// sums added in lane order, and stores the part's sums with device-scope stores; the last
// of a chunk's kColsumParts workgroups to count itself in (a split counter, zero between
// calls) adds the parts in part order and clears the word.  Eight parts: with one workgroup per
// chunk reading every block's partial, C5 LayerNorm's backward took 19.0 us, not 17.9.
constexpr int kColsumRowsPerLane = 32;  // norm_bwd_blocks() <= 16 * this
constexpr int kColsumParts = 8;
__global__ __launch_bounds__(1024) void norm_bwd_colsum_parts(const float* part, float* lvl, unsigned long long* ctr,
                                                              void* dw, void* db, int w_dtype, int b_dtype,
                                                              int nblocks, int width) {
    __shared__ float red[2][16][64];
    __shared__ int last;
    const int cx = blockIdx.x, pi = blockIdx.y;
    const int c = cx * 64 + (threadIdx.x & 63), l = threadIdx.x >> 6;
    const int per = (nblocks + kColsumParts - 1) / kColsumParts;
    const int b0 = pi * per, b1 = min(nblocks, b0 + per);
    float sw = 0.f, sb = 0.f;
    if (c < width) {
        constexpr int KMAX = kColsumRowsPerLane / kColsumParts + 1;  // per <= 16 * KMAX
        float vw[KMAX], vb[KMAX];
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            const int b = min(b0 + l + 16 * i, nblocks - 1);
            vw[i] = part[static_cast<int64_t>(b) * 2 * width + c];
            vb[i] = db ? part[static_cast<int64_t>(b) * 2 * width + width + c] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < KMAX; ++i) {
            if (b0 + l + 16 * i < b1) {
                sw += vw[i];
                sb += vb[i];
            }
        }
    }
    red[0][l][threadIdx.x & 63] = sw;
    red[1][l][threadIdx.x & 63] = sb;
    __syncthreads();
    if (l == 0 && c < width) {
        float tw = 0.f, tb = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            tw += red[0][i][threadIdx.x];
            tb += red[1][i][threadIdx.x];
        }
        uint32_t* lp = reinterpret_cast<uint32_t*>(lvl + static_cast<int64_t>(pi) * 2 * width);
        __hip_atomic_store(lp + c, __builtin_bit_cast(uint32_t, tw), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(lp + width + c, __builtin_bit_cast(uint32_t, tb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!ctr) return;  // the parts are added by norm_bwd_colsum_finish
    // The part's sums are complete device-wide before it counts itself in.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long n = __hip_atomic_fetch_add(ctr + cx, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
        const bool is_last = n == static_cast<unsigned long long>(kColsumParts);
        if (is_last) __hip_atomic_store(ctr + cx, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = is_last ? 1 : 0;
    }
    __syncthreads();
    if (!last || l != 0 || c >= width) return;
    float tw = 0.f, tb = 0.f;
#pragma unroll
    for (int q = 0; q < kColsumParts; ++q) {
        const uint32_t* lp = reinterpret_cast<const uint32_t*>(lvl + static_cast<int64_t>(q) * 2 * width);
        tw += __builtin_bit_cast(float, __hip_atomic_load(lp + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        tb += __builtin_bit_cast(float, __hip_atomic_load(lp + width + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    if (dw) store_any(dw, w_dtype, c, tw);
    if (db) store_any(db, b_dtype, c, tb);
}

// Second launch of the two-level column sums when no split counters are free: the same
// additions in the same order as norm_bwd_colsum_parts' last workgroup.
__global__ __launch_bounds__(256) void norm_bwd_colsum_finish(const float* lvl, void* dw, void* db, int w_dtype,
                                                              int b_dtype, int width) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= width) return;
    float tw = 0.f, tb = 0.f;
#pragma unroll
    for (int q = 0; q < kColsumParts; ++q) {
        tw += lvl[static_cast<int64_t>(q) * 2 * width + c];
        tb += lvl[static_cast<int64_t>(q) * 2 * width + width + c];
    }
    if (dw) store_any(dw, w_dtype, c, tw);
    if (db) store_any(db, b_dtype, c, tb);
}

// Blocks of the one-pass backward: about two per CU, whole wavefront rows each.
int64_t norm_bwd_blocks(int64_t rows) {
    return std::max<int64_t>(1, std::min<int64_t>(512, ceil_div(rows, kNormBwdWaves)));
}
int64_t norm_bwd_rows_per_block(int64_t rows) {
    return ceil_div(ceil_div(rows, norm_bwd_blocks(rows)), kNormBwdWaves) * kNormBwdWaves;
}
// Workspace floats of the one-pass backward: the blocks' partial rows, then the column
// sums' per-part rows.
int64_t norm_bwd_part_floats(int64_t rows, int64_t width) {
    return (2 * norm_bwd_blocks(rows) + 2 * kColsumParts) * width;
}

// The vector lanes the one-pass backward needs for a row (0 when it does not apply: the
// row must be whole 16-byte vectors, 16-byte aligned, at most 4 vectors per lane: more
// would take the column sums past the register file).
int norm_bwd_vpl(const void* dy, const void* x, const void* dx, const void* w, int64_t width, int x_dtype, int w_dtype,
                 int rows_align) {
    const int xs = dtype_size(x_dtype);
    if (xs == 0 || width % (16 / xs) != 0 || !aligned(dy, 16) || !aligned(x, 16) || !aligned(dx, 16)) return 0;
    if (w && !(w_dtype == x_dtype || w_dtype == KMI_F32)) return 0;
    if (w && !aligned(w, 16 / xs * dtype_size(w_dtype))) return 0;
    (void)rows_align;
    const int64_t nvec = width / (16 / xs);
    const int64_t need = ceil_div(nvec, kWave);
    if (need > 4) return 0;
    int n = 1;
    while (n < need) n <<= 1;
    return n;
}

template <typename T, typename W, bool LAYER>
hipError_t launch_norm_bwd(const void* dy, const void* x, const float* mean, const float* rstd, const void* w,
                           void* dx, void* dw, void* db, int64_t rows, int width, int vpl, int w_dtype, int b_dtype,
                           float* part, hipStream_t s) {
    const int64_t nb = norm_bwd_blocks(rows), rpb = norm_bwd_rows_per_block(rows);
    const size_t lds = static_cast<size_t>(2) * width * sizeof(float);
    const bool hb = db != nullptr;
    // Column sums only when dw or db is asked for: the caller's workspace may be absent.
    if (!dw && !db) part = nullptr;
    auto* dyp = static_cast<const T*>(dy);
    auto* xp = static_cast<const T*>(x);
    auto* wp = static_cast<const W*>(w);
    auto* dxp = static_cast<T*>(dx);
#define KMI_BWD_LAUNCH(N, HWV, HBV)                                                                        \
    hipLaunchKernelGGL((norm_bwd_rows<T, W, LAYER, N, HWV, HBV>), dim3(static_cast<unsigned>(nb)), dim3(kNormBwdWaves * kWave), \
                       lds, s, dyp, xp, mean, rstd, wp, dxp, part, rows, width, rpb)
#define KMI_BWD_CASE(N)                                  \
    case N:                                              \
        if (w && hb) KMI_BWD_LAUNCH(N, true, true);      \
        else if (w) KMI_BWD_LAUNCH(N, true, false);      \
        else if (hb) KMI_BWD_LAUNCH(N, false, true);     \
        else KMI_BWD_LAUNCH(N, false, false);            \
        break;
    switch (vpl) {
        KMI_BWD_CASE(1)
        KMI_BWD_CASE(2)
        KMI_BWD_CASE(4)
        default: return hipErrorInvalidValue;
    }
#undef KMI_BWD_CASE
#undef KMI_BWD_LAUNCH
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || (!dw && !db)) return err;
    const int64_t chunks = ceil_div(width, 64);
    float* lvl = part + 2 * nb * width;
    unsigned long long* ctr = fwd::decode_counters(s, chunks);
    hipLaunchKernelGGL(norm_bwd_colsum_parts, dim3(static_cast<unsigned>(chunks), kColsumParts), dim3(1024), 0, s, part,
                       lvl, ctr, dw, db, w_dtype, b_dtype, static_cast<int>(nb), width);
    if (!ctr)
        hipLaunchKernelGGL(norm_bwd_colsum_finish, dim3(static_cast<unsigned>(ceil_div(width, 256))), dim3(256), 0, s,
                           lvl, dw, db, w_dtype, b_dtype, width);
    return hipGetLastError();
}

template <bool LAYER>
hipError_t norm_bwd_dispatch(const void* dy, const void* x, const float* mean, const float* rstd, const void* w,
                             void* dx, void* dw, void* db, int64_t rows, int width, int vpl, int x_dtype, int w_dtype,
                             int b_dtype, float* part, hipStream_t s) {
    const bool pf32 = w && w_dtype == KMI_F32;
    switch (x_dtype) {
        case KMI_BF16:
            return pf32 ? launch_norm_bwd<bf16, float, LAYER>(dy, x, mean, rstd, w, dx, dw, db, rows, width, vpl,
                                                              w_dtype, b_dtype, part, s)
                        : launch_norm_bwd<bf16, bf16, LAYER>(dy, x, mean, rstd, w, dx, dw, db, rows, width, vpl,
                                                             w_dtype, b_dtype, part, s);
        case KMI_F16:
            return pf32 ? launch_norm_bwd<f16, float, LAYER>(dy, x, mean, rstd, w, dx, dw, db, rows, width, vpl,
                                                             w_dtype, b_dtype, part, s)
                        : launch_norm_bwd<f16, f16, LAYER>(dy, x, mean, rstd, w, dx, dw, db, rows, width, vpl,
                                                           w_dtype, b_dtype, part, s);
        default:
            return launch_norm_bwd<float, float, LAYER>(dy, x, mean, rstd, w, dx, dw, db, rows, width, vpl, w_dtype,
                                                        b_dtype, part, s);
    }
}

template <bool LAYER>
int norm_fwd(const char* name, const void* x, const void* w, const void* b, void* y,
             float* mean, float* rstd, int64_t rows, int64_t width, int x_dtype,
             int w_dtype, int b_dtype, double eps, hipStream_t stream) {
    const int xs = dtype_size(x_dtype);
    if (xs == 0) return fail(KMI_EINVAL, std::string(name) + ": x dtype must be BF16, F16 or F32");
    if ((w && dtype_size(w_dtype) == 0) || (b && dtype_size(b_dtype) == 0))
        return fail(KMI_EINVAL, std::string(name) + ": weight / bias dtype must be BF16, F16 or F32");
    if (rows < 0 || width < 0) return fail(KMI_EINVAL, std::string(name) + ": negative size");
    if (rows == 0) return KMI_OK;
    if (width == 0) return fail(KMI_EINVAL, std::string(name) + ": empty rows");
    if (!x || !y) return fail(KMI_EINVAL, std::string(name) + ": null x or y");
    if (rows > (int64_t{1} << 31) * 4 || width > (int64_t{1} << 30))
        return fail(KMI_EUNSUPPORTED, std::string(name) + ": too many rows or too wide");
    const float e = static_cast<float>(eps);
    const int epv = 16 / xs;
    const int64_t nvec = width / epv;
    const int64_t vpl_need = ceil_div(nvec, kWave);
    // Weight and bias share one type on the fast path: x's own type or fp32.
    const bool params_ok =
        (!w || w_dtype == x_dtype || w_dtype == KMI_F32) &&
        (!b || b_dtype == x_dtype || b_dtype == KMI_F32) &&
        (!w || !b || w_dtype == b_dtype);
    const int pdt = w ? w_dtype : (b ? b_dtype : x_dtype);
    const int64_t pbytes = static_cast<int64_t>(epv) * dtype_size(pdt);
    // Rows of up to 4 vectors per lane take one wavefront each; wider rows (up to 8
    // vectors per thread of a 256-thread block) one block each.
    const int64_t vpt_need = ceil_div(nvec, 256);
    const bool vec_ok = width % epv == 0 && params_ok && aligned(x, 16) && aligned(y, 16) &&
                        aligned(w, pbytes) && aligned(b, pbytes);
    const bool by_wave = vec_ok && vpl_need <= 4;
    const bool by_block = vec_ok && !by_wave && vpt_need <= 8;
    hipError_t err;
    if (by_wave || by_block) {
        int n = 1;
        while (n < (by_wave ? vpl_need : vpt_need)) n <<= 1;
        const int wd = static_cast<int>(width);
        const bool pf32 = pdt == KMI_F32;
        auto go = [&](auto tx, auto tw) {
            typedef decltype(tx) TX;
            typedef decltype(tw) TW;
            return by_wave ? launch_wave<TX, TW, LAYER>(x, w, b, y, mean, rstd, rows, wd, e, n, stream)
                           : launch_block<TX, TW, LAYER>(x, w, b, y, mean, rstd, rows, wd, e, n, stream);
        };
        switch (x_dtype) {
            case KMI_BF16: err = pf32 ? go(bf16{}, float{}) : go(bf16{}, bf16{}); break;
            case KMI_F16: err = pf32 ? go(f16{}, float{}) : go(f16{}, f16{}); break;
            default: err = go(float{}, float{});
        }
    } else {
        hipLaunchKernelGGL((norm_rows_generic<LAYER>), block_grid(rows),
                           dim3(256), 0, stream, x, w, b, y, mean, rstd, rows, width, x_dtype,
                           w_dtype, b_dtype, e);
        err = hipGetLastError();
    }
    return hip_status(err, name);
}

}  // namespace
}  // namespace kmi

extern "C" int kmi_layer_norm_fwd(const void* x, const void* weight, const void* bias,
                                  void* y, float* mean, float* rstd, int64_t rows,
                                  int64_t width, int32_t x_dtype, int32_t w_dtype,
                                  int32_t b_dtype, double eps, void* stream) {
    return kmi::norm_fwd<true>("kmi_layer_norm_fwd", x, weight, bias, y, mean, rstd, rows,
                               width, x_dtype, w_dtype, b_dtype, eps,
                               static_cast<hipStream_t>(stream));
}

extern "C" int kmi_rms_norm_fwd(const void* x, const void* weight, const void* bias,
                                void* y, float* rstd, int64_t rows, int64_t width,
                                int32_t x_dtype, int32_t w_dtype, int32_t b_dtype,
                                double eps, void* stream) {
    return kmi::norm_fwd<false>("kmi_rms_norm_fwd", x, weight, bias, y, nullptr, rstd,
                                rows, width, x_dtype, w_dtype, b_dtype, eps,
                                static_cast<hipStream_t>(stream));
}

extern "C" int kmi_rms_norm_bwd_workspace_bytes(int64_t rows, int64_t width, size_t* bytes) {
    using namespace kmi;
    if (!bytes) return fail(KMI_EINVAL, "kmi_rms_norm_bwd_workspace_bytes: null bytes");
    if (rows < 0 || width < 0) return fail(KMI_EINVAL, "kmi_rms_norm_bwd_workspace_bytes: negative size");
    // Enough for either path: the one-pass kernel's per-block partial rows or the
    // row-chunk column sums of the element path.
    const int64_t n = std::max(rms_bwd_chunks(rows) * width, norm_bwd_part_floats(rows, width));
    *bytes = rows == 0 ? 0 : static_cast<size_t>(n) * sizeof(float);
    return KMI_OK;
}

extern "C" int kmi_layer_norm_bwd_workspace_bytes(int64_t rows, int64_t width, size_t* bytes) {
    using namespace kmi;
    if (!bytes) return fail(KMI_EINVAL, "kmi_layer_norm_bwd_workspace_bytes: null bytes");
    if (rows < 0 || width < 0) return fail(KMI_EINVAL, "kmi_layer_norm_bwd_workspace_bytes: negative size");
    *bytes = rows == 0 ? 0 : static_cast<size_t>(norm_bwd_part_floats(rows, width)) * sizeof(float);
    return KMI_OK;
}

extern "C" int kmi_layer_norm_bwd(const void* dy, const void* x, const float* mean, const float* rstd,
                                  const void* weight, void* dx, void* dweight, void* dbias, int64_t rows,
                                  int64_t width, int32_t x_dtype, int32_t w_dtype, int32_t b_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    using namespace kmi;
    const char* name = "kmi_layer_norm_bwd";
    if (dtype_size(x_dtype) == 0) return fail(KMI_EINVAL, std::string(name) + ": x dtype must be BF16, F16 or F32");
    if ((weight || dweight) && dtype_size(w_dtype) == 0)
        return fail(KMI_EINVAL, std::string(name) + ": weight dtype must be BF16, F16 or F32");
    if (dbias && dtype_size(b_dtype) == 0)
        return fail(KMI_EINVAL, std::string(name) + ": bias dtype must be BF16, F16 or F32");
    if (rows < 0 || width < 0) return fail(KMI_EINVAL, std::string(name) + ": negative size");
    if (rows == 0) return KMI_OK;
    if (width == 0) return fail(KMI_EINVAL, std::string(name) + ": empty rows");
    if (!dy || !x || !mean || !rstd || !dx) return fail(KMI_EINVAL, std::string(name) + ": null dy, x, mean, rstd or dx");
    if (dweight && !weight) return fail(KMI_EINVAL, std::string(name) + ": dweight needs weight");
    if (rows > (int64_t{1} << 40) || width > (int64_t{1} << 30))
        return fail(KMI_EUNSUPPORTED, std::string(name) + ": too many rows or too wide");
    const int vpl = norm_bwd_vpl(dy, x, dx, weight, width, x_dtype, w_dtype, 0);
    if (vpl == 0)
        return fail(KMI_EUNSUPPORTED, std::string(name) + ": rows must be whole 16-byte vectors (16-byte aligned, "
                                                          "at most 256 vectors) with weight in x's dtype or fp32");
    const size_t need = static_cast<size_t>(norm_bwd_part_floats(rows, width)) * sizeof(float);
    if ((dweight || dbias) && (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 4))
        return fail(KMI_EWORKSPACE, std::string(name) + ": workspace missing or smaller than "
                                                        "kmi_layer_norm_bwd_workspace_bytes");
    const hipError_t err =
        norm_bwd_dispatch<true>(dy, x, mean, rstd, weight, dx, dweight, dbias, rows, static_cast<int>(width), vpl,
                                x_dtype, w_dtype, b_dtype, static_cast<float*>(workspace),
                                static_cast<hipStream_t>(stream));
    return hip_status(err, name);
}

extern "C" int kmi_rms_norm_bwd(const void* dy, const void* x, const void* weight, const float* rstd, void* dx,
                                void* dweight, int64_t rows, int64_t width, int32_t x_dtype, int32_t w_dtype,
                                void* workspace, size_t workspace_bytes, void* stream) {
    using namespace kmi;
    const char* name = "kmi_rms_norm_bwd";
    if (dtype_size(x_dtype) == 0) return fail(KMI_EINVAL, std::string(name) + ": x dtype must be BF16, F16 or F32");
    if (weight && dtype_size(w_dtype) == 0)
        return fail(KMI_EINVAL, std::string(name) + ": weight dtype must be BF16, F16 or F32");
    if (rows < 0 || width < 0) return fail(KMI_EINVAL, std::string(name) + ": negative size");
    if (rows == 0) return KMI_OK;
    if (width == 0) return fail(KMI_EINVAL, std::string(name) + ": empty rows");
    if (!dy || !x || !rstd || !dx) return fail(KMI_EINVAL, std::string(name) + ": null dy, x, rstd or dx");
    if (dweight && !weight) return fail(KMI_EINVAL, std::string(name) + ": dweight needs weight");
    if (rows > (int64_t{1} << 31) || width > (int64_t{1} << 30))
        return fail(KMI_EUNSUPPORTED, std::string(name) + ": too many rows or too wide");
    const int64_t chunks = rms_bwd_chunks(rows);
    const size_t need = static_cast<size_t>(std::max(chunks * width, norm_bwd_part_floats(rows, width))) * sizeof(float);
    if (dweight && (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 4))
        return fail(KMI_EWORKSPACE, std::string(name) + ": workspace missing or smaller than "
                                                        "kmi_rms_norm_bwd_workspace_bytes");
    hipStream_t s = static_cast<hipStream_t>(stream);
    float* part = static_cast<float*>(workspace);
    // Whole-vector rows: the one-pass kernel (dy and x read once); otherwise the element
    // path (a dx pass and a column-sum pass).
    const int vpl = norm_bwd_vpl(dy, x, dx, weight, width, x_dtype, w_dtype, 0);
    if (vpl > 0) {
        const hipError_t e1 = norm_bwd_dispatch<false>(dy, x, nullptr, rstd, weight, dx, dweight, nullptr, rows,
                                                       static_cast<int>(width), vpl, x_dtype, w_dtype, 0, part, s);
        return hip_status(e1, name);
    }
    const int wd = static_cast<int>(w_dtype);
    hipError_t err;
    switch (x_dtype) {
        case KMI_BF16: err = launch_rms_bwd<bf16>(dy, x, weight, rstd, dx, dweight, rows, width, wd, part, chunks, s); break;
        case KMI_F16: err = launch_rms_bwd<f16>(dy, x, weight, rstd, dx, dweight, rows, width, wd, part, chunks, s); break;
        default: err = launch_rms_bwd<float>(dy, x, weight, rstd, dx, dweight, rows, width, wd, part, chunks, s);
    }
    return hip_status(err, name);
}
