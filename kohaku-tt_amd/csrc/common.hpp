// Shared device helpers of the gfx950 kernels: element types, 16-byte vectors,
// wavefront reductions and the status / error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/kohakutt_amd.h"

namespace kmi {

constexpr int kWave = 64;

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Raw buffer resource over [base, base + bytes) (stride 0, dword data): vector loads at
// offsets at or past `bytes` return zeros.  The descriptor lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Bytes from the first of `rows` rows at `stride` bytes to the end of the last one's
// `row_bytes` of data (0 for no rows).  Ranges built from it read every row in full, also
// rows that overlap (a stride below the row's data), and read zeros past the last row.
__device__ __forceinline__ uint32_t rows_extent(int rows, uint32_t stride, uint32_t row_bytes) {
    return rows > 0 ? static_cast<uint32_t>(rows - 1) * stride + row_bytes : 0u;
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
}

// Conversions through float, rounded to nearest even (hardware cvt on gfx950).
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(f16 x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return static_cast<f16>(x); }

// Sum / max over the 64 lanes of a wavefront (butterfly: every lane gets the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// ---------------------------------------------------------------- attention masks
//
// Mask element types are a template parameter of the attention kernels (no mask code in
// the mask-free variants).  A mask value becomes a logit offset clamped at the
// reference's masked logit -5e5 (ktt_flash/program.cpp:912-919, varlen_plan.hpp:17):
// bool keep -> 0, drop -> -5e5; float masks max(x, -5e5) (-inf and NaN -> -5e5).  A key
// at -5e5 is "masked": it gets exactly zero weight when its row keeps any key, and a row
// whose every key is masked is the softmax over its raw scores.
constexpr float kMaskedLogit = -5e5f;

enum MaskKind { MK_NONE = 0, MK_BOOL = 1, MK_BF16 = 2, MK_F16 = 3, MK_F32 = 4 };

// The raw element type a mask kind is loaded as.
template <int MK>
struct MaskRaw {
    typedef float type;
};
template <>
struct MaskRaw<MK_BOOL> {
    typedef uint8_t type;
};
template <>
struct MaskRaw<MK_BF16> {
    typedef uint16_t type;
};
template <>
struct MaskRaw<MK_F16> {
    typedef uint16_t type;
};

// A loaded mask element in logit units, clamped at the masked logit; a NaN entry is a
// masked key.  NaN is recognised from the bits: the attention kernels are compiled with
// -fno-honor-nans, under which a floating-point NaN test (or fmaxf's NaN rule) may be
// folded away.
template <int MK, typename R>
__device__ __forceinline__ float mask_logit_of(R raw) {
    if constexpr (MK == MK_BOOL) {
        return raw ? 0.f : kMaskedLogit;
    } else if constexpr (MK == MK_BF16) {
        const uint32_t mag = __builtin_bit_cast(uint16_t, raw) & 0x7fffu;
        const float v = fmaxf(static_cast<float>(__builtin_bit_cast(bf16, raw)), kMaskedLogit);
        return mag > 0x7f80u ? kMaskedLogit : v;
    } else if constexpr (MK == MK_F16) {
        const uint32_t mag = __builtin_bit_cast(uint16_t, raw) & 0x7fffu;
        const float v = fmaxf(static_cast<float>(__builtin_bit_cast(f16, raw)), kMaskedLogit);
        return mag > 0x7c00u ? kMaskedLogit : v;
    } else {
        const uint32_t mag = __builtin_bit_cast(uint32_t, raw) & 0x7fffffffu;
        const float v = fmaxf(static_cast<float>(raw), kMaskedLogit);
        return mag > 0x7f800000u ? kMaskedLogit : v;
    }
}

// The mask kind of a kmi_dtype code (MK_NONE for none).
inline int mask_kind_of(int32_t mask_mode, int32_t mask_dtype) {
    if (mask_mode == KMI_MASK_NONE) return MK_NONE;
    switch (mask_dtype) {
        case KMI_BOOL: return MK_BOOL;
        case KMI_BF16: return MK_BF16;
        case KMI_F16: return MK_F16;
        default: return MK_F32;
    }
}

// Head dims: the kernels take multiples of 8 up to 256 and pad them to DP, a whole number
// of 32-wide MFMA blocks (the padded columns hold zeros in registers; no memory past the
// head dim is read or written).
inline bool head_dim_supported(int64_t d) { return d >= 8 && d <= 256 && d % 8 == 0; }
inline int padded_head_dim(int64_t d) {
    if (d <= 32) return 32;
    if (d <= 64) return 64;
    if (d <= 96) return 96;
    if (d <= 128) return 128;
    if (d <= 192) return 192;
    return 256;
}

// Error plumbing of the C ABI (defined in capi.cpp).
int fail(int status, const std::string& message);
int hip_status(hipError_t err, const char* what);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace kmi
