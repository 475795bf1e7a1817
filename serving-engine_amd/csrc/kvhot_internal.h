// Shared device types/helpers and host-side error plumbing for libkvhot.
// gfx950 (CDNA4) only: wave64, MFMA 16x16x32 bf16/f16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/kvhot.h"

namespace kvhot {

// ---------------------------------------------------------------- host side --

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const std::string& msg);
void clear_error();

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(static_cast<int>(e),
                     std::string(what) + ": " + hipGetErrorString(e));
  }
  return 0;
}

inline int64_t dtype_size(int dtype) {
  switch (dtype) {
    case KVHOT_F32: return 4;
    case KVHOT_F16: return 2;
    case KVHOT_BF16: return 2;
    default: return 0;
  }
}

// -------------------------------------------------------------- device side --

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Element-type traits: 16-bit MFMA element types carry their 16x16x32 and
// 16x16x16 MFMAs and their float conversions.
struct BF16 {
  using storage = uint16_t;
  __device__ static inline float to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  // Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
  __device__ static inline uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  __device__ static inline f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
        __builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
};

struct F16 {
  using storage = uint16_t;
  __device__ static inline float to_float(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
  }
  __device__ static inline uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  __device__ static inline f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(
        __builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};

struct F32 {
  using storage = float;
  __device__ static inline float to_float(float f) { return f; }
  __device__ static inline float from_float(float f) { return f; }
};

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace kvhot
