// exq_common.h -- shared host/device helpers of libexq_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "exq_hip.h"

namespace exq {

// ---------------------------------------------------------------------------
// Host-side status handling.  Messages are thread-local so concurrent callers
// on different threads do not clobber each other.
// ---------------------------------------------------------------------------
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define EXQ_REQUIRE(cond, ...)                                                   \
  do {                                                                           \
    if (!(cond)) return ::exq::set_error(EXQ_ERROR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define EXQ_REQUIRE_SUPPORTED(cond, ...)                                   \
  do {                                                                     \
    if (!(cond)) return ::exq::set_error(EXQ_ERROR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)

// Check the launch that was just enqueued.
int check_launch(const char* what);

inline hipStream_t as_stream(exq_stream s) { return reinterpret_cast<hipStream_t>(s); }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

inline bool is_float_dtype(int d) {
  return d == EXQ_DTYPE_F32 || d == EXQ_DTYPE_F16 || d == EXQ_DTYPE_BF16;
}
inline bool is_act_dtype(int d) { return d == EXQ_DTYPE_F16 || d == EXQ_DTYPE_BF16; }
inline bool is_index_dtype(int d) { return d == EXQ_DTYPE_I32 || d == EXQ_DTYPE_I64; }
inline int dtype_bytes(int d) {
  switch (d) {
    case EXQ_DTYPE_F32: case EXQ_DTYPE_I32: return 4;
    case EXQ_DTYPE_F16: case EXQ_DTYPE_BF16: return 2;
    case EXQ_DTYPE_I64: return 8;
    default: return 1;
  }
}

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// Round-to-nearest-even float -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load element i of a float-typed array of runtime dtype as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == EXQ_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  uint32_t b = reinterpret_cast<const uint16_t*>(p)[i];
  return dtype == EXQ_DTYPE_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}
__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float v) {
  if (dtype == EXQ_DTYPE_F32) {
    reinterpret_cast<float*>(p)[i] = v;
  } else {
    uint32_t b = dtype == EXQ_DTYPE_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)b;
  }
}
__device__ __forceinline__ int64_t load_index(const void* p, int dtype, int64_t i) {
  return dtype == EXQ_DTYPE_I64 ? reinterpret_cast<const int64_t*>(p)[i]
                                : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

}  // namespace exq
