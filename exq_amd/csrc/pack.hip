// pack.hip -- weight quantisation on the GPU, bit-exact with the reference's
// torch arithmetic (IEEE fp32 division, round-half-to-even).
//
//   INT4 (moe_int4_kernel.py:37-93): per (row, group) scale = max|w| / 7 in
//   fp32 floored at fp32 eps; q = rint(w / scale) clamped to [-8, 7]; nibble
//   q + 8, even k in the low nibble; scale stored as fp16.
//   INT8 (quant_shim.py:84-96 rule): per row scale = max|w| / 127 (floored at
//   fp32 eps); q = rint(w / scale) clamped to [-128, 127]; scale stored fp16.
#include "exq_internal.h"

namespace exq {
namespace {

constexpr float kFp32Eps = 1.1920928955078125e-07f;  // 2^-23

__device__ __forceinline__ void load8(const void* w, int dtype, int64_t i, float v[8]) {
  if (dtype == EXQ_DTYPE_F32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + i);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 q = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + i);
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (dtype == EXQ_DTYPE_BF16) {
        v[2 * j] = bf16_bits_to_f32(d[j] & 0xffffu);
        v[2 * j + 1] = bf16_bits_to_f32(d[j] >> 16);
      } else {
        v[2 * j] = f16_bits_to_f32(d[j] & 0xffffu);
        v[2 * j + 1] = f16_bits_to_f32(d[j] >> 16);
      }
    }
  }
}

__device__ __forceinline__ float load1(const void* w, int dtype, int64_t i) {
  return load_as_f32(w, dtype, i);
}

// One thread per 8 consecutive k; the tpg threads of a group (tpg = g/8, a
// power of two <= 64) reduce max|w| with lane shuffles.
__global__ void __launch_bounds__(256) pack_int4_kernel(const void* __restrict__ w, int dtype,
                                                        int64_t rows, int K, int g, int tpg,
                                                        uint8_t* __restrict__ packed,
                                                        uint16_t* __restrict__ scales) {
  const int cpr = K / 8;  // chunks per row
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool act = tid < rows * cpr;
  const int64_t row = act ? tid / cpr : 0;
  const int c = act ? (int)(tid - row * cpr) : 0;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (act) load8(w, dtype, row * K + (int64_t)c * 8, v);
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
  for (int d = 1; d < tpg; d <<= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  const float scale = fmaxf(m / 7.0f, kFp32Eps);
  if (!act) return;
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float q = rintf(v[j] / scale);
    q = fminf(fmaxf(q, -8.f), 7.f);
    word |= (uint32_t)((int)q + 8) << (4 * j);
  }
  reinterpret_cast<uint32_t*>(packed + row * (K / 2))[c] = word;
  if (c % tpg == 0) scales[row * (K / g) + c / tpg] = (uint16_t)f32_to_f16_bits(scale);
}

// Fallback for group sizes whose chunk count is not a power of two (e.g. the
// K < 128 collapse to g = K): one thread per (row, group), serial over g.
__global__ void __launch_bounds__(256) pack_int4_serial_kernel(
    const void* __restrict__ w, int dtype, int64_t rows, int K, int g,
    uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
  const int ng = K / g;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= rows * ng) return;
  const int64_t row = tid / ng;
  const int grp = (int)(tid - row * ng);
  const int64_t base = row * K + (int64_t)grp * g;
  float m = 0.f;
  for (int k = 0; k < g; ++k) m = fmaxf(m, fabsf(load1(w, dtype, base + k)));
  const float scale = fmaxf(m / 7.0f, kFp32Eps);
  for (int k = 0; k < g; k += 2) {
    float q0 = fminf(fmaxf(rintf(load1(w, dtype, base + k) / scale), -8.f), 7.f);
    float q1 = fminf(fmaxf(rintf(load1(w, dtype, base + k + 1) / scale), -8.f), 7.f);
    packed[(base + k) / 2] = (uint8_t)(((int)q0 + 8) | (((int)q1 + 8) << 4));
  }
  scales[row * ng + grp] = (uint16_t)f32_to_f16_bits(scale);
}

// One work-group per row: max|w| over K, then quantise.
__global__ void __launch_bounds__(256) quant_int8_kernel(const void* __restrict__ w, int dtype,
                                                         int K, int8_t* __restrict__ q,
                                                         uint16_t* __restrict__ scales) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = row * K;
  float m = 0.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) m = fmaxf(m, fabsf(load1(w, dtype, base + k)));
  for (int d = 1; d < 64; d <<= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float scale = fmaxf(m / 127.0f, kFp32Eps);
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const float v = rintf(load1(w, dtype, base + k) / scale);
    q[base + k] = (int8_t)(int)fminf(fmaxf(v, -128.f), 127.f);
  }
  if (threadIdx.x == 0) scales[row] = (uint16_t)f32_to_f16_bits(scale);
}

// Store v (fp32) in the weights' dtype, rounded to nearest even.
__device__ __forceinline__ void store1(void* out, int dtype, int64_t i, float v) {
  if (dtype == EXQ_DTYPE_F32)
    reinterpret_cast<float*>(out)[i] = v;
  else if (dtype == EXQ_DTYPE_BF16)
    reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
  else
    reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_f16_bits(v);
}

// Maximum and clamp that keep NaN, as torch's amax and clamp do (quant_shim.py:
// 92-95): a NaN or infinite weight makes its whole row (INT8) or group (INT4)
// NaN.  fmaxf / fminf alone would return the other operand.
__device__ __forceinline__ float max_keep_nan(float a, float b) {
  return __builtin_isnan(a) ? a : (__builtin_isnan(b) ? b : fmaxf(a, b));
}
__device__ __forceinline__ float clamp_keep_nan(float v, float lo, float hi) {
  return __builtin_isnan(v) ? v : fminf(fmaxf(v, lo), hi);
}

// Fake quantisation (quantise then dequantise in place of the weights):
// INT4 per group of g along the row (a short last group counts as padded with
// zeros), INT8 per row; out = q * scale with the fp32 scale, in the weights'
// dtype.  One wave per (row, group) for INT4 (g <= 512, lanes stride the
// group), one work-group per row for INT8.
// (`out` may alias `w`: each element is read, then written, by one lane.)
__global__ void __launch_bounds__(256) fake_int4_kernel(const void* w, int dtype, int64_t rows,
                                                        int K, int g, void* out) {
  const int ng = (K + g - 1) / g;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= rows * ng) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int64_t row = unit / ng;
  const int k0 = (int)(unit - row * ng) * g;
  const int k1 = k0 + g < K ? k0 + g : K;
  const int64_t base = row * K;
  float m = 0.f;
  for (int k = k0 + lane; k < k1; k += 64) m = max_keep_nan(m, fabsf(load1(w, dtype, base + k)));
  for (int d = 1; d < 64; d <<= 1) m = max_keep_nan(m, __shfl_xor(m, d, 64));
  const float scale = max_keep_nan(m / 7.0f, kFp32Eps);
  for (int k = k0 + lane; k < k1; k += 64) {
    const float q = clamp_keep_nan(rintf(load1(w, dtype, base + k) / scale), -8.f, 7.f);
    store1(out, dtype, base + k, q * scale);
  }
}

__global__ void __launch_bounds__(256) fake_int8_kernel(const void* w, int dtype, int K,
                                                        void* out) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * K;
  float m = 0.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x)
    m = max_keep_nan(m, fabsf(load1(w, dtype, base + k)));
  for (int d = 1; d < 64; d <<= 1) m = max_keep_nan(m, __shfl_xor(m, d, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = max_keep_nan(max_keep_nan(red[0], red[1]), max_keep_nan(red[2], red[3]));
  const float scale = max_keep_nan(m / 127.0f, kFp32Eps);
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const float q = clamp_keep_nan(rintf(load1(w, dtype, base + k) / scale), -128.f, 127.f);
    store1(out, dtype, base + k, q * scale);
  }
}

}  // namespace
}  // namespace exq

using namespace exq;

extern "C" int exq_fake_quant(const void* weights, int dtype, int64_t rows, int64_t K, int bits,
                              int64_t group_size, void* out, exq_stream stream) {
  const char* fn = "exq_fake_quant";
  EXQ_REQUIRE(is_float_dtype(dtype), "%s: dtype must be f32, f16 or bf16", fn);
  EXQ_REQUIRE(bits == 4 || bits == 8, "%s: bits must be 4 or 8 (got %d)", fn, bits);
  EXQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && K >= 1 && K <= INT32_MAX, "%s: bad sizes", fn);
  EXQ_REQUIRE(bits == 8 || (group_size >= 1 && group_size <= 512),
              "%s: group_size=%lld must be in [1, 512]", fn, (long long)group_size);
  if (rows == 0) return EXQ_SUCCESS;
  EXQ_REQUIRE(weights && out, "%s: null pointer", fn);
  hipStream_t s = as_stream(stream);
  if (bits == 4) {
    const int64_t units = rows * cdiv(K, group_size);
    EXQ_REQUIRE(cdiv(units, 4) <= INT32_MAX, "%s: too many groups", fn);
    hipLaunchKernelGGL(fake_int4_kernel, dim3((unsigned)cdiv(units, 4)), dim3(256), 0, s, weights,
                       dtype, rows, (int)K, (int)group_size, out);
  } else {
    hipLaunchKernelGGL(fake_int8_kernel, dim3((unsigned)rows), dim3(256), 0, s, weights, dtype,
                       (int)K, out);
  }
  return check_launch(fn);
}

extern "C" int exq_pack_int4(const void* weights, int dtype, int64_t rows, int64_t K,
                             int64_t group_size, uint8_t* packed, uint16_t* scales,
                             exq_stream stream) {
  const char* fn = "exq_pack_int4";
  EXQ_REQUIRE(is_float_dtype(dtype), "%s: dtype must be f32, f16 or bf16", fn);
  EXQ_REQUIRE(rows >= 0 && K >= 2 && K % 2 == 0 && K <= INT32_MAX,
              "%s: K=%lld must be even and positive", fn, (long long)K);
  EXQ_REQUIRE(group_size >= 2, "%s: group_size=%lld", fn, (long long)group_size);
  const int64_t g = K < group_size ? K : group_size;  // K < g collapses to one group
  EXQ_REQUIRE(K % g == 0 && g % 2 == 0, "%s: K=%lld must be divisible by group_size=%lld", fn,
              (long long)K, (long long)g);
  if (rows == 0) return EXQ_SUCCESS;
  EXQ_REQUIRE(weights && packed && scales, "%s: null pointer", fn);
  EXQ_REQUIRE(cdiv(rows * (K / 2), 256) <= INT32_MAX, "%s: %lld x %lld weights is too large", fn,
              (long long)rows, (long long)K);
  const int tpg = (int)(g / 8);
  const bool fast = g % 8 == 0 && tpg <= 64 && (tpg & (tpg - 1)) == 0 &&
                    ((uintptr_t)weights % 16 == 0) && ((uintptr_t)packed % 4 == 0);
  hipStream_t s = as_stream(stream);
  if (fast) {
    const int64_t threads = rows * (K / 8);
    hipLaunchKernelGGL(pack_int4_kernel, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0, s,
                       weights, dtype, rows, (int)K, (int)g, tpg, packed, scales);
  } else {
    const int64_t threads = rows * (K / g);
    hipLaunchKernelGGL(pack_int4_serial_kernel, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0,
                       s, weights, dtype, rows, (int)K, (int)g, packed, scales);
  }
  return check_launch(fn);
}

extern "C" int exq_quantize_int8(const void* weights, int dtype, int64_t rows, int64_t K,
                                 int8_t* q, uint16_t* scales, exq_stream stream) {
  const char* fn = "exq_quantize_int8";
  EXQ_REQUIRE(is_float_dtype(dtype), "%s: dtype must be f32, f16 or bf16", fn);
  EXQ_REQUIRE(rows >= 0 && rows <= INT32_MAX && K >= 1 && K <= INT32_MAX, "%s: bad sizes", fn);
  if (rows == 0) return EXQ_SUCCESS;
  EXQ_REQUIRE(weights && q && scales, "%s: null pointer", fn);
  hipLaunchKernelGGL(quant_int8_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream),
                     weights, dtype, (int)K, q, scales);
  return check_launch(fn);
}
