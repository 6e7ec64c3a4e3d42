// dev_util.h -- device helpers shared by the decode kernels (gfx950 only):
// MFMA wrappers, exact INT4 / INT8 -> 16-bit float conversion, k-order
// permutations, buffer resources with out-of-range zero loads, LDS DMA and
// wave-local waits.  Not part of the C ABI.
#pragma once

#include "exq_internal.h"

namespace exq {
namespace dev {

constexpr int CPOL_SC1 = 16;  // cache-policy bits: sc1 (agent-coherent access)

template <bool BF>
__device__ __forceinline__ f32x4_t dmfma(const uint4& a, const uint4& b, f32x4_t c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// 8 packed nibbles (k offsets 0..7) -> 8 exact 16-bit floats (base + nibble)
// in k order (0,4,1,5,2,6,3,7).  `mask` (0x000F000F) is wave-uniform and
// `magic` (the base's exponent bits) lives in a VGPR, so each pair is one
// v_and_or_b32 plus a shift.
__device__ __forceinline__ uint4 ddeq4(uint32_t p, uint32_t mask, uint32_t magic) {
  uint4 o;
  o.x = (p & mask) | magic;
  o.y = ((p >> 4) & mask) | magic;
  o.z = ((p >> 8) & mask) | magic;
  o.w = ((p >> 12) & mask) | magic;
  return o;
}

// 4 int8 (k offsets 0..3) -> 4 exact 16-bit floats of value (q + 128), k order.
template <bool BF>
__device__ __forceinline__ uint2 ddeq8(uint32_t p) {
  const uint32_t u = p ^ 0x80808080u;
  const float f0 = (float)(u & 0xffu), f1 = (float)((u >> 8) & 0xffu);
  const float f2 = (float)((u >> 16) & 0xffu), f3 = (float)(u >> 24);
  uint2 o;
  if constexpr (BF) {
    o.x = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
    o.y = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
  } else {
    o.x = f32_to_f16_bits(f0) | (f32_to_f16_bits(f1) << 16);
    o.y = f32_to_f16_bits(f2) | (f32_to_f16_bits(f3) << 16);
  }
  return o;
}

// Natural k order (x0..x7) -> INT4 pairing order (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ uint4 dperm(const uint4& v) {
  uint4 o;
  o.x = (v.x & 0xffffu) | (v.z << 16);
  o.y = (v.x >> 16) | (v.z & 0xffff0000u);
  o.z = (v.y & 0xffffu) | (v.w << 16);
  o.w = (v.y >> 16) | (v.w & 0xffff0000u);
  return o;
}

// Inverse of dperm: INT4 pairing order -> natural k order.
__device__ __forceinline__ uint4 dperm_inv(const uint4& o) {
  uint4 v;
  v.x = (o.x & 0xffffu) | (o.y << 16);
  v.y = (o.z & 0xffffu) | (o.w << 16);
  v.z = (o.x >> 16) | (o.y & 0xffff0000u);
  v.w = (o.z >> 16) | (o.w & 0xffff0000u);
  return v;
}

// Position of natural k-offset j (0..7) of an 8-group in INT4 pairing order.
__device__ __forceinline__ int pair_pos(int j) { return ((j & 3) << 1) | (j >> 2); }

// Constant B operand holding -base in every element.
template <int TIER, bool BF>
__device__ __forceinline__ uint4 neg_base_operand() {
  // INT4: base 136 (bf16 128+n-8 form) or 1032 (f16); INT8: 128.
  constexpr uint32_t h = TIER == 2 ? (BF ? 0xC308u : 0xE408u) : (BF ? 0xC300u : 0xD800u);
  constexpr uint32_t d = h | (h << 16);
  return uint4{d, d, d, d};
}

template <bool BF>
__device__ __forceinline__ uint32_t to_act_bits(float v) {
  return BF ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// Wave-local waits written as volatile asm with a memory clobber, so the
// compiler moves no memory access across them: LDS written by an LDS DMA
// (global_load_lds) is only ordered by the vmcnt wait, which the compiler
// does not model as a dependency of later LDS reads.
__device__ __forceinline__ void wave_lds_fence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS ops have completed
}

// The builtin wait tells the compiler's own wait insertion that nothing is in
// flight any more (so it adds no waits of its own for older loads later);
// the empty asm keeps memory accesses on their side of it.
__device__ __forceinline__ void wait_vm_all() {
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): loads, stores and LDS DMA have landed
  asm volatile("" ::: "memory");
}

typedef void __attribute__((address_space(3)))* lptr_t;
typedef const void __attribute__((address_space(1)))* gptr_t;

// 16 bytes per lane from buffer `r` at byte offset `voff` into LDS at
// lds + 16 * lane (buffer_load_dwordx4 ... lds); `lds` is wave-uniform.  The
// builtin exists only for the device target.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, int voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)lds, 16, voff, 0, 0, 0);
#endif
}

// The same with the nontemporal hint (`nt`): for bytes read once, whose lines
// need not stay in the caches.
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t r, unsigned char* lds, int voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)lds, 16, voff, 0, 0, 2);
#endif
}

// 4 bytes per lane into LDS at lds + 4 * lane (buffer_load_dword ... lds).
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, unsigned char* lds, int voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)lds, 4, voff, 0, 0, 0);
#endif
}

template <int N>
__device__ __forceinline__ void wait_vm_le() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Buffer resource over `bytes` bytes at `base` (gfx9 word 3): loads beyond
// the range return zero instead of touching other memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// A byte offset past every resource that a per-lane out-of-range access uses
// (group scales of one expert, the partial rows; the host keeps both below
// it): such a lane reads zero without a memory access, while the resource
// itself stays wave-uniform.  (A per-lane choice of resource would make the
// compiler loop over the distinct values, one load per iteration.)
constexpr int OOB_OFF = 0x7ffffff0;

// Wave-uniform copies of values the compiler cannot prove uniform, so that
// buffer offsets and resource choices stay in scalar registers.
__device__ __forceinline__ bool uni_b(bool v) { return __builtin_amdgcn_readfirstlane((int)v) != 0; }
__device__ __forceinline__ int uni_i(int v) { return __builtin_amdgcn_readfirstlane(v); }


// Index (0..63) of the q-th set bit of a 64-bit mask (q < popcount).
__device__ __forceinline__ int nth_set_bit(uint64_t m, int q) {
  int base = 0;
  uint32_t w = (uint32_t)m;
  const int c = __popc(w);
  if (q >= c) {
    q -= c;
    w = (uint32_t)(m >> 32);
    base = 32;
  }
#pragma unroll
  for (int half = 16; half >= 1; half >>= 1) {
    const uint32_t lo = w & ((1u << half) - 1u);
    const int cl = __popc(lo);
    if (q >= cl) {
      q -= cl;
      w >>= half;
      base += half;
    } else {
      w = lo;
    }
  }
  return base;
}

}  // namespace dev
}  // namespace exq
