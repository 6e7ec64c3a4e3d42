// moe_mfma.hip -- grouped expert GEMMs on gfx950 MFMA with in-register
// dequantisation, and the fused / mixed-precision MoE layer entry points.
//
// Work decomposition.  A token group (TgEntry: one expert, <= 64 expert-sorted
// rows) times a block of weight rows is one work-group unit:
//   GATEUP: 16 gate rows j and the 16 matching up rows I + j  (SiLU fused)
//   PLAIN / DOWN: 32 consecutive weight rows
// The four waves of a work-group split the contraction (K) into 128-element
// k-blocks; their fp32 partial tiles are summed through LDS at the end.
//
// Per wave and k-block each lane streams one 16-byte piece of INT4 weights
// (32 consecutive k of one row; 4 lanes cover the row's 64-byte k-block),
// converts nibbles to exact bf16/f16 values (128+n or 1024+n with one
// AND-OR per pair) and feeds v_mfma_f32_16x16x32_{bf16,f16} with the
// activation tile as the 16x32 A operand and the weights as the 32x16 B
// operand.  Because every element is offset by a constant (136 or 1032 for
// INT4, 128 for INT8), the accumulator starts at -c * sum_k x[m, k] (row sums
// computed while staging the activations), and the per-(row, k-block) fp16
// scale is applied to the exact k-block sum in fp32.  Weight bytes are read
// exactly once per token group; activations are staged in LDS per wave.
#include "exq_internal.h"

namespace exq {
namespace {

constexpr int NW = 4;                // waves per work-group
constexpr int NTH = NW * 64;         // threads per work-group
constexpr int WAVE_LDS = 18432;      // LDS bytes per wave
constexpr int XS_OFF = 17408;        // offset of the row-sum area inside a wave's LDS
constexpr int WG_LDS = NW * WAVE_LDS;


template <bool BF>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, f32x4_t c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// 8 packed nibbles (k offsets 0..7) -> 8 exact 16-bit floats of value
// (base + nibble) in k order (0,4,1,5,2,6,3,7).
template <bool BF>
__device__ __forceinline__ uint4 deq_int4(uint32_t p) {
  constexpr uint32_t M = BF ? 0x43004300u : 0x64006400u;
  uint4 o;
  o.x = (p & 0x000F000Fu) | M;
  o.y = ((p >> 4) & 0x000F000Fu) | M;
  o.z = ((p >> 8) & 0x000F000Fu) | M;
  o.w = ((p >> 12) & 0x000F000Fu) | M;
  return o;
}

// 4 int8 (k offsets 0..3) -> 4 exact 16-bit floats of value (q + 128), k order.
template <bool BF>
__device__ __forceinline__ uint2 deq_int8(uint32_t p) {
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

// Activation order used with INT4 weights: (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ uint4 perm_for_int4(const uint4& v) {
  uint4 o;
  o.x = (v.x & 0xffffu) | (v.z << 16);
  o.y = (v.x >> 16) | (v.z & 0xffff0000u);
  o.z = (v.y & 0xffffu) | (v.w << 16);
  o.w = (v.y >> 16) | (v.w & 0xffff0000u);
  return o;
}

template <bool BF>
__device__ __forceinline__ float sum8(const uint4& v) {
  float s = 0.f;
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (BF) {
      s += __uint_as_float(d[i] << 16) + __uint_as_float(d[i] & 0xffff0000u);
    } else {
      s += f16_bits_to_f32(d[i] & 0xffffu) + f16_bits_to_f32(d[i] >> 16);
    }
  }
  return s;
}

template <bool BF>
__device__ __forceinline__ uint32_t to_act_bits(float v) {
  return BF ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// The per-lane weight stream of one wave for one round: up to 32 dwords.
struct WBuf {
  uint4 q[8];
  uint32_t s[8];  // INT4 raw fp16 scale bits, [kbl * 2 + rs]
};

template <int TIER, bool BF, int MODE>
__device__ __forceinline__ void gemm_body(const GemmArgs& a, const TgEntry& te, int blk,
                                          unsigned char* lds) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, kq = lane >> 4;
  const int cnt = te.cnt;
  const int ntiles = (cnt + 15) >> 4;
  const int ntp = ntiles == 3 ? 4 : ntiles;
  constexpr int KG_T = TIER == 2 ? 4 : (TIER == 1 ? 2 : 1);
  const int KG = KG_T < 4 / ntp ? KG_T : 4 / ntp;
  const int xstride = KG * 128 + 8;  // halfs per staged row
  const int nkb = a.K >> 7;
  const int R = NW * KG;
  const int rounds = (nkb + R - 1) / R;

  int rows[2];
  if (MODE == MODE_GATEUP) {
    rows[0] = blk * 16 + r16;
    rows[1] = a.inter + blk * 16 + r16;
  } else {
    rows[0] = blk * 32 + r16;
    rows[1] = rows[0] + 16;
  }
  const int widx = a.w.index ? a.w.index[te.e] : te.e;
  const int64_t ebase = (int64_t)widx * a.n_rows;

  // Row base pointers (bytes for quantised tiers, halfs for BF16).
  const unsigned char* rp[2];
  const uint16_t* sp[2] = {nullptr, nullptr};
  int ngs = 1;
  float rowscale[2] = {1.f, 1.f};
#pragma unroll
  for (int rs = 0; rs < 2; ++rs) {
    const int64_t r = ebase + rows[rs];
    if constexpr (TIER == 2) {
      ngs = a.K / a.group_size;
      rp[rs] = a.w.i4 + r * (a.K / 2);
      sp[rs] = a.w.i4_scales + r * ngs;
    } else if constexpr (TIER == 1) {
      rp[rs] = reinterpret_cast<const unsigned char*>(a.w.i8) + r * a.K;
      rowscale[rs] = f16_bits_to_f32(a.w.i8_scales[r]);
    } else {
      rp[rs] = reinterpret_cast<const unsigned char*>(a.w.bf16 + r * a.K);
    }
  }

  uint16_t* xw = reinterpret_cast<uint16_t*>(lds + wave * WAVE_LDS);
  float* xsw = reinterpret_cast<float*>(lds + wave * WAVE_LDS + XS_OFF);

  auto wave_range = [&](int r, int& kb_lo, int& nmy) {
    const int lo = r * R;
    const int n_r = nkb - lo < R ? nkb - lo : R;
    kb_lo = lo + (wave * n_r) / NW;
    nmy = lo + ((wave + 1) * n_r) / NW - kb_lo;
  };

  auto load_round = [&](int r, WBuf& b) {
    int kb_lo, nmy;
    wave_range(r, kb_lo, nmy);
#pragma unroll
    for (int q = 0; q < KG_T; ++q) {
      if (q < nmy) {
        const int kb = kb_lo + q;
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
          if constexpr (TIER == 2) {
            b.q[q * 2 + rs] = *reinterpret_cast<const uint4*>(rp[rs] + kb * 64 + kq * 16);
            b.s[q * 2 + rs] = sp[rs][(kb * 128) / a.group_size];
          } else if constexpr (TIER == 1) {
            const uint4* src = reinterpret_cast<const uint4*>(rp[rs] + kb * 128 + kq * 32);
            b.q[(q * 2 + rs) * 2 + 0] = src[0];
            b.q[(q * 2 + rs) * 2 + 1] = src[1];
          } else {
            const uint4* src = reinterpret_cast<const uint4*>(rp[rs] + (kb * 128 + kq * 32) * 2);
#pragma unroll
            for (int h = 0; h < 4; ++h) b.q[rs * 4 + h] = src[h];
          }
        }
      }
    }
  };

  auto stage_round = [&](int r) {
    int kb_lo, nmy;
    wave_range(r, kb_lo, nmy);
    const int ppr = nmy * 16;  // 16-byte pieces per staged row
    const int P = cnt * ppr;
    for (int base = 0; base < P; base += 64) {
      const int p = base + lane;
      const bool act = p < P;
      float sum = 0.f;
      int m = 0, kbl = 0;
      if (act) {
        m = p / ppr;
        const int rem = p - m * ppr;
        kbl = rem >> 4;
        const int q = rem & 15;
        const uint16_t* src;
        if constexpr (MODE == MODE_GATEUP) {
          const int slot = a.row_slot[te.pos0 + m];
          src = a.x + (int64_t)(slot / a.slot_div) * a.x_stride;
        } else {
          src = a.x + (int64_t)(te.pos0 + m) * a.x_stride;
        }
        uint4 v = *reinterpret_cast<const uint4*>(src + (kb_lo + kbl) * 128 + q * 8);
        sum = sum8<BF>(v);
        if constexpr (TIER == 2) v = perm_for_int4(v);
        *reinterpret_cast<uint4*>(xw + m * xstride + kbl * 128 + q * 8) = v;
      }
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      sum += __shfl_xor(sum, 4, 64);
      sum += __shfl_xor(sum, 8, 64);
      if (act && (lane & 15) == 0) xsw[kbl * 64 + m] = sum;
    }
  };

  f32x4_t tot0[4], tot1[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    tot0[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tot1[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  constexpr float CORR = TIER == 2 ? (BF ? -136.f : -1032.f) : (TIER == 1 ? -128.f : 0.f);

  auto compute_round = [&](int r, const WBuf& b) {
    int kb_lo, nmy;
    wave_range(r, kb_lo, nmy);
#pragma unroll
    for (int q = 0; q < KG_T; ++q) {
      if (q < nmy) {
        uint4 bf[2][4];
        float sc[2] = {1.f, 1.f};
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
          if constexpr (TIER == 2) {
            const uint4 w = b.q[q * 2 + rs];
            bf[rs][0] = deq_int4<BF>(w.x);
            bf[rs][1] = deq_int4<BF>(w.y);
            bf[rs][2] = deq_int4<BF>(w.z);
            bf[rs][3] = deq_int4<BF>(w.w);
            sc[rs] = f16_bits_to_f32(b.s[q * 2 + rs]);
          } else if constexpr (TIER == 1) {
            const uint4 w0 = b.q[(q * 2 + rs) * 2 + 0], w1 = b.q[(q * 2 + rs) * 2 + 1];
            uint2 d0 = deq_int8<BF>(w0.x), d1 = deq_int8<BF>(w0.y);
            uint2 d2 = deq_int8<BF>(w0.z), d3 = deq_int8<BF>(w0.w);
            uint2 d4 = deq_int8<BF>(w1.x), d5 = deq_int8<BF>(w1.y);
            uint2 d6 = deq_int8<BF>(w1.z), d7 = deq_int8<BF>(w1.w);
            bf[rs][0] = uint4{d0.x, d0.y, d1.x, d1.y};
            bf[rs][1] = uint4{d2.x, d2.y, d3.x, d3.y};
            bf[rs][2] = uint4{d4.x, d4.y, d5.x, d5.y};
            bf[rs][3] = uint4{d6.x, d6.y, d7.x, d7.y};
          } else {
#pragma unroll
            for (int h = 0; h < 4; ++h) bf[rs][h] = b.q[rs * 4 + h];
          }
        }
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          if (tt < ntiles) {
            f32x4_t init = {0.f, 0.f, 0.f, 0.f};
            if constexpr (TIER != 0) {
              const float4 xs4 =
                  *reinterpret_cast<const float4*>(xsw + q * 64 + tt * 16 + kq * 4);
              init = f32x4_t{CORR * xs4.x, CORR * xs4.y, CORR * xs4.z, CORR * xs4.w};
            }
            f32x4_t acc0 = init, acc1 = init;
            const uint16_t* arow = xw + (tt * 16 + r16) * xstride + q * 128 + kq * 32;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const uint4 av = *reinterpret_cast<const uint4*>(arow + d * 8);
              acc0 = mfma16<BF>(av, bf[0][d], acc0);
              acc1 = mfma16<BF>(av, bf[1][d], acc1);
            }
            if constexpr (TIER == 2) {
              tot0[tt] += sc[0] * acc0;
              tot1[tt] += sc[1] * acc1;
            } else {
              tot0[tt] += acc0;
              tot1[tt] += acc1;
            }
          }
        }
      }
    }
  };

  WBuf bufA, bufB;
  load_round(0, bufA);
  for (int r = 0; r < rounds; r += 2) {
    stage_round(r);
    __syncthreads();
    if (r + 1 < rounds) load_round(r + 1, bufB);
    compute_round(r, bufA);
    __syncthreads();
    if (r + 1 >= rounds) break;
    stage_round(r + 1);
    __syncthreads();
    if (r + 2 < rounds) load_round(r + 2, bufA);
    compute_round(r + 1, bufB);
    __syncthreads();
  }

  // Cross-wave reduction of the K-split partial tiles.
  float4* red = reinterpret_cast<float4*>(lds);  // [NW][4 tiles][2 row sets][64 lanes]
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    if (tt < ntiles) {
      red[((wave * 4 + tt) * 2 + 0) * 64 + lane] =
          float4{tot0[tt][0], tot0[tt][1], tot0[tt][2], tot0[tt][3]};
      red[((wave * 4 + tt) * 2 + 1) * 64 + lane] =
          float4{tot1[tt][0], tot1[tt][1], tot1[tt][2], tot1[tt][3]};
    }
  }
  __syncthreads();
  if (wave < ntiles) {
    const int tt = wave;
    float v0[4] = {0.f, 0.f, 0.f, 0.f}, v1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float4 p0 = red[((w * 4 + tt) * 2 + 0) * 64 + lane];
      const float4 p1 = red[((w * 4 + tt) * 2 + 1) * 64 + lane];
      v0[0] += p0.x; v0[1] += p0.y; v0[2] += p0.z; v0[3] += p0.w;
      v1[0] += p1.x; v1[1] += p1.y; v1[2] += p1.z; v1[3] += p1.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = tt * 16 + kq * 4 + i;
      if (m >= cnt) continue;
      const int pos = te.pos0 + m;
      const float g0 = v0[i] * rowscale[0], g1 = v1[i] * rowscale[1];
      if constexpr (MODE == MODE_GATEUP) {
        uint16_t* mid = reinterpret_cast<uint16_t*>(a.out);
        mid[(int64_t)pos * a.out_stride + blk * 16 + r16] =
            (uint16_t)to_act_bits<BF>(silu_f32(g0) * g1);
      } else if constexpr (MODE == MODE_PLAIN) {
        uint16_t* c = reinterpret_cast<uint16_t*>(a.out);
        c[(int64_t)pos * a.out_stride + rows[0]] = (uint16_t)to_act_bits<BF>(g0);
        c[(int64_t)pos * a.out_stride + rows[1]] = (uint16_t)to_act_bits<BF>(g1);
      } else {
        float* part = reinterpret_cast<float*>(a.out);
        const int slot = a.row_slot[pos];
        part[(int64_t)slot * a.out_stride + rows[0]] = g0;
        part[(int64_t)slot * a.out_stride + rows[1]] = g1;
      }
    }
  }

}

template <bool BF, int MODE>
__global__ void __launch_bounds__(NTH, 2) moe_gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[WG_LDS];
  // Token groups are ordered BF16, INT8, INT4; the BF16 head and the INT4 tail
  // go to the tiled kernels when those run.
  const int lo = a.skip_bf ? a.hdr[2] : 0;
  const int n_tg = (a.skip_i4 ? a.hdr[1] : a.hdr[0]) - lo;
  const int U = n_tg * a.n_blocks;
  // XCD-aware order: work-group i runs on XCD i % 8, so each XCD takes a
  // contiguous range of units and neighbouring blocks of one token group
  // (which share the staged activations) stay in one L2.
  // A grid smaller than 8 * per (when only the INT8 groups are left here)
  // strides over the order.
  const int per = (U + 7) >> 3;
  for (int idx = blockIdx.x; idx < 8 * per; idx += gridDim.x) {
    const int local = idx >> 3;
    const int unit = (idx & 7) * per + local;
    if (unit >= U) continue;
    const int tgi = unit / a.n_blocks;
    const int blk = unit - tgi * a.n_blocks;
    const TgEntry te = a.tg[lo + tgi];
    if (te.tier == 0) {
      gemm_body<0, BF, MODE>(a, te, blk, lds);
    } else if (te.tier == 1) {
      gemm_body<1, BF, MODE>(a, te, blk, lds);
    } else {
      gemm_body<2, BF, MODE>(a, te, blk, lds);
    }
    __syncthreads();  // the staged rows and partial tiles of this unit are dead
  }
}

// out[t, h] = sum_j w[t, j] * partial[t*kp + j, h] over the routed slots that
// were not dropped (shared-expert slots j >= k have weight 1), fp32 in the
// fixed order j = 0..kp-1, rounded once to the activation dtype.  One thread
// per 4 consecutive h.  A separate launch: the kernel boundary makes every
// partial row visible without a device-wide fence in the down kernel.
template <bool BF>
__global__ void __launch_bounds__(256) combine_partials_kernel(
    const float* __restrict__ part, const void* __restrict__ ids, int ids_dtype,
    const void* __restrict__ topk_w, int w_dtype, int T, int k, int kp, int E, int H,
    uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int hq = H >> 2;
  if (idx >= (int64_t)T * hq) return;
  const int t = (int)(idx / hq);
  const int h = (int)(idx - (int64_t)t * hq) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < kp; ++j) {
    float wgt = 1.f;
    if (j < k) {
      const int64_t id = load_index(ids, ids_dtype, (int64_t)t * k + j);
      if (id < 0 || id >= E) continue;
      wgt = load_as_f32(topk_w, w_dtype, (int64_t)t * k + j);
    }
    const float4 pv = *reinterpret_cast<const float4*>(part + ((int64_t)t * kp + j) * H + h);
    acc[0] += wgt * pv.x;
    acc[1] += wgt * pv.y;
    acc[2] += wgt * pv.z;
    acc[3] += wgt * pv.w;
  }
  uint2 o;
  o.x = to_act_bits<BF>(acc[0]) | (to_act_bits<BF>(acc[1]) << 16);
  o.y = to_act_bits<BF>(acc[2]) | (to_act_bits<BF>(acc[3]) << 16);
  *reinterpret_cast<uint2*>(out + (int64_t)t * H + h) = o;
}

template <int MODE>
int launch_gemm(bool bf, const GemmArgs& a, int64_t units_cap, hipStream_t s) {
  int64_t grid = 8 * cdiv(units_cap, 8);
  // With the tiled kernels running, only INT8 groups (if any) are left here:
  // a resident-sized grid strides over them instead of launching the cap.
  if ((a.skip_i4 || a.skip_bf) && grid > 2048) grid = 2048;
  if (grid <= 0) return EXQ_SUCCESS;
  if (grid > INT32_MAX)
    return set_error(EXQ_ERROR_UNSUPPORTED, "moe_gemm: grid of %lld work-groups too large",
                     (long long)grid);
  if (bf)
    hipLaunchKernelGGL((moe_gemm_kernel<true, MODE>), dim3((unsigned)grid), dim3(NTH), 0, s, a);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<false, MODE>), dim3((unsigned)grid), dim3(NTH), 0, s, a);
  return check_launch("moe_gemm_kernel");
}

// ---- measurement hook ----------------------------------------------------------
thread_local hipEvent_t g_stage_events[4] = {nullptr, nullptr, nullptr, nullptr};
thread_local bool g_stage_events_set = false;

int record_stage(int i, hipStream_t s) {
  if (!g_stage_events_set) return EXQ_SUCCESS;
  hipError_t e = hipEventRecord(g_stage_events[i], s);
  if (e != hipSuccess)
    return set_error(EXQ_ERROR_HIP, "hipEventRecord(stage %d): %s", i, hipGetErrorString(e));
  return EXQ_SUCCESS;
}

}  // namespace

const hipEvent_t* stage_events() { return g_stage_events_set ? g_stage_events : nullptr; }

namespace {

// ---- workspace layout of the fused forward --------------------------------------
struct FusedLayout {
  size_t sync, hdr, ends, sorted, tg, mid, partial, rs, blk, plan, total;
  int64_t n, tg_cap;
};

// The decode counters sit at offset 0 with a fixed size, so every fused call
// finds them at the same place whatever its problem size; each decode launch
// leaves them zero again.
FusedLayout fused_layout(const exq_moe_problem& p) {
  FusedLayout L;
  const int64_t kp = p.top_k + p.n_shared;
  const int64_t Ep = p.n_experts + p.n_shared;
  L.n = p.n_tokens * kp;
  L.tg_cap = tg_capacity(L.n, Ep);
  size_t off = 0;
  L.sync = off;     off = align_up(off + kDecodeSyncBytes, 256);
  L.hdr = off;      off = align_up(off + 64, 256);
  L.ends = off;     off = align_up(off + (size_t)(Ep + 1) * 4, 256);
  L.sorted = off;   off = align_up(off + (size_t)L.n * 4, 256);
  L.tg = off;       off = align_up(off + (size_t)L.tg_cap * sizeof(TgEntry), 256);
  L.mid = off;      off = align_up(off + (size_t)L.n * p.inter_size * 2, 256);
  // decode batches: one partial set per down k-split
  const bool dec = decode_path_supported(p.n_tokens, p.top_k, p.n_experts + p.n_shared,
                                         p.n_shared, p.hidden_size, p.inter_size, p.group_size);
  L.partial = off;
  off = align_up(off + (size_t)L.n * p.hidden_size * 4 * (dec ? kDecodeMaxSplit : 1), 256);
  // group row sums of the tiled prefill kernel: x rows (GATEUP), then mid rows (DOWN)
  const int64_t rs_x = tile_rowsum_floats(p.n_tokens, p.hidden_size);
  const int64_t rs_mid = tile_rowsum_floats(L.n, p.inter_size);
  L.rs = off;       off = align_up(off + (size_t)(rs_x > rs_mid ? rs_x : rs_mid) * 4, 256);
  L.blk = off;      off = align_up(off + (size_t)route_plan_blocks(L.n) * Ep * 4, 256);
  L.plan = off;     off = align_up(off + (dec ? decode_plan_bytes(p.n_tokens, p.top_k,
                                                                    p.n_experts, p.n_shared)
                                              : 0), 256);
  L.total = off;
  return L;
}

int validate_problem(const exq_moe_problem* p, const char* fn) {
  EXQ_REQUIRE(p != nullptr, "%s: null problem", fn);
  EXQ_REQUIRE(is_act_dtype(p->act_dtype), "%s: act dtype must be f16 or bf16", fn);
  EXQ_REQUIRE(is_index_dtype(p->ids_dtype), "%s: ids dtype must be i32 or i64", fn);
  EXQ_REQUIRE(is_float_dtype(p->weights_dtype), "%s: weights dtype must be f32/f16/bf16", fn);
  EXQ_REQUIRE(p->n_tokens >= 0 && p->top_k >= 1 && p->n_shared >= 0 && p->n_experts >= 1,
              "%s: bad sizes (T=%lld k=%lld E=%lld shared=%lld)", fn, (long long)p->n_tokens,
              (long long)p->top_k, (long long)p->n_experts, (long long)p->n_shared);
  EXQ_REQUIRE(p->n_experts + p->n_shared <= 1024, "%s: at most 1024 experts (got %lld)", fn,
              (long long)(p->n_experts + p->n_shared));
  EXQ_REQUIRE(p->n_tokens * (p->top_k + p->n_shared) <= (1 << 24),
              "%s: T*(k+shared) = %lld exceeds 2^24 slots", fn,
              (long long)(p->n_tokens * (p->top_k + p->n_shared)));
  EXQ_REQUIRE_SUPPORTED(p->hidden_size >= 32 && p->hidden_size % 32 == 0,
                        "%s: hidden_size=%lld must be a positive multiple of 32", fn,
                        (long long)p->hidden_size);
  EXQ_REQUIRE_SUPPORTED(p->inter_size >= 32 && p->inter_size % 32 == 0,
                        "%s: inter_size=%lld must be a positive multiple of 32", fn,
                        (long long)p->inter_size);
  EXQ_REQUIRE_SUPPORTED(general_shape(p->hidden_size, p->group_size) &&
                            general_shape(p->inter_size, p->group_size),
                        "%s: group_size=%lld must be a multiple of 32 dividing H and I", fn,
                        (long long)p->group_size);
  return EXQ_SUCCESS;
}

// Shapes the decode, tiled and grouped kernels take: H, I and the group size
// multiples of 128.  Other all-INT4 shapes run on the general kernels.
bool standard_shape(const exq_moe_problem* p) {
  return p->hidden_size % 128 == 0 && p->inter_size % 128 == 0 && p->group_size % 128 == 0;
}

int fused_forward_impl(const exq_moe_problem* p, const void* hidden, const void* topk_ids,
                       const void* topk_weights, const Bank& b13, const Bank& b2,
                       const int8_t* tier, void* out, int64_t* sort_order_out,
                       int32_t* expert_ends_out, void* workspace, size_t workspace_bytes,
                       hipStream_t s, const char* fn) {
  const FusedLayout L = fused_layout(*p);
  if (p->n_tokens == 0) return EXQ_SUCCESS;
  if (workspace_bytes < L.total)
    return set_error(EXQ_ERROR_WORKSPACE_TOO_SMALL, "%s: workspace %zu < %zu bytes", fn,
                     workspace_bytes, L.total);
  EXQ_REQUIRE(hidden && topk_ids && out && workspace, "%s: null pointer", fn);
  EXQ_REQUIRE(p->top_k == 0 || topk_weights, "%s: null topk_weights", fn);
  EXQ_REQUIRE(((uintptr_t)hidden | (uintptr_t)out | (uintptr_t)workspace) % 16 == 0,
              "%s: hidden, out and workspace must be 16-byte aligned", fn);
  unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
  const int T = (int)p->n_tokens, H = (int)p->hidden_size, I = (int)p->inter_size;
  const int k = (int)p->top_k, kp = (int)(p->top_k + p->n_shared);
  const int E = (int)p->n_experts, Ep = (int)(p->n_experts + p->n_shared);
  const bool bf = p->act_dtype == EXQ_DTYPE_BF16;

  RoutePlanParams rp;
  rp.ids = topk_ids;
  rp.ids_dtype = p->ids_dtype;
  rp.T = T; rp.k = k; rp.kp = kp; rp.E = E; rp.Ep = Ep;
  rp.n = (int)L.n;
  rp.tier = tier;
  rp.hdr = reinterpret_cast<int*>(ws + L.hdr);
  rp.ends = reinterpret_cast<int*>(ws + L.ends);
  rp.sorted = reinterpret_cast<int*>(ws + L.sorted);
  rp.tg = reinterpret_cast<TgEntry*>(ws + L.tg);
  rp.tg_cap = (int)L.tg_cap;
  // INT4 and BF16 experts run on the tiled kernels (128- or 64-row token
  // groups) when both projections fit them and the gathered activations are 32-bit
  // addressable; INT8 experts (and everything else) on the grouped kernel.
  const int gs = (int)p->group_size;
  // all-INT4 layers of other shapes: routing plan + general kernels + combine
  const bool general = !standard_shape(p);
  EXQ_REQUIRE_SUPPORTED(!general || tier == nullptr,
                        "%s: mixed-precision banks need H, I and group_size multiples of 128 "
                        "(got H=%d I=%d g=%d)", fn, H, I, gs);
  const bool x32 = (int64_t)T * H * 2 <= 0x7fffffffLL;
  const bool tile = !general && x32 && tile_gemm_applies(2, MODE_GATEUP, 2 * I, I, H, gs) &&
                    tile_gemm_applies(2, MODE_DOWN, H, I, I, gs) &&
                    tile_rowsum_floats(L.n, I) * 4 <= 0x7fffffffLL;
  const bool tile_bf = tier != nullptr && x32 &&
                       tile_gemm_applies(0, MODE_GATEUP, 2 * I, I, H, gs) &&
                       tile_gemm_applies(0, MODE_DOWN, H, I, I, gs);
  // INT4 tile shape, when both projections take the 256-row tiles:
  // * experts averaging fewer than 512 routed rows: 64 sorted rows x 256 weight
  //   rows, the same MFMA work per chunk from fewer bytes of copies and about
  //   half the padding rows of 128-row groups (DeepSeek-V2-Lite at 2048 tokens,
  //   192 rows per expert: 627 -> 585 us against 128 x 128);
  // * more rows per expert: 128 x 256 with scaled weight operands, each
  //   activation chunk feeding twice the weight rows of a 128 x 128 tile
  //   (Mixtral at 4096 tokens, 1024 rows per expert: 3375 -> 3040 us against
  //   128 x 128; 128-row groups would pad DeepSeek's experts: 560 -> 579 us).
  // Otherwise 128 x 128.
  const bool wide_ok = tile && tile_gemm_wide_applies(MODE_GATEUP, 2 * I, I) &&
                       tile_gemm_wide_applies(MODE_DOWN, H, I);
  // With the 64 x 256 tiles, the INT4 experts that received at least
  // kI4BigMinRows rows take the 128 x 256 scaled-operand tiles in the same
  // launch (128-row token groups listed first): a skewed router leaves a few
  // experts with most of the rows (DeepSeek-V2-Lite at 2048 tokens: 8 of 64
  // experts hold 72 % of the routed rows).  An expert has at most T rows
  // unless a token repeats an id, so smaller batches keep one shape.
  const int shape = !wide_ok ? TILE_128x128
                             : ((int64_t)T * k < 512 * (int64_t)E ? TILE_64x256 : TILE_PS_128x256);
  const bool i4_mixed = shape == TILE_64x256 && T >= kI4BigMinRows;
  rp.i4_group = tile && shape != TILE_64x256 ? kTokenGroupI4 : kTokenGroup;
  rp.i4_big_rows = !tile ? 0 : (shape == TILE_PS_128x256 ? 1 : (i4_mixed ? kI4BigMinRows : 0));
  rp.i4_big_group = kTokenGroupI4;
  rp.bf_group = tile_bf ? kTokenGroupI4 : kTokenGroup;
  rp.counters = nullptr;
  rp.n_counters = 0;
  rp.sort_order_out = sort_order_out;
  rp.ends_out = expert_ends_out;
  rp.out = out;
  rp.out_bytes = (int64_t)T * H * 2;
  rp.blk_cnt = reinterpret_cast<int*>(ws + L.blk);
  struct HookReset {  // the hook is consumed by this call, whatever happens
    ~HookReset() { g_stage_events_set = false; }
  } hook_reset;
  const bool decode = !general && decode_path_supported(T, k, Ep, p->n_shared, p->hidden_size,
                                                       p->inter_size, p->group_size);
  int st = EXQ_SUCCESS;
  if (!decode) {
    st = record_stage(0, s);
    if (st) return st;
  }
  // The decode kernels route for themselves; the routing plan runs only when
  // the caller asked for the routing arrays.
  if (!decode || sort_order_out || expert_ends_out) {
    st = launch_route_plan(rp, s);
    if (st) return st;
  }
  if (!decode) {
    st = record_stage(1, s);
    if (st) return st;
  }

  if (decode) {
    DecodeLaunch d{};
    d.ids = topk_ids;
    d.ids_dtype = p->ids_dtype;
    d.topk_w = topk_weights;
    d.w_dtype = p->weights_dtype;
    d.T = T; d.k = k; d.kp = kp; d.E = E; d.Ep = Ep;
    d.x = reinterpret_cast<const uint16_t*>(hidden);
    d.w13_bf16 = b13.bf16; d.w13_i8 = b13.i8; d.w13_i8_scales = b13.i8_scales;
    d.w13_i4 = b13.i4; d.w13_i4_scales = b13.i4_scales;
    d.w2_bf16 = b2.bf16; d.w2_i8 = b2.i8; d.w2_i8_scales = b2.i8_scales;
    d.w2_i4 = b2.i4; d.w2_i4_scales = b2.i4_scales;
    d.tier = b13.tier;
    d.index = b13.index;
    d.H = H; d.I = I; d.group_size = (int)p->group_size;
    d.mid = reinterpret_cast<uint16_t*>(ws + L.mid);
    d.part = reinterpret_cast<float*>(ws + L.partial);
    d.out = reinterpret_cast<uint16_t*>(out);
    d.sync = reinterpret_cast<int*>(ws + L.sync);
    d.plan = reinterpret_cast<int*>(ws + L.plan);
    d.bf = bf;
    return launch_decode_layer(d, s);  // times its two kernels with the stage events
  } else if (general) {
    GemmArgs g{};
    g.hdr = rp.hdr;
    g.tg = rp.tg;
    g.row_slot = rp.sorted;
    g.slot_div = kp;
    g.group_size = gs;
    g.inter = I;
    // gate/up + SiLU -> mid [n, I]; down -> partial [slot, H]
    g.n_blocks = (int)cdiv(I, 16);
    g.x = reinterpret_cast<const uint16_t*>(hidden);
    g.x_stride = H;
    g.K = H;
    g.w = b13;
    g.n_rows = 2 * I;
    g.out = ws + L.mid;
    g.out_stride = I;
    st = launch_general_gemm(MODE_GATEUP, bf, g, L.tg_cap, s);
    if (st) return st;
    st = record_stage(2, s);
    if (st) return st;
    g.n_blocks = (int)cdiv(H, 16);
    g.x = reinterpret_cast<const uint16_t*>(ws + L.mid);
    g.x_stride = I;
    g.K = I;
    g.w = b2;
    g.n_rows = H;
    g.out = ws + L.partial;
    g.out_stride = H;
    g.H = H;
    st = launch_general_gemm(MODE_DOWN, bf, g, L.tg_cap, s);
    if (st) return st;
  } else {
    GemmArgs g{};
    g.hdr = rp.hdr;
    g.tg = rp.tg;
    g.row_slot = rp.sorted;
    g.slot_div = kp;
    g.group_size = gs;
    g.inter = I;
    g.skip_i4 = tile ? 1 : 0;
    g.skip_bf = tile_bf ? 1 : 0;
    // The grouped kernel runs only for what the tiles leave: INT8 experts, and
    // INT4 / BF16 experts whose tiled kernel does not apply.  Without a tier
    // array every expert is INT4.  A tile kernel runs only if its tier has
    // experts (an empty launch still costs its grid).
    const bool has_i4 = tier == nullptr || b13.i4 != nullptr;
    const bool has_bf = tier != nullptr && b13.bf16 != nullptr;
    const bool old_kernel = tier == nullptr ? !tile
                                            : (b13.i8 != nullptr || (has_i4 && !tile) ||
                                               (has_bf && !tile_bf));
    const bool run_tile = tile && has_i4, run_tile_bf = tile_bf && has_bf;
    // INT4 tiles 256 rows wide of both shapes, and BF16 tiles: one launch per
    // projection (tile_mix_kernel), each range bounded by cap_*
    const bool mix = run_tile && shape != TILE_128x128 && (run_tile_bf || i4_mixed);
    const int64_t cap_ps =
        shape == TILE_PS_128x256
            ? L.tg_cap
            : (i4_mixed ? std::min<int64_t>(L.tg_cap, cdiv(L.n, kTokenGroupI4) + L.n / kI4BigMinRows)
                        : 0);
    const int64_t cap_64 = shape == TILE_64x256 ? L.tg_cap : 0;
    const int64_t cap_bf = run_tile_bf ? L.tg_cap : 0;
    float* rs = reinterpret_cast<float*>(ws + L.rs);
    // gate/up + SiLU: x = hidden, K = H, rows = 2I, out = mid [n, I] (sorted rows)
    g.n_blocks = I / 16;
    g.x = reinterpret_cast<const uint16_t*>(hidden);
    g.x_stride = H;
    g.K = H;
    g.w = b13;
    g.n_rows = 2 * I;
    g.out = ws + L.mid;
    g.out_stride = I;
    if (old_kernel) {
      st = launch_gemm<MODE_GATEUP>(bf, g, L.tg_cap * g.n_blocks, s);
      if (st) return st;
    }
    if (run_tile_bf && !mix) {
      st = launch_tile_gemm(0, MODE_GATEUP, bf, g, nullptr, 0, (int64_t)T * H * 2, L.tg_cap, s);
      if (st) return st;
    }
    if (run_tile) {
      if (shape != TILE_PS_128x256) {
        st = launch_group_rowsum(bf, g.x, H, T, H, gs, rs, s);
        if (st) return st;
      }
      st = mix ? launch_tile_mix(MODE_GATEUP, bf, g, rs, T, (int64_t)T * H * 2, cap_ps, cap_64,
                                 cap_bf, s)
               : launch_tile_gemm(2, MODE_GATEUP, bf, g, rs, T, (int64_t)T * H * 2, L.tg_cap, s,
                                  shape);
      if (st) return st;
    }
    st = record_stage(2, s);
    if (st) return st;
    // down: x = mid rows (expert-sorted), K = I, rows = H, out = partial [slot, H]
    g.n_blocks = H / 32;
    g.x = reinterpret_cast<const uint16_t*>(ws + L.mid);
    g.x_stride = I;
    g.K = I;
    g.w = b2;
    g.n_rows = H;
    g.out = ws + L.partial;
    g.out_stride = H;
    g.H = H;
    if (old_kernel) {
      st = launch_gemm<MODE_DOWN>(bf, g, L.tg_cap * g.n_blocks, s);
      if (st) return st;
    }
    if (run_tile_bf && !mix) {
      st = launch_tile_gemm(0, MODE_DOWN, bf, g, nullptr, 0, 0, L.tg_cap, s);
      if (st) return st;
    }
    if (run_tile) {
      if (shape != TILE_PS_128x256) {  // sums of the rows the row-sum tiles read
        st = launch_group_rowsum_tg(bf, g.x, I, I, rp.hdr, rp.tg, L.tg_cap, L.n, rs, s);
        if (st) return st;
      }
      st = mix ? launch_tile_mix(MODE_DOWN, bf, g, rs, L.n, 0, cap_ps, cap_64, cap_bf, s)
               : launch_tile_gemm(2, MODE_DOWN, bf, g, rs, L.n, 0, L.tg_cap, s, shape);
      if (st) return st;
    }
  }
  const int64_t threads = (int64_t)T * (H / 4);
  if (bf)
    hipLaunchKernelGGL(combine_partials_kernel<true>, dim3((unsigned)cdiv(threads, 256)),
                       dim3(256), 0, s, reinterpret_cast<const float*>(ws + L.partial),
                       topk_ids, p->ids_dtype, topk_weights, p->weights_dtype, T, k, kp, E, H,
                       reinterpret_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(combine_partials_kernel<false>, dim3((unsigned)cdiv(threads, 256)),
                       dim3(256), 0, s, reinterpret_cast<const float*>(ws + L.partial),
                       topk_ids, p->ids_dtype, topk_weights, p->weights_dtype, T, k, kp, E, H,
                       reinterpret_cast<uint16_t*>(out));
  st = check_launch("combine_partials_kernel");
  if (st) return st;
  return record_stage(3, s);
}

int sorted_gemm_impl(const void* a_sorted, int act_dtype, int64_t n_rows, int64_t K,
                     const Bank& bank, int tier, int64_t n_experts, int64_t N, int64_t gs,
                     const int32_t* ends, const int32_t* mask, void* c, void* workspace,
                     size_t workspace_bytes, hipStream_t s, const char* fn) {
  EXQ_REQUIRE(is_act_dtype(act_dtype), "%s: act dtype must be f16 or bf16", fn);
  EXQ_REQUIRE(n_rows >= 0 && n_rows <= INT32_MAX && n_experts >= 1 && n_experts <= 1024,
              "%s: bad sizes", fn);
  // INT4 weights of other shapes (K % 32, a group size that is a multiple of
  // 32 dividing K, any N) run on the general kernel; BF16 weights need the
  // tiled / grouped kernels' shapes.
  const bool general = tier == 2 && !(K % 128 == 0 && N % 32 == 0 && gs % 128 == 0);
  if (tier == 2) {
    EXQ_REQUIRE_SUPPORTED(general_shape(K, gs),
                          "%s: K=%lld and group_size=%lld: the group size must be a multiple "
                          "of 32 dividing K", fn, (long long)K, (long long)gs);
    EXQ_REQUIRE_SUPPORTED(N >= 1 && N <= INT32_MAX, "%s: bad N=%lld", fn, (long long)N);
  } else {
    EXQ_REQUIRE_SUPPORTED(K >= 128 && K % 128 == 0, "%s: K=%lld must be a multiple of 128",
                          fn, (long long)K);
    EXQ_REQUIRE_SUPPORTED(N >= 32 && N % 32 == 0, "%s: N=%lld must be a multiple of 32", fn,
                          (long long)N);
  }
  const int64_t tg_cap = tg_capacity(n_rows, n_experts);
  const size_t tg_off = align_up(64, 256);
  const size_t rs_off = tg_off + align_up((size_t)tg_cap * sizeof(TgEntry), 256);
  const size_t need = rs_off + align_up((size_t)tile_rowsum_floats(n_rows, K) * 4, 256);
  if (n_rows == 0) return EXQ_SUCCESS;
  if (workspace_bytes < need)
    return set_error(EXQ_ERROR_WORKSPACE_TOO_SMALL, "%s: workspace %zu < %zu bytes", fn,
                     workspace_bytes, need);
  EXQ_REQUIRE(a_sorted && c && ends && workspace, "%s: null pointer", fn);
  EXQ_REQUIRE(((uintptr_t)a_sorted | (uintptr_t)workspace) % 16 == 0,
              "%s: A and workspace must be 16-byte aligned", fn);
  unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
  int* hdr = reinterpret_cast<int*>(ws);
  TgEntry* tg = reinterpret_cast<TgEntry*>(ws + tg_off);
  const bool bf = act_dtype == EXQ_DTYPE_BF16;
  const bool tile = !general && (tier == 2 || tier == 0) &&
                    tile_gemm_applies(tier, MODE_PLAIN, (int)N, 0, (int)K, (int)gs) &&
                    tile_rowsum_floats(n_rows, K) * 4 <= 0x7fffffffLL;
  int st = launch_tg_from_ends(ends, (int)n_experts, mask, tier,
                               tile ? kTokenGroupI4 : kTokenGroup, hdr, tg, (int)tg_cap, s);
  if (st) return st;
  GemmArgs g{};
  g.hdr = hdr;
  g.tg = tg;
  g.n_blocks = (int)(N / 32);
  g.x = reinterpret_cast<const uint16_t*>(a_sorted);
  g.x_stride = K;
  g.K = (int)K;
  g.w = bank;
  g.n_rows = (int)N;
  g.group_size = (int)gs;
  g.out = c;
  g.out_stride = N;
  if (general) {
    g.n_blocks = (int)cdiv(N, 16);
    return launch_general_gemm(MODE_PLAIN, bf, g, tg_cap, s);
  }
  if (tile && tier == 0) return launch_tile_gemm(0, MODE_PLAIN, bf, g, nullptr, 0, 0, tg_cap, s);
  if (tile) {
    float* rs = reinterpret_cast<float*>(ws + rs_off);
    st = launch_group_rowsum(bf, g.x, K, n_rows, (int)K, (int)gs, rs, s);
    if (st) return st;
    return launch_tile_gemm(2, MODE_PLAIN, bf, g, rs, n_rows, 0, tg_cap, s);
  }
  return launch_gemm<MODE_PLAIN>(bf, g, tg_cap * g.n_blocks, s);
}

}  // namespace
}  // namespace exq

using namespace exq;

extern "C" size_t exq_moe_workspace_size(const exq_moe_problem* problem) {
  if (!problem) return 0;
  return fused_layout(*problem).total;
}

extern "C" int exq_set_stage_events(void* const* events, int n_events) {
  if (events == nullptr || n_events == 0) {
    g_stage_events_set = false;
    return EXQ_SUCCESS;
  }
  EXQ_REQUIRE(n_events == 4, "exq_set_stage_events: need 4 events (got %d)", n_events);
  for (int i = 0; i < 4; ++i) {
    EXQ_REQUIRE(events[i] != nullptr, "exq_set_stage_events: null event %d", i);
    g_stage_events[i] = reinterpret_cast<hipEvent_t>(events[i]);
  }
  g_stage_events_set = true;
  return EXQ_SUCCESS;
}

extern "C" size_t exq_moe_gemm_workspace_size(int64_t n_rows, int64_t n_experts, int64_t K) {
  const int64_t r = n_rows > 0 ? n_rows : 0;
  return align_up(64, 256) + align_up((size_t)tg_capacity(r, n_experts) * sizeof(TgEntry), 256) +
         align_up((size_t)tile_rowsum_floats(r, K > 0 ? K : 0) * 4, 256);
}

extern "C" int exq_moe_int4_fused_forward(const exq_moe_problem* problem, const void* hidden,
                                          const void* topk_ids, const void* topk_weights,
                                          const uint8_t* w13_packed, const uint16_t* w13_scales,
                                          const uint8_t* w2_packed, const uint16_t* w2_scales,
                                          void* out, int64_t* sort_order_out,
                                          int32_t* expert_ends_out, void* workspace,
                                          size_t workspace_bytes, exq_stream stream) {
  const char* fn = "exq_moe_int4_fused_forward";
  int st = validate_problem(problem, fn);
  if (st) return st;
  EXQ_REQUIRE(problem->n_shared == 0, "%s: shared experts need exq_moe_mixed_forward", fn);
  EXQ_REQUIRE(w13_packed && w13_scales && w2_packed && w2_scales, "%s: null weights", fn);
  Bank b13{}, b2{};
  b13.i4 = w13_packed;
  b13.i4_scales = w13_scales;
  b2.i4 = w2_packed;
  b2.i4_scales = w2_scales;
  return fused_forward_impl(problem, hidden, topk_ids, topk_weights, b13, b2, nullptr, out,
                            sort_order_out, expert_ends_out, workspace, workspace_bytes,
                            as_stream(stream), fn);
}

extern "C" int exq_moe_mixed_forward(const exq_moe_problem* problem, const void* hidden,
                                     const void* topk_ids, const void* topk_weights,
                                     const exq_expert_bank* bank, void* out,
                                     int64_t* sort_order_out, int32_t* expert_ends_out,
                                     void* workspace, size_t workspace_bytes,
                                     exq_stream stream) {
  const char* fn = "exq_moe_mixed_forward";
  int st = validate_problem(problem, fn);
  if (st) return st;
  EXQ_REQUIRE(bank && bank->tier && bank->index, "%s: bank needs tier and index arrays", fn);
  Bank b13{}, b2{};
  b13.tier = b2.tier = bank->tier;
  b13.index = b2.index = bank->index;
  b13.bf16 = reinterpret_cast<const uint16_t*>(bank->bf16_w13);
  b2.bf16 = reinterpret_cast<const uint16_t*>(bank->bf16_w2);
  b13.i8 = bank->int8_w13;
  b13.i8_scales = bank->int8_w13_scales;
  b2.i8 = bank->int8_w2;
  b2.i8_scales = bank->int8_w2_scales;
  b13.i4 = bank->int4_w13;
  b13.i4_scales = bank->int4_w13_scales;
  b2.i4 = bank->int4_w2;
  b2.i4_scales = bank->int4_w2_scales;
  return fused_forward_impl(problem, hidden, topk_ids, topk_weights, b13, b2, bank->tier, out,
                            sort_order_out, expert_ends_out, workspace, workspace_bytes,
                            as_stream(stream), fn);
}

extern "C" int exq_moe_int4_gemm(const void* a_sorted, int act_dtype, int64_t n_rows, int64_t K,
                                 const uint8_t* packed, const uint16_t* scales,
                                 int64_t n_experts, int64_t N, int64_t group_size,
                                 const int32_t* expert_ends, void* c, void* workspace,
                                 size_t workspace_bytes, exq_stream stream) {
  const char* fn = "exq_moe_int4_gemm";
  EXQ_REQUIRE(packed && scales, "%s: null weights", fn);
  Bank b{};
  b.i4 = packed;
  b.i4_scales = scales;
  return sorted_gemm_impl(a_sorted, act_dtype, n_rows, K, b, 2, n_experts, N, group_size,
                          expert_ends, nullptr, c, workspace, workspace_bytes,
                          as_stream(stream), fn);
}

extern "C" int exq_moe_grouped_gemm(const void* a_sorted, int act_dtype, int64_t n_rows,
                                    int64_t K, const void* weights, int64_t n_experts,
                                    int64_t N, const int32_t* expert_ends,
                                    const int32_t* expert_mask, void* c, void* workspace,
                                    size_t workspace_bytes, exq_stream stream) {
  const char* fn = "exq_moe_grouped_gemm";
  EXQ_REQUIRE(weights, "%s: null weights", fn);
  Bank b{};
  b.bf16 = reinterpret_cast<const uint16_t*>(weights);
  return sorted_gemm_impl(a_sorted, act_dtype, n_rows, K, b, 0, n_experts, N, 128,
                          expert_ends, expert_mask, c, workspace, workspace_bytes,
                          as_stream(stream), fn);
}
