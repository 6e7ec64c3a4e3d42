// general.hip -- INT4 grouped GEMMs for the shapes the tiled and grouped
// kernels do not take: a group size below 128 or not a multiple of 128 (any
// multiple of 32 that divides K), a contraction length that is a multiple of
// 32 but not of 128, and any number of weight rows.  These are the shapes the
// reference accepts (moe_int4_kernel.py:61-64 collapses K < group_size to one
// group; :274-292 derives the group from the scales' shape and needs
// group >= 32; :206-207, 238-240 mask the N tail).
//
// One wave per work-group.  Unit = (token group of <= 64 expert-sorted rows,
// 16 output columns):
//   GATEUP: gate rows j0..j0+15 and the matching up rows I + j0..; SiLU(gate)
//           * up is written to `mid`;
//   PLAIN / DOWN: 16 consecutive weight rows.
// The contraction runs in k-steps of 32, one v_mfma_f32_16x16x32 per 16-row
// tile and weight set: lane (r, q) feeds activations k0 + 8q .. k0 + 8q + 7 of
// row r (one 16-byte load) and the same eight k of weight row r (one dword of
// packed nibbles), so every step lies inside one scale group.  Nibbles become
// exact 16-bit floats of (q - 8) (small integers convert exactly), the steps of
// a group accumulate exactly in fp32, and the group's fp16 scale multiplies the
// group sum.  Rows past the token group load zeros and are not stored; weight
// rows past N load zeros and are not stored.
#include "exq_internal.h"

#include "dev_util.h"

namespace exq {
namespace {

using namespace dev;

constexpr int GMT = 4;  // 16-row tiles per unit (kTokenGroup rows)

// 8 packed nibbles (low nibble = even k) of one dword -> 8 exact 16-bit floats
// of (nibble - 8), natural k order.
template <bool BF>
__device__ __forceinline__ uint4 signed_nibbles(uint32_t p) {
  uint32_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float v = (float)((int)((p >> (4 * i)) & 15u) - 8);
    h[i] = BF ? (__float_as_uint(v) >> 16) : f32_to_f16_bits(v);  // exact: |v| <= 8
  }
  return uint4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
               h[6] | (h[7] << 16)};
}

template <bool BF, int MODE>
__global__ void __launch_bounds__(64) general_gemm_kernel(GemmArgs a) {
  constexpr int NS = MODE == MODE_GATEUP ? 2 : 1;  // weight sets (gate, up)
  const int first = a.hdr[1];                      // INT4 token groups [hdr[1], hdr[0])
  const int n_tg = a.hdr[0] - first;
  const int U = n_tg * a.n_blocks;
  const int lane = threadIdx.x, r16 = lane & 15, kq = lane >> 4;
  const int K = a.K, ngs = K / a.group_size, spg = a.group_size / 32;
  const int n_out = MODE == MODE_GATEUP ? a.inter : a.n_rows;  // output columns
  for (int unit = blockIdx.x; unit < U; unit += gridDim.x) {
    const int tgi = unit / a.n_blocks;
    const int blk = unit - tgi * a.n_blocks;
    const TgEntry te = a.tg[first + tgi];
    if (te.cnt <= 0) continue;
    const int widx = a.w.index ? a.w.index[te.e] : te.e;
    const int64_t ebase = (int64_t)widx * a.n_rows;
    const int col = blk * 16 + r16;   // this lane's output column (B operand row)
    const bool col_ok = col < n_out;
    // weight rows of the lane's column, one per set
    const uint32_t* wrow[NS];
    const uint16_t* srow[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int64_t r = ebase + (MODE == MODE_GATEUP ? s * a.inter : 0) + (col_ok ? col : 0);
      wrow[s] = reinterpret_cast<const uint32_t*>(a.w.i4 + r * (K / 2));
      srow[s] = a.w.i4_scales + r * ngs;
    }
    // activation rows of the lane's tile rows
    const uint16_t* xrow[GMT];
    bool xok[GMT];
#pragma unroll
    for (int mt = 0; mt < GMT; ++mt) {
      const int m = mt * 16 + r16;
      xok[mt] = m < te.cnt;
      const int mm = xok[mt] ? m : 0;
      const int64_t row = MODE == MODE_GATEUP ? a.row_slot[te.pos0 + mm] / a.slot_div
                                              : te.pos0 + mm;
      xrow[mt] = a.x + row * a.x_stride;
    }
    f32x4_t tot[GMT][NS];
#pragma unroll
    for (int mt = 0; mt < GMT; ++mt)
#pragma unroll
      for (int s = 0; s < NS; ++s) tot[mt][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int g = 0; g < ngs; ++g) {
      f32x4_t acc[GMT][NS];
#pragma unroll
      for (int mt = 0; mt < GMT; ++mt)
#pragma unroll
        for (int s = 0; s < NS; ++s) acc[mt][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int st = 0; st < spg; ++st) {
        const int k0 = (g * spg + st) * 32 + kq * 8;  // this lane's eight k
        uint4 wb[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s)
          wb[s] = signed_nibbles<BF>(col_ok ? wrow[s][k0 >> 3] : 0x88888888u);
#pragma unroll
        for (int mt = 0; mt < GMT; ++mt) {
          const uint4 xa = xok[mt] ? *reinterpret_cast<const uint4*>(xrow[mt] + k0)
                                   : uint4{0u, 0u, 0u, 0u};
#pragma unroll
          for (int s = 0; s < NS; ++s) acc[mt][s] = dmfma<BF>(xa, wb[s], acc[mt][s]);
        }
      }
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float sc = col_ok ? f16_bits_to_f32(srow[s][g]) : 0.f;
#pragma unroll
        for (int mt = 0; mt < GMT; ++mt) tot[mt][s] += sc * acc[mt][s];
      }
    }
    // D layout: lane (r16, kq) holds rows 4 kq + i of each tile, column col
    if (col_ok) {
#pragma unroll
      for (int mt = 0; mt < GMT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mt * 16 + kq * 4 + i;
          if (m >= te.cnt) continue;
          const int pos = te.pos0 + m;
          if constexpr (MODE == MODE_GATEUP) {
            uint16_t* mid = reinterpret_cast<uint16_t*>(a.out);
            mid[(int64_t)pos * a.out_stride + col] =
                (uint16_t)to_act_bits<BF>(silu_f32(tot[mt][0][i]) * tot[mt][NS - 1][i]);
          } else if constexpr (MODE == MODE_PLAIN) {
            uint16_t* c = reinterpret_cast<uint16_t*>(a.out);
            c[(int64_t)pos * a.out_stride + col] = (uint16_t)to_act_bits<BF>(tot[mt][0][i]);
          } else {
            float* part = reinterpret_cast<float*>(a.out);
            part[(int64_t)a.row_slot[pos] * a.out_stride + col] = tot[mt][0][i];
          }
        }
      }
    }
  }
}

template <int MODE>
int launch_mode(bool bf, const GemmArgs& a, int64_t grid, hipStream_t s) {
  if (bf)
    hipLaunchKernelGGL((general_gemm_kernel<true, MODE>), dim3((unsigned)grid), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL((general_gemm_kernel<false, MODE>), dim3((unsigned)grid), dim3(64), 0, s,
                       a);
  return check_launch("general_gemm_kernel");
}

}  // namespace

bool general_shape(int64_t K, int64_t group_size) {
  return K >= 32 && K % 32 == 0 && group_size >= 32 && group_size % 32 == 0 &&
         K % group_size == 0;
}

int launch_general_gemm(int mode, bool bf, const GemmArgs& a, int64_t tg_cap, hipStream_t s) {
  // one work-group per (token group, 16 columns) up to the capacity bound;
  // work-groups past the actual count exit at once, and a grid beyond 2^20
  // strides instead
  int64_t grid = tg_cap * a.n_blocks;
  if (grid > (1 << 20)) grid = 1 << 20;
  if (grid <= 0) return EXQ_SUCCESS;
  if (mode == MODE_GATEUP) return launch_mode<MODE_GATEUP>(bf, a, grid, s);
  if (mode == MODE_DOWN) return launch_mode<MODE_DOWN>(bf, a, grid, s);
  return launch_mode<MODE_PLAIN>(bf, a, grid, s);
}

}  // namespace exq
