// decode.hip -- self-routing grouped expert kernels for decode batches.
//
// For T <= 64 tokens the routing preparation is folded into the GEMM waves:
// every wave reads the (<= 1024) top-k ids into registers, marks the active
// experts in a per-wave LDS bitmap, picks its expert (the a-th active one in
// ascending id order) and collects that expert's slots with ballots -- the
// slots come out ascending, i.e. in the canonical stable-argsort order.  No
// routing kernel, no workspace plan and no inter-kernel dependency precede
// the first weight load, which is what bounds a decode step.
//
// Unit of work = one wave: (expert, 16 gate rows + 16 matching up rows) for
// GATEUP, (expert, 32 output rows) for DOWN, over the full contraction.  The
// wave streams its weights through a register ring of P k-blocks (16 bytes
// of INT4 per lane per k-block and row set), loads the 16x32 activation
// fragments straight from L2, and runs v_mfma_f32_16x16x32_{bf16,f16}.
//
// Nibble offset: weights enter the MFMA as exact (base + q) values; the
// accumulator of each k-block starts from four MFMAs of the same activation
// fragments against a constant -base operand (sum_k x * -base, identical for
// all 16 weight rows), so no activation row sums are needed.  The fp16 group
// scale multiplies the exact k-block sum in fp32.
#include "exq_internal.h"

namespace exq {
namespace {

constexpr int DW = 4;              // independent waves per work-group
constexpr int DNT = DW * 64;
constexpr int MAX_ID_REGS = 16;    // ids per lane: T * k <= 1024
constexpr int MAX_BM_WORDS = 32;   // active-expert bitmap: E + shared <= 1024

enum DMode { D_GATEUP = 0, D_DOWN = 1 };

struct DBank {
  const int8_t* tier;
  const int32_t* index;
  const uint16_t* bf16;
  const int8_t* i8;
  const uint16_t* i8_scales;
  const uint8_t* i4;
  const uint16_t* i4_scales;
};

struct DecodeArgs {
  const void* ids;
  int ids_dtype;
  int T, k, kp, E, Ep;      // kp = k + n_shared, Ep = E + n_shared
  const uint16_t* x;        // GATEUP: hidden [T, H]; DOWN: mid [T*kp, I]
  int64_t x_stride;
  int K;                    // contraction length (multiple of 128)
  DBank w;
  int n_rows;               // weight rows per expert (2I or H)
  int inter;                // I
  int group_size;
  void* out;                // GATEUP: mid [T*kp, I] act; DOWN: partial [T*kp, H] f32
  int64_t out_stride;
  int n_blocks;             // row blocks per expert (I/16 or H/32)
};

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

// (a & m) | c in one VALU op.  gfx9 VOP3 encodings take no literal
// constants, so the compiler splits the expression into AND + OR; with the
// constants held in VGPRs v_and_or_b32 does it in one.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
  return r;
}

// 8 packed nibbles (k offsets 0..7) -> 8 exact 16-bit floats (base + nibble)
// in k order (0,4,1,5,2,6,3,7); mask = 0x000F000F, magic = base exponent bits.
__device__ __forceinline__ uint4 ddeq4(uint32_t p, uint32_t mask, uint32_t magic) {
  uint4 o;
  o.x = and_or(p, mask, magic);
  o.y = and_or(p >> 4, mask, magic);
  o.z = and_or(p >> 8, mask, magic);
  o.w = and_or(p >> 12, mask, magic);
  return o;
}

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

__device__ __forceinline__ uint4 dperm(const uint4& v) {
  uint4 o;
  o.x = (v.x & 0xffffu) | (v.z << 16);
  o.y = (v.x >> 16) | (v.z & 0xffff0000u);
  o.z = (v.y & 0xffffu) | (v.w << 16);
  o.w = (v.y >> 16) | (v.w & 0xffff0000u);
  return o;
}

// Constant B operand holding -base in every element.
template <int TIER, bool BF>
__device__ __forceinline__ uint4 neg_base_operand() {
  // INT4: base 136 (bf16 128+n-8 form) or 1032 (f16); INT8: 128.
  constexpr uint32_t h = TIER == 2 ? (BF ? 0xC308u : 0xE408u) : (BF ? 0xC300u : 0xD800u);
  constexpr uint32_t d = h | (h << 16);
  return uint4{d, d, d, d};
}

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

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS ops have completed
  __builtin_amdgcn_wave_barrier();
}

// Staged activation rows per work-group: rows * kc <= X_ELEMS halfs.
constexpr int X_ELEMS = 32768;

typedef const void __attribute__((address_space(1)))* gptr_t;
typedef void __attribute__((address_space(3)))* lptr_t;

// Stage activation rows [0, nrows) x k in [k0, k0 + kcc) into LDS with
// global_load_lds_dwordx4: each wave instruction moves 64 16-byte pieces to 64
// consecutive LDS slots (lane i -> base + 16 i), so no registers are used and
// the copy overlaps nothing else in the wave.  Row m's piece q sits at slot
// m * ppr + (q ^ (m & 15)): the XOR swizzle spreads the 16 rows that one
// MFMA A-operand read touches over distinct banks.  Returns once this wave's
// copies have landed; the caller synchronises the work-group.
template <int MODE>
__device__ __forceinline__ void stage_rows_lds(const DecodeArgs& a, const int* row_slot,
                                               int nrows, int k0, int kcc, int ppr,
                                               uint4* xs) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int total = nrows * ppr;
  const int pcc = kcc >> 3;
  for (int pb = wave * 64; pb < total; pb += DNT) {
    const int p = pb + lane;
    const int m = p / ppr;
    const int qs = p - m * ppr;
    if (p < total && qs < pcc) {
      const int q = qs ^ (m & 15);
      const int slot = row_slot[m];
      const int64_t row = MODE == D_GATEUP ? (int64_t)(slot / a.kp) : (int64_t)slot;
      __builtin_amdgcn_global_load_lds((gptr_t)(a.x + row * a.x_stride + k0 + q * 8),
                                       (lptr_t)(xs + pb), 16, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this wave's copies have landed
}

template <int TIER, bool BF, int MODE, int NT, int P>
__device__ __forceinline__ void decode_body(const DecodeArgs& a, int e, int jb, bool active,
                                            int cnt, const int* row_slot, int kc, int gshift,
                                            uint4* xs) {
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15, kq = lane >> 4;
  const int ntiles = NT == 1 ? 1 : (cnt + 15) >> 4;
  const int nkb = a.K >> 7;
  const int kcb = kc >> 7;            // k-blocks per staged chunk (power of two if < nkb)
  const bool chunked = kc < a.K;
  const int ppr = kc >> 3;            // 16-byte pieces per staged row

  int rows[2];
  if (MODE == D_GATEUP) {
    rows[0] = jb * 16 + r16;
    rows[1] = a.inter + jb * 16 + r16;
  } else {
    rows[0] = jb * 32 + r16;
    rows[1] = rows[0] + 16;
  }
  const int widx = a.w.index ? a.w.index[e] : e;
  const int64_t ebase = (int64_t)widx * a.n_rows;
  const unsigned char* rp[2] = {nullptr, nullptr};
  const uint16_t* sp[2] = {nullptr, nullptr};
  float rowscale[2] = {1.f, 1.f};
  if (active) {
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) {
      const int64_t r = ebase + rows[rs];
      if constexpr (TIER == 2) {
        rp[rs] = a.w.i4 + r * (a.K / 2) + kq * 16;
        sp[rs] = a.w.i4_scales + r * (a.K / a.group_size);
      } else if constexpr (TIER == 1) {
        rp[rs] = reinterpret_cast<const unsigned char*>(a.w.i8) + r * a.K + kq * 32;
        rowscale[rs] = f16_bits_to_f32(a.w.i8_scales[r]);
      } else {
        rp[rs] = reinterpret_cast<const unsigned char*>(a.w.bf16 + r * a.K) + kq * 64;
      }
    }
  }
  constexpr int QPK = TIER == 2 ? 1 : (TIER == 1 ? 2 : 4);  // uint4 per lane, k-block, row set
  constexpr int KBSTRIDE = TIER == 2 ? 64 : (TIER == 1 ? 128 : 256);  // row bytes per k-block

  uint4 wq[P][2][QPK];
  uint32_t wsc[P][2];
  auto load_w = [&](int slotp, int kb) {
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) {
      const uint4* src = reinterpret_cast<const uint4*>(rp[rs] + (int64_t)kb * KBSTRIDE);
#pragma unroll
      for (int h = 0; h < QPK; ++h) wq[slotp][rs][h] = src[h];
      if constexpr (TIER == 2) wsc[slotp][rs] = sp[rs][kb >> gshift];
    }
  };

  // Activations land in LDS before the weight stream is issued (vector-memory
  // results return in issue order, so staging behind the weights would wait
  // for them).
  stage_rows_lds<MODE>(a, row_slot, cnt, 0, kc < a.K ? kc : a.K, ppr, xs);
  __syncthreads();
  if (active) {
#pragma unroll
    for (int p = 0; p < P; ++p)
      if (p < nkb) load_w(p, p);
  }

  f32x4_t tot0[NT], tot1[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    tot0[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tot1[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint4 negb = neg_base_operand<TIER, BF>();
  uint32_t dq_mask = 0x000F000Fu, dq_magic = BF ? 0x43004300u : 0x64006400u;
  // A-operand rows beyond cnt read row cnt-1: finite values whose outputs are
  // dropped.  arow = first slot of the row, aswz = its XOR swizzle.
  int arow[NT], aswz[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int q = tt * 16 + r16;
    const int row = q < cnt ? q : cnt - 1;
    arow[tt] = row * ppr;
    aswz[tt] = row & 15;
  }

  for (int kb0 = 0; kb0 < nkb; kb0 += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int kb = kb0 + p;
      if (kb < nkb) {
        if (chunked && kb > 0 && (kb & (kcb - 1)) == 0) {  // next chunk (uniform)
          __syncthreads();
          const int k0 = kb * 128;
          const int kcc = a.K - k0 < kc ? a.K - k0 : kc;
          stage_rows_lds<MODE>(a, row_slot, cnt, k0, kcc, ppr, xs);
          __syncthreads();
        }
        if (active) {
          uint4 bfr[2][4];
          float sc[2] = {1.f, 1.f};
#pragma unroll
          for (int rs = 0; rs < 2; ++rs) {
            if constexpr (TIER == 2) {
              const uint4 w = wq[p][rs][0];
              bfr[rs][0] = ddeq4(w.x, dq_mask, dq_magic);
              bfr[rs][1] = ddeq4(w.y, dq_mask, dq_magic);
              bfr[rs][2] = ddeq4(w.z, dq_mask, dq_magic);
              bfr[rs][3] = ddeq4(w.w, dq_mask, dq_magic);
              sc[rs] = f16_bits_to_f32(wsc[p][rs]);
            } else if constexpr (TIER == 1) {
              const uint4 w0 = wq[p][rs][0], w1 = wq[p][rs][1];
              const uint2 d0 = ddeq8<BF>(w0.x), d1 = ddeq8<BF>(w0.y);
              const uint2 d2 = ddeq8<BF>(w0.z), d3 = ddeq8<BF>(w0.w);
              const uint2 d4 = ddeq8<BF>(w1.x), d5 = ddeq8<BF>(w1.y);
              const uint2 d6 = ddeq8<BF>(w1.z), d7 = ddeq8<BF>(w1.w);
              bfr[rs][0] = uint4{d0.x, d0.y, d1.x, d1.y};
              bfr[rs][1] = uint4{d2.x, d2.y, d3.x, d3.y};
              bfr[rs][2] = uint4{d4.x, d4.y, d5.x, d5.y};
              bfr[rs][3] = uint4{d6.x, d6.y, d7.x, d7.y};
            } else {
#pragma unroll
              for (int h = 0; h < 4; ++h) bfr[rs][h] = wq[p][rs][h];
            }
          }
          if (kb + P < nkb) load_w(p, kb + P);  // refill this ring slot
          const int kpiece = (chunked ? (kb & (kcb - 1)) : kb) * 16 + kq * 4;
#pragma unroll
          for (int tt = 0; tt < NT; ++tt) {
            if (tt < ntiles) {
              uint4 xa[4];
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                xa[d] = xs[arow[tt] + ((kpiece + d) ^ aswz[tt])];
                if constexpr (TIER == 2) xa[d] = dperm(xa[d]);
              }
              f32x4_t init = {0.f, 0.f, 0.f, 0.f};
              if constexpr (TIER != 0) {
#pragma unroll
                for (int d = 0; d < 4; ++d) init = dmfma<BF>(xa[d], negb, init);
              }
              f32x4_t acc0 = init, acc1 = init;
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                acc0 = dmfma<BF>(xa[d], bfr[0][d], acc0);
                acc1 = dmfma<BF>(xa[d], bfr[1][d], acc1);
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
    }
  }
  if (!active) return;

  // Epilogue: lane holds rows (tokens) tt*16 + 4*kq + i, column r16.
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    if (tt >= ntiles) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tt * 16 + kq * 4 + i;
      if (q >= cnt) continue;
      const int slot = row_slot[q];
      const float g0 = tot0[tt][i] * rowscale[0], g1 = tot1[tt][i] * rowscale[1];
      if constexpr (MODE == D_GATEUP) {
        uint16_t* mid = reinterpret_cast<uint16_t*>(a.out);
        const float v = silu_f32(g0) * g1;
        mid[(int64_t)slot * a.out_stride + jb * 16 + r16] =
            (uint16_t)(BF ? f32_to_bf16_bits(v) : f32_to_f16_bits(v));
      } else {
        float* part = reinterpret_cast<float*>(a.out);
        part[(int64_t)slot * a.out_stride + rows[0]] = g0;
        part[(int64_t)slot * a.out_stride + rows[1]] = g1;
      }
    }
  }
}

template <bool BF, int MODE, int NT, bool MIXED>
__global__ void __launch_bounds__(DNT) moe_decode_kernel(DecodeArgs a, int kc, int gshift) {
  extern __shared__ uint4 dyn_lds[];
  __shared__ uint32_t bitmap[DW][MAX_BM_WORDS];
  __shared__ int row_slot[64 * MAX_ID_REGS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = a.T * a.k;
  const int nw = (a.Ep + 31) >> 5;

  // 1. the routed ids, into registers (ids outside [0, E) are dropped)
  int idr[MAX_ID_REGS];
#pragma unroll
  for (int i = 0; i < MAX_ID_REGS; ++i) {
    const int s = lane + 64 * i;
    int v = -1;
    if (s < n) {
      const int64_t id = load_index(a.ids, a.ids_dtype, s);
      v = (id >= 0 && id < a.E) ? (int)id : -1;
    }
    idr[i] = v;
  }
  // 2. active-expert bitmap (each wave builds its own copy in LDS)
  uint32_t* bm = bitmap[wave];
  if (lane < nw) bm[lane] = 0u;
  wave_lds_fence();
#pragma unroll
  for (int i = 0; i < MAX_ID_REGS; ++i)
    if (idr[i] >= 0) atomicOr(&bm[idr[i] >> 5], 1u << (idr[i] & 31));
  if (lane < a.Ep - a.E && a.T > 0) atomicOr(&bm[(a.E + lane) >> 5], 1u << ((a.E + lane) & 31));
  wave_lds_fence();
  const uint32_t word = lane < nw ? bm[lane] : 0u;
  const int c = __popc(word);
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  const int n_active = __shfl(incl, 63, 64);

  // 3. the work-group's unit (expert, group of 4 row blocks).  Work-group i
  //    runs on XCD i % 8; each XCD takes a contiguous range of units.
  const int nbw = (a.n_blocks + DW - 1) / DW;
  const int U = n_active * nbw;
  const int per = (U + 7) >> 3;
  const int local = blockIdx.x >> 3;
  const int u = (blockIdx.x & 7) * per + local;
  if (local >= per || u >= U) return;  // uniform across the work-group
  const int ai = u / nbw;
  const int jb = (u - ai * nbw) * DW + wave;
  const bool active = jb < a.n_blocks;

  // 4. the ai-th active expert
  const uint64_t hit = __ballot(incl - c <= ai && ai < incl);
  const int wl = __ffsll((unsigned long long)hit) - 1;
  uint32_t wbits = __shfl(word, wl, 64);
  const int q0 = ai - (__shfl(incl, wl, 64) - __shfl(c, wl, 64));
  for (int t = 0; t < q0; ++t) wbits &= wbits - 1u;
  const int e = wl * 32 + (__ffs(wbits) - 1);

  // 5. the expert's slots in ascending order (extended slot t*kp + j), as a
  //    table in LDS.  A token routed twice to one expert (repeated ids) adds
  //    rows; cnt <= T*k <= 1024.
  int cnt;
  if (e < a.E) {
    uint64_t m[MAX_ID_REGS];
    int pre[MAX_ID_REGS + 1];
    pre[0] = 0;
#pragma unroll
    for (int i = 0; i < MAX_ID_REGS; ++i) {
      m[i] = __ballot(idr[i] == e);
      pre[i + 1] = pre[i] + __popcll(m[i]);
    }
    cnt = pre[MAX_ID_REGS];
    for (int r = threadIdx.x; r < cnt; r += DNT) {
      int i = 0;
#pragma unroll
      for (int j = 1; j < MAX_ID_REGS; ++j) i = (r >= pre[j]) ? j : i;
      uint64_t mi = m[0];
      int pi = 0;
#pragma unroll
      for (int j = 1; j < MAX_ID_REGS; ++j) {
        if (j == i) {
          mi = m[j];
          pi = pre[j];
        }
      }
      const int s = 64 * i + nth_set_bit(mi, r - pi);
      const int t = s / a.k;
      row_slot[r] = t * a.kp + (s - t * a.k);
    }
  } else {
    cnt = a.T;
    for (int r = threadIdx.x; r < cnt; r += DNT) row_slot[r] = r * a.kp + a.k + (e - a.E);
  }
  __syncthreads();

  uint4* xs = dyn_lds;
  const int tier = MIXED ? (int)a.w.tier[e] : 2;
  // Rows are processed 16*NT at a time (one pass unless ids repeat).
  for (int r0 = 0; r0 < cnt; r0 += NT * 16) {
    const int cc = cnt - r0 < NT * 16 ? cnt - r0 : NT * 16;
    // Every tier streams 256 bytes per lane per ring (8 / 4 / 2 k-blocks).
    if (!MIXED || tier == 2) {
      decode_body<2, BF, MODE, NT, 8>(a, e, jb, active, cc, row_slot + r0, kc, gshift, xs);
    } else if (tier == 1) {
      decode_body<1, BF, MODE, NT, 4>(a, e, jb, active, cc, row_slot + r0, kc, gshift, xs);
    } else {
      decode_body<0, BF, MODE, NT, 2>(a, e, jb, active, cc, row_slot + r0, kc, gshift, xs);
    }
    __syncthreads();  // the next pass restages the same LDS rows
  }
}

template <int MODE, int NT>
int launch_decode_nt(bool bf, const DecodeArgs& a, int kc, int gshift, size_t lds,
                     int64_t grid, hipStream_t s) {
  const dim3 g((unsigned)grid), b(DNT);
  const bool mixed = a.w.tier != nullptr;
  if (bf && mixed)
    hipLaunchKernelGGL((moe_decode_kernel<true, MODE, NT, true>), g, b, lds, s, a, kc, gshift);
  else if (bf)
    hipLaunchKernelGGL((moe_decode_kernel<true, MODE, NT, false>), g, b, lds, s, a, kc, gshift);
  else if (mixed)
    hipLaunchKernelGGL((moe_decode_kernel<false, MODE, NT, true>), g, b, lds, s, a, kc, gshift);
  else
    hipLaunchKernelGGL((moe_decode_kernel<false, MODE, NT, false>), g, b, lds, s, a, kc, gshift);
  return check_launch("moe_decode_kernel");
}

}  // namespace

bool decode_path_supported(int64_t T, int64_t k, int64_t Ep, int64_t n_shared,
                           int64_t group_size) {
  const int64_t gkb = group_size / 128;  // k-blocks per scale group: a power of two
  return T >= 1 && T <= 64 && T * k <= 64 * MAX_ID_REGS && Ep <= 32 * MAX_BM_WORDS &&
         n_shared <= 64 && gkb >= 1 && (gkb & (gkb - 1)) == 0;
}

int launch_decode(bool bf, int mode, const void* ids, int ids_dtype, int T, int k, int kp,
                  int E, int Ep, const uint16_t* x, int64_t x_stride, int K,
                  const int8_t* tier, const int32_t* index, const uint16_t* bf16,
                  const int8_t* i8, const uint16_t* i8_scales, const uint8_t* i4,
                  const uint16_t* i4_scales, int n_rows, int inter, int group_size, void* out,
                  int64_t out_stride, int n_blocks, hipStream_t s) {
  DecodeArgs a{};
  a.ids = ids;
  a.ids_dtype = ids_dtype;
  a.T = T; a.k = k; a.kp = kp; a.E = E; a.Ep = Ep;
  a.x = x;
  a.x_stride = x_stride;
  a.K = K;
  a.w = DBank{tier, index, bf16, i8, i8_scales, i4, i4_scales};
  a.n_rows = n_rows;
  a.inter = inter;
  a.group_size = group_size;
  a.out = out;
  a.out_stride = out_stride;
  a.n_blocks = n_blocks;
  const int64_t max_active = (int64_t)(T * k < E ? T * k : E) + (Ep - E);
  const int64_t units = max_active * ((n_blocks + DW - 1) / DW);
  const int64_t grid = 8 * cdiv(units, 8);
  if (grid == 0) return EXQ_SUCCESS;
  // Staged rows: the most rows one pass can hold; the contraction is staged
  // in power-of-two chunks of kc elements so rows * kc <= X_ELEMS.
  const int nt = T <= 16 ? 1 : (T <= 32 ? 2 : 4);
  const int rows = T * k < nt * 16 ? T * k : nt * 16;
  int kc = K;
  if ((int64_t)rows * K > X_ELEMS) {
    kc = 128;
    while ((int64_t)rows * kc * 2 <= X_ELEMS) kc *= 2;
  }
  const size_t lds = (size_t)rows * kc * 2;
  int gshift = 0;
  if (group_size > 0) {
    while ((128 << gshift) < group_size) ++gshift;
  }
  if (mode == D_GATEUP) {
    if (nt == 1) return launch_decode_nt<D_GATEUP, 1>(bf, a, kc, gshift, lds, grid, s);
    if (nt == 2) return launch_decode_nt<D_GATEUP, 2>(bf, a, kc, gshift, lds, grid, s);
    return launch_decode_nt<D_GATEUP, 4>(bf, a, kc, gshift, lds, grid, s);
  }
  if (nt == 1) return launch_decode_nt<D_DOWN, 1>(bf, a, kc, gshift, lds, grid, s);
  if (nt == 2) return launch_decode_nt<D_DOWN, 2>(bf, a, kc, gshift, lds, grid, s);
  return launch_decode_nt<D_DOWN, 4>(bf, a, kc, gshift, lds, grid, s);
}

}  // namespace exq
