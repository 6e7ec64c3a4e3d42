// decode.hip -- the whole MoE layer in one launch for decode batches (T <= 64).
//
// Persistent work-groups.  Every wave reads the (<= 1024) routed ids into
// registers, marks the active experts in an LDS bitmap and counts them; the
// work-group then loops over units
//
//   gate/up  (expert, 16 gate rows + the 16 matching up rows)     u <  NA
//   down     (expert, 64 output rows)                             u >= NA
//
// taken round-robin (u = blockIdx.x, + gridDim.x, ...), all gate/up units
// before any down unit.  The four waves of a work-group split the
// contraction of a unit into contiguous k-block ranges, so many short weight
// streams run at once and the tail of the launch stays short.
//
// Dataflow instead of a kernel boundary: a down unit of expert e issues its
// weight loads, then waits until all gate/up units of e have published their
// `mid` rows (per-expert counter), then stages those rows.  Every down unit adds its fp32 partial rows for one 64-column
// block of H and bumps that block's counter; the last unit to arrive sums the
// block's partials over each token's k slots in fixed order (deterministic)
// and writes the output.  Data shared between work-groups (mid rows, fp32
// partials) is written and read with agent-coherent (sc1) accesses, and every
// storing wave waits for its stores to complete before its work-group bumps a
// counter, so no whole-cache writeback or invalidate is needed (on this part
// agent-scope fences write back / invalidate the whole L2 of an XCD).  The
// last combine zeroes the counters, so the sync
// region is zero again when the launch ends.  Waits are bounded: a wait that
// runs out sets an error word instead of hanging (the grid never exceeds the
// number of co-resident work-groups, so waits end in practice).
//
// Per unit and wave: the weight stream goes through a register ring of P
// k-blocks (one 128-bit load per lane per row set and k-block), issued before
// the activation rows are staged into LDS with global_load_lds_dwordx4 (XOR
// swizzled); weights and scales come through bounds-checked buffer loads.  Nibbles become exact bf16/f16 values (base + n) with one
// v_and_or_b32 per pair (the exponent-OR method of Kim et al., "Who Says
// Elephants Can't Run", 2022) and feed v_mfma_f32_16x16x32_{bf16,f16}; the
// constant base is removed by MFMAs of the same activations against a -base
// operand; the fp16 group scale multiplies each exact k-block sum in fp32.
// The four waves' partial tiles are summed through LDS.
#include <mutex>

#include "exq_internal.h"

namespace exq {
namespace {

constexpr int DW = 4;              // waves per work-group
constexpr int DNT = DW * 64;
constexpr int MAX_ID_REGS = 16;    // ids per lane: T * k <= 1024
constexpr int MAX_BM_WORDS = 32;   // active-expert bitmap: E + shared <= 1024
constexpr int RING = 8;            // 128-bit weight registers per lane
// Output rows of a down unit: 64 (four row sets), 32 when a pass holds
// four 16-row tiles (register budget).
__host__ __device__ constexpr int rows_b(int nt) { return nt == 4 ? 32 : 64; }
constexpr int64_t SPIN_LIMIT = 1 << 22;
constexpr int CPOL_SC1 = 16;       // cache-policy bits: sc1 (agent-coherent access)

struct Proj {
  const uint16_t* bf16;
  const int8_t* i8;
  const uint16_t* i8_scales;
  const uint8_t* i4;
  const uint16_t* i4_scales;
};

struct LayerArgs {
  const void* ids;
  int ids_dtype;
  const void* topk_w;
  int w_dtype;
  int T, k, kp, E, Ep;          // kp = k + n_shared, Ep = E + n_shared
  const uint16_t* x;            // hidden [T, H]
  Proj w13, w2;
  const int8_t* tier;           // [Ep] or null (all INT4)
  const int32_t* index;         // [Ep] or null (identity)
  int H, I, gshift;             // group size = 128 << gshift
  uint16_t* mid;                // [T * kp, I] activation dtype
  float* part;                  // [T * kp, H] fp32
  uint16_t* out;                // [T, H]
  int* sync;                    // counters, see sync_* below
  int nbA, nbB;                 // units per expert: I / 16, H / rows_b(NT)
  int xw;                       // per-wave LDS staging budget (16-bit elements)
};

// Counter layout of the sync region (fixed, independent of the problem size):
// one 128-byte line per counter.
constexpr int SYNC_INTS = 32;
__device__ __forceinline__ int* sync_a(const LayerArgs& a, int e) { return a.sync + e * SYNC_INTS; }
__device__ __forceinline__ int* sync_c(const LayerArgs& a, int hb) {
  return a.sync + (kDecodeMaxBuckets + hb) * SYNC_INTS;
}
__device__ __forceinline__ int* sync_done(const LayerArgs& a) {
  return a.sync + (kDecodeMaxBuckets + kDecodeMaxHBlocks) * SYNC_INTS;
}
__device__ __forceinline__ int* sync_err(const LayerArgs& a) {
  return a.sync + (kDecodeMaxBuckets + kDecodeMaxHBlocks + 1) * SYNC_INTS;
}

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

// (a & m) | c.  Plain C: gfx950 fuses it into one v_bitop3_b32 (or
// v_and_or_b32), and the compiler's hazard tracking sees every instruction.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  return (a & m) | c;
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

// Activation order used with INT4 weights: (x0,x4),(x1,x5),(x2,x6),(x3,x7).
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

template <bool BF>
__device__ __forceinline__ uint32_t to_act_bits(float v) {
  return BF ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
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

// Wave-local waits written as volatile asm with a memory clobber, so the
// compiler moves no memory access across them: LDS written by an LDS DMA
// (global_load_lds) is only ordered by the vmcnt wait, which the compiler
// does not model as a dependency of later LDS reads.
__device__ __forceinline__ void wave_lds_fence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS ops have completed
}

__device__ __forceinline__ void wait_vm_all() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads and LDS DMA have landed
}

typedef void __attribute__((address_space(3)))* lptr_t;

typedef const void __attribute__((address_space(1)))* gptr_t;

// Buffer resource over `bytes` bytes at `base` (gfx9 word 3): loads beyond
// the range return zero instead of touching other memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// Stage activation rows [0, nrows) x k-blocks [kb0, kb0 + nkbc) into this
// wave's LDS region with global_load_lds_dwordx4: each wave instruction moves
// 64 16-byte pieces to 64 consecutive LDS slots, so no registers are used.
// Row m's piece q sits at slot m * ppr + (q ^ (m & 15)): the XOR swizzle
// spreads the 16 rows that one MFMA A-operand read touches over distinct
// banks.  The caller waits (wait_vm_all) before reading.
template <int PH>
__device__ __forceinline__ void stage_rows(const LayerArgs& a, const int* row_slot, int nrows,
                                           int kb0, int nkbc, int ppr, uint4* xs) {
  const int lane = threadIdx.x & 63;
  const int total = nrows * ppr;
  const int pcc = nkbc * 16;
  for (int pb = 0; pb < total; pb += 64) {
    const int p = pb + lane;
    const int m = p / ppr;
    const int qs = p - m * ppr;
    if (p < total && qs < pcc) {
      const int q = qs ^ (m & 15);
      const int slot = row_slot[m];
      const uint16_t* src = PH == 0 ? a.x + (int64_t)(slot / a.kp) * a.H
                                    : a.mid + (int64_t)slot * a.I;
      __builtin_amdgcn_global_load_lds((gptr_t)(src + kb0 * 128 + q * 8), (lptr_t)(xs + pb), 16,
                                       0, PH == 0 ? 0 : CPOL_SC1);
    }
  }
}

// Waits until *cnt >= target (agent scope), at most SPIN_LIMIT polls.
__device__ void wait_counter(const LayerArgs& a, const int* cnt, int target) {
  if ((threadIdx.x & 63) == 0) {
    int64_t spins = 0;
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (++spins > SPIN_LIMIT) {
        __hip_atomic_fetch_or(sync_err(a), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __builtin_amdgcn_wave_barrier();
  wait_vm_all();
}

// One unit of work (phase PH: 0 gate/up + SiLU, 1 down + combine) for an
// expert of precision tier TIER, in passes of NT*16 rows.
template <int TIER, bool BF, int PH, int NT>
__device__ void unit_body(const LayerArgs& a, int e, int blk, int cnt, const int* row_slot,
                          unsigned char* lds, int* s_flag, int n_active) {
  constexpr int ROWS_B = rows_b(NT);
  constexpr int RS = PH == 0 ? 2 : ROWS_B / 16;                 // row sets of 16 rows
  constexpr int QPK = TIER == 2 ? 1 : (TIER == 1 ? 2 : 4);      // uint4 per lane, k-block, row set
  constexpr int RING_NT = NT <= 2 ? RING : RING / 2;            // fewer ring registers at NT=4
  constexpr int P0 = RING_NT / (RS * QPK);
  constexpr int P = P0 > 0 ? P0 : 1;                            // ring depth (k-blocks)
  constexpr int KBSTRIDE = TIER == 2 ? 64 : (TIER == 1 ? 128 : 256);  // row bytes per k-block
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int K = PH == 0 ? a.H : a.I;
  const int nkb = K >> 7;
  const int lo = (wave * nkb) >> 2;
  const int nmy = (((wave + 1) * nkb) >> 2) - lo;  // k-blocks of this wave
  const Proj& W = PH == 0 ? a.w13 : a.w2;
  const int n_rows = PH == 0 ? 2 * a.I : a.H;
  const int widx = a.index ? a.index[e] : e;
  const int64_t ebase = (int64_t)widx * n_rows;

  int rows[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    if (PH == 0)
      rows[rs] = (rs == 0 ? 0 : a.I) + blk * 16 + r16;
    else
      rows[rs] = blk * ROWS_B + rs * 16 + r16;
  }
  // This expert's weights (and INT4 scales) behind bounds-checked buffer
  // resources; each lane keeps a 32-bit offset per row set.
  const int rowbytes = TIER == 2 ? K / 2 : (TIER == 1 ? K : 2 * K);
  const unsigned char* wbase =
      TIER == 2 ? W.i4
                : (TIER == 1 ? reinterpret_cast<const unsigned char*>(W.i8)
                             : reinterpret_cast<const unsigned char*>(W.bf16));
  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(wbase + ebase * rowbytes, (int64_t)n_rows * rowbytes);
  const int ng = nkb >> a.gshift;  // scale groups per row
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(TIER == 2 ? W.i4_scales + ebase * ng : nullptr, (int64_t)n_rows * ng * 2);
  int voff[RS], soff[RS];
  float rowscale[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
    voff[rs] = rows[rs] * rowbytes + kq * 16 * QPK;
    soff[rs] = rows[rs] * ng * 2;
    rowscale[rs] = 1.f;
    if constexpr (TIER == 1) rowscale[rs] = f16_bits_to_f32(W.i8_scales[ebase + rows[rs]]);
  }

  uint4 wq[P][RS][QPK];
  uint32_t wsc[P][RS];
  auto load_w = [&](int slotp, int kb) {
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
      for (int h = 0; h < QPK; ++h)
        wq[slotp][rs][h] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff[rs] + h * 16, kb * KBSTRIDE, 0));
      if constexpr (TIER == 2)
        wsc[slotp][rs] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff[rs], (kb >> a.gshift) * 2, 0);
    }
  };

  uint4* xs = reinterpret_cast<uint4*>(lds + (size_t)wave * a.xw * 2);
  const __amdgpu_buffer_rsrc_t mid_r = make_rsrc(a.mid, (int64_t)a.T * a.kp * a.I * 2);
  const __amdgpu_buffer_rsrc_t part_r = make_rsrc(a.part, (int64_t)a.T * a.kp * a.H * 4);
  const uint4 negb = neg_base_operand<TIER, BF>();
  const uint32_t dq_mask = 0x000F000Fu, dq_magic = BF ? 0x43004300u : 0x64006400u;

  for (int r0 = 0; r0 < cnt; r0 += NT * 16) {
    const int cc = cnt - r0 < NT * 16 ? cnt - r0 : NT * 16;
    const int ntiles = (cc + 15) >> 4;
    const int* rsl = row_slot + r0;
    // k-blocks per staged chunk: a power of two covering this wave's range
    // when the rows fit, else the most that fit (restaged chunk by chunk)
    int kcb = 1;
    while (kcb < nmy && cc * (kcb * 2) * 128 <= a.xw) kcb *= 2;
    const int ppr = kcb * 16;  // 16-byte pieces per staged row

    // 1. weights first: they do not depend on anything
#pragma unroll
    for (int p = 0; p < P; ++p)
      if (p < nmy) load_w(p, lo + p);
    // 2. a down unit needs every gate/up unit of its expert
    if (PH == 1 && r0 == 0) wait_counter(a, sync_a(a, e), a.nbA);
    // 3. activation rows of the first chunk
    if (nmy > 0) stage_rows<PH>(a, rsl, cc, lo, nmy < kcb ? nmy : kcb, ppr, xs);
    wait_vm_all();

    f32x4_t tot[RS][NT];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int t = 0; t < NT; ++t) tot[rs][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // A-operand rows beyond cc read row cc-1: finite values whose outputs are dropped.
    int arow[NT], aswz[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int q = tt * 16 + r16;
      const int row = q < cc ? q : cc - 1;
      arow[tt] = row * ppr;
      aswz[tt] = row & 15;
    }

    for (int kb0 = 0; kb0 < nmy; kb0 += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int kbl = kb0 + p;  // k-block index within this wave's range
        if (kbl < nmy) {
          if (kbl > 0 && (kbl & (kcb - 1)) == 0) {  // next staged chunk (wave-local)
            wave_lds_fence();
            const int rem = nmy - kbl;
            stage_rows<PH>(a, rsl, cc, lo + kbl, rem < kcb ? rem : kcb, ppr, xs);
            wait_vm_all();
          }
          const int kpiece = (kbl & (kcb - 1)) * 16 + kq * 4;
          // One row set's weights as MFMA B operands (exact base + q values).
          auto dequant = [&](int rs, uint4 (&bfr)[4], float& sc) {
            sc = 1.f;
            if constexpr (TIER == 2) {
              const uint4 w = wq[p][rs][0];
              bfr[0] = ddeq4(w.x, dq_mask, dq_magic);
              bfr[1] = ddeq4(w.y, dq_mask, dq_magic);
              bfr[2] = ddeq4(w.z, dq_mask, dq_magic);
              bfr[3] = ddeq4(w.w, dq_mask, dq_magic);
              sc = f16_bits_to_f32(wsc[p][rs]);
            } else if constexpr (TIER == 1) {
              const uint4 w0 = wq[p][rs][0], w1 = wq[p][rs][1];
              const uint2 d0 = ddeq8<BF>(w0.x), d1 = ddeq8<BF>(w0.y);
              const uint2 d2 = ddeq8<BF>(w0.z), d3 = ddeq8<BF>(w0.w);
              const uint2 d4 = ddeq8<BF>(w1.x), d5 = ddeq8<BF>(w1.y);
              const uint2 d6 = ddeq8<BF>(w1.z), d7 = ddeq8<BF>(w1.w);
              bfr[0] = uint4{d0.x, d0.y, d1.x, d1.y};
              bfr[1] = uint4{d2.x, d2.y, d3.x, d3.y};
              bfr[2] = uint4{d4.x, d4.y, d5.x, d5.y};
              bfr[3] = uint4{d6.x, d6.y, d7.x, d7.y};
            } else {
#pragma unroll
              for (int h = 0; h < 4; ++h) bfr[h] = wq[p][rs][h];
            }
          };
          // A operand of tile tt (four 16x32 pieces) and its -base sum.
          auto load_a = [&](int tt, uint4 (&xa)[4], f32x4_t& init) {
            init = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              xa[d] = xs[arow[tt] + ((kpiece + d) ^ aswz[tt])];
              if constexpr (TIER == 2) xa[d] = dperm(xa[d]);
            }
            if constexpr (TIER != 0) {
#pragma unroll
              for (int d = 0; d < 4; ++d) init = dmfma<BF>(xa[d], negb, init);
            }
          };
          if constexpr (NT <= 2) {
            // A operands of every tile first, then one row set at a time
            uint4 xa[NT][4];
            f32x4_t init[NT];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
              if (tt < ntiles) load_a(tt, xa[tt], init[tt]);
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) {
              uint4 bfr[4];
              float sc;
              dequant(rs, bfr, sc);
#pragma unroll
              for (int tt = 0; tt < NT; ++tt) {
                if (tt < ntiles) {
                  f32x4_t acc = init[tt];
#pragma unroll
                  for (int d = 0; d < 4; ++d) acc = dmfma<BF>(xa[tt][d], bfr[d], acc);
                  tot[rs][tt] += sc * acc;
                }
              }
            }
          } else {
            // four tiles: one tile's A operand at a time (fewer live registers)
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
              if (tt < ntiles) {
                uint4 xa[4];
                f32x4_t init;
                load_a(tt, xa, init);
#pragma unroll
                for (int rs = 0; rs < RS; ++rs) {
                  uint4 bfr[4];
                  float sc;
                  dequant(rs, bfr, sc);
                  f32x4_t acc = init;
#pragma unroll
                  for (int d = 0; d < 4; ++d) acc = dmfma<BF>(xa[d], bfr[d], acc);
                  tot[rs][tt] += sc * acc;
                }
              }
            }
          }
          if (kbl + P < nmy) load_w(p, lo + kbl + P);  // refill this ring slot
        }
      }
    }

    // 4. sum the four waves' partial tiles through LDS (aliases the staging area)
    __syncthreads();
    float4* red = reinterpret_cast<float4*>(lds);  // [wave][rs][tt][lane]
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (tt < ntiles)
          red[((wave * RS + rs) * NT + tt) * 64 + lane] =
              float4{tot[rs][tt][0], tot[rs][tt][1], tot[rs][tt][2], tot[rs][tt][3]};
    __syncthreads();

    // 5. epilogue: lane (r16, kq) of tile tt holds rows tt*16 + 4*kq + i, column r16
    bool stored = false;
    if constexpr (PH == 0) {
      const int tt = wave;
      if (tt < ntiles) {
        float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < DW; ++w) {
          const float4 pg = red[((w * RS + 0) * NT + tt) * 64 + lane];
          const float4 pu = red[((w * RS + 1) * NT + tt) * 64 + lane];
          g[0] += pg.x; g[1] += pg.y; g[2] += pg.z; g[3] += pg.w;
          u[0] += pu.x; u[1] += pu.y; u[2] += pu.z; u[3] += pu.w;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = tt * 16 + kq * 4 + i;
          if (q < cc) {
            const float v = silu_f32(g[i] * rowscale[0]) * (u[i] * rowscale[1]);
            __builtin_amdgcn_raw_buffer_store_b16((uint16_t)to_act_bits<BF>(v), mid_r,
                                                  (rsl[q] * a.I + blk * 16 + r16) * 2, 0, CPOL_SC1);
          }
        }
        stored = true;
      }
    } else {
      for (int it = threadIdx.x; it < RS * ntiles * 64; it += DNT) {
        const int rt = it >> 6;
        const int rs = rt / ntiles, tt = rt - rs * ntiles;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < DW; ++w) {
          const float4 pv = red[((w * RS + rs) * NT + tt) * 64 + lane];
          s[0] += pv.x; s[1] += pv.y; s[2] += pv.z; s[3] += pv.w;
        }
        float rsc = 1.f;
#pragma unroll
        for (int j = 0; j < RS; ++j)
          if (j == rs) rsc = rowscale[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = tt * 16 + kq * 4 + i;
          if (q < cc)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s[i] * rsc), part_r,
                                                  (rsl[q] * a.H + blk * ROWS_B + rs * 16 + r16) * 4,
                                                  0, CPOL_SC1);
        }
        stored = true;
      }
    }
    if (stored) wait_vm_all();  // this wave's shared stores have completed
    __syncthreads();  // red / staging area and row_slot free again
  }

  // 6. publish
  if constexpr (PH == 0) {
    if (threadIdx.x == 0)
      __hip_atomic_fetch_add(sync_a(a, e), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (threadIdx.x == 0) {
      const int old =
          __hip_atomic_fetch_add(sync_c(a, blk), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_flag = old == n_active - 1;
    }
    __syncthreads();
    if (*s_flag) {
      // Last down unit of this column block: combine it.
      const int h0 = blk * ROWS_B;
      for (int idx = threadIdx.x; idx < a.T * (ROWS_B / 4); idx += DNT) {
        const int t = idx / (ROWS_B / 4);
        const int h = h0 + (idx - t * (ROWS_B / 4)) * 4;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < a.kp; ++j) {
          float wgt = 1.f;
          if (j < a.k) {
            const int64_t id = load_index(a.ids, a.ids_dtype, (int64_t)t * a.k + j);
            if (id < 0 || id >= a.E) continue;
            wgt = load_as_f32(a.topk_w, a.w_dtype, (int64_t)t * a.k + j);
          }
          const float4 pv = __builtin_bit_cast(
              float4, __builtin_amdgcn_raw_buffer_load_b128(
                          part_r, ((t * a.kp + j) * a.H + h) * 4, 0, CPOL_SC1));
          acc[0] += wgt * pv.x;
          acc[1] += wgt * pv.y;
          acc[2] += wgt * pv.z;
          acc[3] += wgt * pv.w;
        }
        uint2 o;
        o.x = to_act_bits<BF>(acc[0]) | (to_act_bits<BF>(acc[1]) << 16);
        o.y = to_act_bits<BF>(acc[2]) | (to_act_bits<BF>(acc[3]) << 16);
        *reinterpret_cast<uint2*>(a.out + (int64_t)t * a.H + h) = o;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        __hip_atomic_store(sync_c(a, blk), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int d =
            __hip_atomic_fetch_add(sync_done(a), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = d == a.nbB - 1;
      }
      __syncthreads();
      if (*s_flag) {  // every block is combined: no wait is pending, reset the counters
        for (int i = threadIdx.x; i < a.Ep; i += DNT)
          __hip_atomic_store(sync_a(a, i), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x == 0)
          __hip_atomic_store(sync_done(a), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <bool BF, int NT, bool MIXED>
__global__ void __launch_bounds__(DNT, 2) moe_layer_kernel(LayerArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn_lds[];
  __shared__ uint32_t bitmap[MAX_BM_WORDS];
  __shared__ int s_ids[64 * MAX_ID_REGS];
  __shared__ int row_slot[64 * MAX_ID_REGS];
  __shared__ int s_flag;
  const int lane = threadIdx.x & 63;
  const int n = a.T * a.k;
  const int nw = (a.Ep + 31) >> 5;

  // 1. the routed ids into LDS (ids outside [0, E) become -1) and the
  //    active-expert bitmap (shared experts are always active)
  if (threadIdx.x < MAX_BM_WORDS) bitmap[threadIdx.x] = 0u;
  __syncthreads();
  for (int s = threadIdx.x; s < n; s += DNT) {
    const int64_t id = load_index(a.ids, a.ids_dtype, s);
    const int v = (id >= 0 && id < a.E) ? (int)id : -1;
    s_ids[s] = v;
    if (v >= 0) atomicOr(&bitmap[v >> 5], 1u << (v & 31));
  }
  if (threadIdx.x < a.Ep - a.E && a.T > 0)
    atomicOr(&bitmap[(a.E + threadIdx.x) >> 5], 1u << ((a.E + threadIdx.x) & 31));
  __syncthreads();
  const uint32_t word = lane < nw ? bitmap[lane] : 0u;
  const int c = __popc(word);
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  const int n_active = __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));

  if (n_active == 0) {  // nothing routed: the output is zero
    uint4* o = reinterpret_cast<uint4*>(a.out);
    const int64_t n16 = (int64_t)a.T * a.H / 8;
    for (int64_t i = (int64_t)blockIdx.x * DNT + threadIdx.x; i < n16; i += (int64_t)gridDim.x * DNT)
      o[i] = uint4{0u, 0u, 0u, 0u};
    return;
  }

  const int NA = n_active * a.nbA, NB = n_active * a.nbB;
  for (int u = blockIdx.x; u < NA + NB; u += gridDim.x) {
    const int ph = u >= NA;
    const int uu = ph ? u - NA : u;
    const int nb = ph ? a.nbB : a.nbA;
    const int ai = uu / nb;
    const int blk = uu - ai * nb;

    // 3. the ai-th active expert
    const uint64_t hit = __ballot(incl - c <= ai && ai < incl);
    const int wl = __ffsll((unsigned long long)hit) - 1;
    uint32_t wbits = __shfl(word, wl, 64);
    const int q0 = ai - (__shfl(incl, wl, 64) - __shfl(c, wl, 64));
    for (int t = 0; t < q0; ++t) wbits &= wbits - 1u;
    const int e = __builtin_amdgcn_readfirstlane(wl * 32 + (__ffs(wbits) - 1));

    // 4. the expert's slots in ascending order (extended slot t*kp + j), as a
    //    table in LDS.  A token routed twice to one expert (repeated ids) adds
    //    rows; cnt <= T*k <= 1024.
    __syncthreads();  // the previous unit is done with row_slot
    int cnt;
    if (e < a.E) {
      uint64_t m[MAX_ID_REGS];
      int pre[MAX_ID_REGS + 1];
      pre[0] = 0;
#pragma unroll
      for (int i = 0; i < MAX_ID_REGS; ++i) {
        m[i] = 64 * i < n ? __ballot(lane + 64 * i < n && s_ids[lane + 64 * i] == e) : 0ull;
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

    const int tier = MIXED ? (int)a.tier[e] : 2;
    if (!MIXED || tier == 2) {
      if (ph == 0)
        unit_body<2, BF, 0, NT>(a, e, blk, cnt, row_slot, dyn_lds, &s_flag, n_active);
      else
        unit_body<2, BF, 1, NT>(a, e, blk, cnt, row_slot, dyn_lds, &s_flag, n_active);
    } else if (tier == 1) {
      if (ph == 0)
        unit_body<1, BF, 0, NT>(a, e, blk, cnt, row_slot, dyn_lds, &s_flag, n_active);
      else
        unit_body<1, BF, 1, NT>(a, e, blk, cnt, row_slot, dyn_lds, &s_flag, n_active);
    } else {
      if (ph == 0)
        unit_body<0, BF, 0, NT>(a, e, blk, cnt, row_slot, dyn_lds, &s_flag, n_active);
      else
        unit_body<0, BF, 1, NT>(a, e, blk, cnt, row_slot, dyn_lds, &s_flag, n_active);
    }
  }
}

typedef void (*layer_kernel_t)(LayerArgs);

template <bool BF, int NT>
layer_kernel_t pick_nt(bool mixed) {
  return mixed ? moe_layer_kernel<BF, NT, true> : moe_layer_kernel<BF, NT, false>;
}

layer_kernel_t pick_kernel(bool bf, int nt, bool mixed) {
  if (bf) {
    if (nt == 1) return pick_nt<true, 1>(mixed);
    if (nt == 2) return pick_nt<true, 2>(mixed);
    return pick_nt<true, 4>(mixed);
  }
  if (nt == 1) return pick_nt<false, 1>(mixed);
  if (nt == 2) return pick_nt<false, 2>(mixed);
  return pick_nt<false, 4>(mixed);
}

// Co-resident work-groups per CU for (kernel, dynamic LDS), cached.
struct OccEntry {
  const void* fn;
  size_t lds;
  int dev;
  int blocks;
};
std::mutex g_occ_mu;
OccEntry g_occ[64];
int g_occ_n = 0;

int resident_blocks(layer_kernel_t fn, size_t lds, int* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(EXQ_ERROR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  {
    std::lock_guard<std::mutex> g(g_occ_mu);
    for (int i = 0; i < g_occ_n; ++i)
      if (g_occ[i].fn == (const void*)fn && g_occ[i].lds == lds && g_occ[i].dev == dev) {
        *out = g_occ[i].blocks;
        return EXQ_SUCCESS;
      }
  }
  int per_cu = 0, n_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                   DNT, lds);
  if (e != hipSuccess)
    return set_error(EXQ_ERROR_HIP, "occupancy query: %s", hipGetErrorString(e));
  e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess)
    return set_error(EXQ_ERROR_HIP, "CU count query: %s", hipGetErrorString(e));
  if (per_cu < 1 || n_cu < 1)
    return set_error(EXQ_ERROR_UNSUPPORTED, "moe_layer_kernel cannot be resident (%d per CU)",
                     per_cu);
  *out = per_cu * n_cu;
  std::lock_guard<std::mutex> g(g_occ_mu);
  if (g_occ_n < 64) g_occ[g_occ_n++] = OccEntry{(const void*)fn, lds, dev, *out};
  return EXQ_SUCCESS;
}

}  // namespace

bool decode_path_supported(int64_t T, int64_t k, int64_t Ep, int64_t n_shared, int64_t H,
                           int64_t group_size) {
  const int64_t gkb = group_size / 128;  // k-blocks per scale group: a power of two
  return T >= 1 && T <= 64 && T * k <= 64 * MAX_ID_REGS && Ep <= kDecodeMaxBuckets &&
         n_shared <= 64 && H / 32 <= kDecodeMaxHBlocks && H % 64 == 0 && gkb >= 1 &&
         (gkb & (gkb - 1)) == 0;
}

int launch_decode_layer(const DecodeLaunch& d, hipStream_t s) {
  LayerArgs a{};
  a.ids = d.ids;
  a.ids_dtype = d.ids_dtype;
  a.topk_w = d.topk_w;
  a.w_dtype = d.w_dtype;
  a.T = d.T; a.k = d.k; a.kp = d.kp; a.E = d.E; a.Ep = d.Ep;
  a.x = d.x;
  a.w13 = Proj{d.w13_bf16, d.w13_i8, d.w13_i8_scales, d.w13_i4, d.w13_i4_scales};
  a.w2 = Proj{d.w2_bf16, d.w2_i8, d.w2_i8_scales, d.w2_i4, d.w2_i4_scales};
  a.tier = d.tier;
  a.index = d.index;
  a.H = d.H;
  a.I = d.I;
  a.gshift = 0;
  while ((128 << a.gshift) < d.group_size) ++a.gshift;
  a.mid = d.mid;
  a.part = d.part;
  a.out = d.out;
  a.sync = d.sync;
  // A pass holds NT*16 rows; each wave stages its k-range of those rows in
  // an LDS region of xw 16-bit elements (at least one k-block of a full pass).
  const int nt = d.T <= 16 ? 1 : (d.T <= 32 ? 2 : 4);
  a.nbA = d.I / 16;
  a.nbB = d.H / rows_b(nt);
  const int xw_min = nt * 16 * 128;
  a.xw = xw_min > 4096 ? xw_min : 4096;
  size_t lds = (size_t)DW * a.xw * 2;
  const size_t red = (size_t)DW * (rows_b(nt) / 16) * nt * 64 * 16;
  if (red > lds) lds = red;

  layer_kernel_t fn = pick_kernel(d.bf, nt, d.tier != nullptr);
  int resident = 0;
  int st = resident_blocks(fn, lds, &resident);
  if (st) return st;
  const int64_t max_active = (int64_t)(d.T * d.k < d.E ? d.T * d.k : d.E) + (d.Ep - d.E);
  const int64_t units = max_active * (a.nbA + a.nbB);
  int64_t grid = units < resident ? units : resident;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(DNT), lds, s, a);
  return check_launch("moe_layer_kernel");
}

}  // namespace exq
