// prefill.hip -- tiled grouped GEMMs for INT4 and BF16 experts on gfx950 MFMA
// (the prefill / large-batch path of the fused layers and of the sorted-row
// GEMM entry points).
//
// Work decomposition.  One work-group computes a 128 x 128 output tile: the
// <= 128 expert-sorted rows of one token group (one expert) times 128 weight
// rows of that expert:
//   GATEUP: 64 gate rows j0..j0+63 and the matching up rows I+j0.., SiLU(g)*u
//           written to `mid` (each wave holds gate and up columns of the same j,
//           so the product is lane-local);
//   DOWN / PLAIN: 128 consecutive weight rows.
// Four waves split the tile (2 x 2 of 64 x 64, or 1 x 4 of 128 x 32); each
// wave owns its sub-tile over the whole contraction, so no cross-wave
// reduction is needed.
//
// Data movement.  The contraction runs in chunks of 128 k (one fp16 scale
// group step).  A chunk of activations (128 rows x 256 B, gathered rows for
// GATEUP) and of packed weights (128 rows x 64 B) is copied straight from
// global memory into LDS by buffer_load ... lds (16 B per lane, 64 lanes per
// 1 KiB instruction), double-buffered: chunk c+1 is in flight while chunk c
// is multiplied.  Both LDS images are XOR-swizzled in 16-byte columns so the
// MFMA operand reads (16 rows, one column) are free of bank conflicts.
//
// Arithmetic.  Lane (r, q) of an MFMA 16x16x32 operand holds 8 k values; the
// k assignment is chosen so that a lane's B values for the whole chunk are 16
// consecutive packed bytes (k = 32q + 8s + i at k-step s): one ds_read_b128
// per weight tile and chunk, and the A fragment for step s is 16 consecutive
// bytes of the staged row.  Nibbles become exact 16-bit floats 128+n (bf16)
// or 1024+n (f16) in natural k order with one v_perm_b32 and one
// v_and_or_b32 per pair; the constant base (136 / 1032) times the row's group
// sum -- precomputed by group_rowsum_kernel -- is the MFMA accumulator's
// starting value, so each group's sum is exact before the fp16 group scale
// multiplies it in fp32.
#include "exq_internal.h"

namespace exq {
namespace {

constexpr int TT = 256;              // threads per work-group (4 waves)
constexpr int KC = 128;              // contraction per chunk

typedef void __attribute__((address_space(3)))* lptr_t;

// 16 bytes per lane from buffer `r` at byte offset voff + soff into LDS at
// lds + 16 * lane (buffer_load_dwordx4 ... lds); `lds` and `soff` are
// wave-uniform.  The builtin exists only for the device target.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, int voff,
                                      int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lptr_t)lds, 16, voff, soff, 0, 0);
#endif
}

// Buffer resource over `bytes` bytes at `base`: loads beyond the range return
// zero without a memory access (a zero-length resource never touches memory).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// Waits written as volatile asm with a memory clobber so that no LDS access
// moves across them: LDS written by buffer_load ... lds is ordered only by the
// vmcnt wait, which the compiler does not model as a dependency of LDS reads.
__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Every wave's chunk has landed and every wave has finished reading the other
// stage.  (__syncthreads would add a release fence that also waits for the
// prefetch just issued.)
__device__ __forceinline__ void chunk_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

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

// 8 packed nibbles (k offsets 0..7, low nibble = even k) -> 8 exact 16-bit
// floats (base + nibble) in natural k order.  Pair j takes byte j of p (low
// nibble, k = 2j) and byte j of p >> 4 (its low nibble is k = 2j + 1).
__device__ __forceinline__ uint4 deq_nat(uint32_t p, uint32_t mask, uint32_t magic) {
  const uint32_t h = p >> 4;
  uint4 o;
  o.x = (__builtin_amdgcn_perm(h, p, 0x0c040c00u) & mask) | magic;
  o.y = (__builtin_amdgcn_perm(h, p, 0x0c050c01u) & mask) | magic;
  o.z = (__builtin_amdgcn_perm(h, p, 0x0c060c02u) & mask) | magic;
  o.w = (__builtin_amdgcn_perm(h, p, 0x0c070c03u) & mask) | magic;
  return o;
}

// Lane n of each 16-lane row, broadcast to the whole row (DPP row_newbcast).
// `n` is a constant after unrolling; the switch folds away.
template <int N>
__device__ __forceinline__ float row_bcast_n(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + N, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_bcast(float v, int n) {
  switch (n) {
    case 0: return row_bcast_n<0>(v);
    case 1: return row_bcast_n<1>(v);
    case 2: return row_bcast_n<2>(v);
    case 3: return row_bcast_n<3>(v);
    case 4: return row_bcast_n<4>(v);
    case 5: return row_bcast_n<5>(v);
    case 6: return row_bcast_n<6>(v);
    case 7: return row_bcast_n<7>(v);
    case 8: return row_bcast_n<8>(v);
    case 9: return row_bcast_n<9>(v);
    case 10: return row_bcast_n<10>(v);
    case 11: return row_bcast_n<11>(v);
    case 12: return row_bcast_n<12>(v);
    case 13: return row_bcast_n<13>(v);
    case 14: return row_bcast_n<14>(v);
    default: return row_bcast_n<15>(v);
  }
}

template <bool BF>
__device__ __forceinline__ uint32_t to_act_bits(float v) {
  return BF ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// LDS swizzles.  gfx950 serves a ds_read_b128 in four cycles of 256 bytes
// (16-byte units u = (address >> 4) & 15); the lanes served together are those
// with equal bit 5 and equal parity of bits 2..4 of the lane id (measured with
// SQ_LDS_BANK_CONFLICT over a set of access patterns).  An MFMA operand read
// (lane = row r + 16 q, column from q) is conflict-free when each such group
// of 16 lanes covers 16 distinct units; these maps of the row's low 4 bits
// achieve that:
//   activation rows (256 B, 16 columns): c ^ a_swz(r)
//   packed weight rows (64 B, 4 columns): c ^ b_swz(r)
__device__ __forceinline__ int a_swz(int r) {
  return (r & 3) | ((r >> 1) & 4) | (((r << 1) ^ r) & 8);
}
__device__ __forceinline__ int b_swz(int r) {
  return ((r >> 3) & 1) | ((((r >> 2) ^ (r >> 3)) & 1) << 1);
}

struct TileArgs {
  const float* rs;   // INT4: [K / 128][rs_rows] base * (row sum over the group)
  int rs_rows;
  int64_t x_bytes;   // bytes addressable from a.x (GATEUP gather)
  int n_tiles;       // weight tiles per expert (I / (TN / 2) for GATEUP, rows / TN otherwise)
  int h_lo, h_hi;    // INT4 tiles: token groups [hdr[h_lo], hdr[h_hi]) of the list
};

// ---- shared pieces of the tiled kernels --------------------------------------

// Unit (token group, weight tile) of this work-group over token groups
// [t0, t0 + n), in XCD-aware order: work-group i runs on XCD i % 8 and each
// XCD takes a contiguous range of units; inside it, 64 consecutive units are
// 8 token groups x 8 weight tiles, so concurrently running tiles share
// activation and weight chunks in that XCD's L2.  False: no unit.
__device__ __forceinline__ bool tile_unit(const GemmArgs& a, int t0, int n, int NT, int bid,
                                          TgEntry& te, int& nt) {
  const int U = ((n + 7) >> 3) * 8 * NT;
  const int per = (U + 7) >> 3;
  const int local = bid >> 3;
  const int v = (bid & 7) * per + local;
  if (local >= per || v >= U) return false;
  const int tb = v / (8 * NT);
  const int rem = v - tb * 8 * NT;
  nt = rem >> 3;
  const int tgi = tb * 8 + (rem & 7);
  if (tgi >= n) return false;
  te = a.tg[t0 + tgi];
  return true;
}

// Weight row (within the expert) of LDS weight row rho of tile nt, for a
// tile of TN weight rows (GATEUP: TN / 2 gate rows j0.. and the matching up rows).
template <int MODE, int TN = 128>
__device__ __forceinline__ int tile_wrow(const GemmArgs& a, int nt, int rho) {
  constexpr int HN = TN / 2;
  if constexpr (MODE == MODE_GATEUP)
    return rho < HN ? nt * HN + rho : a.inter + nt * HN + (rho - HN);
  else
    return nt * TN + rho;
}

// First LDS weight row of n-tile t of wave column wn (NTW tiles per wave) in
// a tile of TN weight rows.  GATEUP: the first half of a wave's tiles are gate
// rows, the second half the up rows of the same j.
template <int MODE, int NTW, int TN = 128>
__device__ __forceinline__ int tile_brow(int wn, int t) {
  constexpr int HALF = NTW / 2;
  constexpr int HN = TN / 2;  // gate rows of the tile
  if constexpr (MODE == MODE_GATEUP)
    return t < HALF ? wn * HALF * 16 + t * 16 : HN + wn * HALF * 16 + (t - HALF) * 16;
  else
    return wn * NTW * 16 + t * 16;
}

// Activation row (GATEUP: token) of tile row m; rows past the group repeat
// its last row (finite values whose outputs are never stored).
template <int MODE>
__device__ __forceinline__ int tile_xrow(const GemmArgs& a, const TgEntry& te, int m) {
  const int mm = m < te.cnt ? m : te.cnt - 1;
  if constexpr (MODE == MODE_GATEUP)
    return a.row_slot[te.pos0 + mm] / a.slot_div;
  else
    return te.pos0 + mm;
}

// Store a wave's finished sub-tile (rows wm*MT*16.., MFMA output layout) of a
// tile TN weight rows wide.
template <bool BF, int MODE, int MT, int NTW, int TN = 128>
__device__ __forceinline__ void tile_store(const GemmArgs& a, const TgEntry& te, int nt, int wm,
                                           int wn, int r16, int kq,
                                           const f32x4_t (&tot)[MT][NTW]) {
  constexpr int HALF = NTW / 2;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int v_ = 0; v_ < 4; ++v_) {
      const int m = wm * MT * 16 + mt * 16 + kq * 4 + v_;
      if (m >= te.cnt) continue;
      const int pos = te.pos0 + m;
      if constexpr (MODE == MODE_GATEUP) {
        uint16_t* mid = reinterpret_cast<uint16_t*>(a.out) + (int64_t)pos * a.out_stride +
                        nt * (TN / 2) + wn * HALF * 16 + r16;
#pragma unroll
        for (int t = 0; t < HALF; ++t)
          mid[t * 16] = (uint16_t)to_act_bits<BF>(silu_f32(tot[mt][t][v_]) * tot[mt][t + HALF][v_]);
      } else if constexpr (MODE == MODE_PLAIN) {
        uint16_t* c = reinterpret_cast<uint16_t*>(a.out) + (int64_t)pos * a.out_stride +
                      nt * TN + wn * NTW * 16 + r16;
#pragma unroll
        for (int t = 0; t < NTW; ++t) c[t * 16] = (uint16_t)to_act_bits<BF>(tot[mt][t][v_]);
      } else {
        const int slot = a.row_slot[pos];
        float* part = reinterpret_cast<float*>(a.out) + (int64_t)slot * a.out_stride + nt * TN +
                      wn * NTW * 16 + r16;
#pragma unroll
        for (int t = 0; t < NTW; ++t) part[t * 16] = tot[mt][t][v_];
      }
    }
  }
}

// Scheduling-group hints for one software-pipelined k-step: NM MFMAs and NV
// VALU instructions in four groups of (NM / 4 MFMAs, one of the ND LDS reads,
// VALU); the scheduler places the remaining reads.  (Groups of one, two or
// four MFMAs measured alike for Mixtral; four was about 1 % faster for the
// 64 x 256 tiles.)
template <int NM, int ND, int NV>
__device__ __forceinline__ void tile_interleave_hint() {
  constexpr int G = 4;
  static_assert(NM % G == 0, "groups");
#pragma unroll
  for (int i = 0; i < G; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, NM / G, 0);  // MFMA
    if (i < ND) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x002, (NV + G - 1) / G, 0);  // VALU
  }
}

// The same for the first k-step, which also issues the next chunk's NL copies
// and loads.
template <int NM, int ND, int NV, int NL>
__device__ __forceinline__ void tile_interleave_hint_vm() {
  constexpr int G = 4;
  static_assert(NM % G == 0, "groups");
#pragma unroll
  for (int i = 0; i < G; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, NM / G, 0);  // MFMA
    if (i < ND) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x002, (NV + G - 1) / G, 0);  // VALU
    __builtin_amdgcn_sched_group_barrier(0x020, (NL + G - 1) / G, 0);  // VMEM read
  }
}

// Hints for the last k-step of a chunk: NM MFMAs with the NV scaling VALU
// instructions one MFMA pair behind (each pair's products are ready by the
// time its scaling issues).
template <int NM, int NV>
__device__ __forceinline__ void tile_scale_hint() {
  constexpr int G = NM / 2;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
    if (i > 0) __builtin_amdgcn_sched_group_barrier(0x002, NV / G, 0);  // VALU
  }
  __builtin_amdgcn_sched_group_barrier(0x002, NV - (G - 1) * (NV / G), 0);
}

// The four waves are one row of the tile (1 x 4): each wave holds all TM =
// 16 MT token rows and NTW 16-row weight tiles, so TN = 64 NTW.
//   MT = 8, NTW = 2: 128 x 128 (each dequantised weight fragment feeds 8 MFMAs);
//   MT = 4, NTW = 4:  64 x 256 (the same MFMA work per chunk from 16 + 16 KiB of
//                     copies instead of 32 + 8 KiB: activation chunks, re-read
//                     from L2 for every weight tile, are the larger stream).
// LDS stage sizes of the INT4 tile (activations per chunk, packed weights per chunk).
template <int MT, int NTW>
constexpr int tile_a_stage() { return MT * 16 * KC * 2; }
template <int MT, int NTW>
constexpr int tile_b_stage() { return NTW * 16 * 4 * KC / 2; }

// Work-group bid of the INT4 tiles; sA* / sB* are the two stages of each operand.
template <bool BF, int MODE, int MT, int NTW>
__device__ __forceinline__ void tile_gemm_body(const GemmArgs& a, const TileArgs& ta, int bid,
                                               unsigned char* sA0, unsigned char* sA1,
                                               unsigned char* sB0, unsigned char* sB1) {
  constexpr int WAVES_N = 4;
  constexpr int TM = MT * 16, TN = NTW * 16 * WAVES_N;
  constexpr int QA = TM / 16;           // activation copies per wave and chunk (4 rows each)
  constexpr int QB = TN / 64;           // weight copies per wave and chunk (16 rows each)
  constexpr int RSR = MT / 4;           // row sums held per lane (64 rows each)

  TgEntry te;
  int nt;
  if (!tile_unit(a, a.hdr[ta.h_lo], a.hdr[ta.h_hi] - a.hdr[ta.h_lo], ta.n_tiles, bid, te, nt))
    return;  // INT4 groups [hdr[h_lo], hdr[h_hi])
  const int cnt = te.cnt, pos0 = te.pos0;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS DMA bases in SGPRs
  const int r16 = lane & 15, kq = lane >> 4;
  const int wm = 0, wn = wave;
  const int K = a.K;
  const int nch = K / KC;
  const int ngs = K / KC;  // scale groups (group_size == KC)

  const int widx = a.w.index ? a.w.index[te.e] : te.e;
  const int64_t ebase = (int64_t)widx * a.n_rows;
  const int rowbytes = K / 2;
  auto wrow = [&](int rho) { return tile_wrow<MODE, TN>(a, nt, rho); };
  auto brow = [&](int t) { return tile_brow<MODE, NTW, TN>(wn, t); };
  auto x_row = [&](int m) { return tile_xrow<MODE>(a, te, m); };

  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(a.w.i4 + ebase * rowbytes, (int64_t)a.n_rows * rowbytes);
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(a.w.i4_scales + ebase * ngs, (int64_t)a.n_rows * ngs * 2);
  const __amdgpu_buffer_rsrc_t xr =
      MODE == MODE_GATEUP
          ? make_rsrc(a.x, ta.x_bytes)
          : make_rsrc(a.x + (int64_t)pos0 * a.x_stride, (int64_t)cnt * a.x_stride * 2);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(ta.rs, (int64_t)ngs * ta.rs_rows * 4);
  const __amdgpu_buffer_rsrc_t wnull = make_rsrc(a.w.i4, 0);
  const __amdgpu_buffer_rsrc_t snull = make_rsrc(a.w.i4_scales, 0);
  const __amdgpu_buffer_rsrc_t xnull = make_rsrc(a.x, 0);
  const __amdgpu_buffer_rsrc_t rnull = make_rsrc(ta.rs, 0);

  // ---- per-lane DMA offsets ------------------------------------------------
  int voffA[QA], voffB[QB];
#pragma unroll
  for (int q = 0; q < QA; ++q) {  // LDS rows 4j..4j+3 per instruction, 16 columns each
    const int m = (wave * QA + q) * 4 + (lane >> 4);
    const int c = (lane & 15) ^ a_swz(m & 15);
    const int xrow = x_row(m);
    voffA[q] = (MODE == MODE_GATEUP ? xrow : xrow - pos0) * (int)a.x_stride * 2 + c * 16;
  }
#pragma unroll
  for (int q = 0; q < QB; ++q) {  // LDS rows 16j..16j+15 per instruction, 4 columns each
    const int rho = (wave * QB + q) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ b_swz(rho & 15);
    voffB[q] = wrow(rho) * rowbytes + c * 16;
  }
  // Scale of weight row wrow(brow(t) + r16): lane part + a wave-uniform delta.
  const int soffS = wrow(brow(0) + r16) * ngs * 2;
  int sdel[NTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
    sdel[t] = __builtin_amdgcn_readfirstlane((wrow(brow(t) + r16) - wrow(brow(0) + r16)) * ngs * 2);
  // Row sums: lane kq*16 + n holds tile row (n >> 2) * 16 + kq * 4 + (n & 3)
  // (+ 64 per register), so that the accumulator start of m-tile mt, element
  // v, is lane mt*4 + v of the lane's own 16-lane row (DPP row_newbcast).
  int soffR[RSR];
#pragma unroll
  for (int i = 0; i < RSR; ++i)
    soffR[i] = x_row(wm * MT * 16 + i * 64 + (r16 >> 2) * 16 + kq * 4 + (r16 & 3)) * 4;

  // LDS read offsets: A fragment of k-step s = aoff ^ (16 s) (+ 4 KiB per
  // m-tile); weight tile t = boff + bdel(t).
  const int aoff = (wm * MT * 16 + r16) * 256 + (((kq * 4) ^ a_swz(r16)) * 16);
  const int boff = (brow(0) + r16) * 64 + ((kq ^ b_swz(r16)) * 16);
  uint32_t sc_raw[2][NTW];
  float rs_raw[2][RSR];

  auto prefetch = [&](int st, int ch) {
    const bool ok = ch < nch;
    const int chl = ok ? ch : 0;
    const int g = chl;
    unsigned char* A = st ? sA1 : sA0;
    unsigned char* B = st ? sB1 : sB0;
#pragma unroll
    for (int q = 0; q < QA; ++q) dma16(ok ? xr : xnull, A + (wave * QA + q) * 1024, voffA[q], chl * 256);
#pragma unroll
    for (int q = 0; q < QB; ++q) dma16(ok ? wr : wnull, B + (wave * QB + q) * 1024, voffB[q], chl * 64);
#pragma unroll
    for (int t = 0; t < NTW; ++t)
      sc_raw[st][t] =
          __builtin_amdgcn_raw_buffer_load_b16(ok ? sr : snull, soffS, g * 2 + sdel[t], 0);
#pragma unroll
    for (int i = 0; i < RSR; ++i)
      rs_raw[st][i] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(ok ? rr : rnull, soffR[i], g * ta.rs_rows * 4, 0));
  };

  const uint32_t dq_mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(dq_magic));  // magic in a VGPR: one v_and_or_b32 per pair

  f32x4_t tot[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTW; ++t) tot[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One chunk (= one scale group): the accumulators start from the base
  // correction and end scaled into tot.  Software-pipelined by k-step: while
  // step s's MT x NTW MFMAs issue, step s + 1's activation fragments are read
  // from LDS and its weight fragments dequantised (both independent of the
  // MFMAs in flight), and scheduling-group hints interleave the three streams
  // so that the VALU and LDS work issues in the matrix pipe's shadow.
#define EXQ_TILE_CHUNK(ST, PF)                                                               \
  do {                                                                                       \
    const unsigned char* A_ = ST ? sA1 : sA0;                                                \
    const unsigned char* B_ = ST ? sB1 : sB0;                                                \
    uint4 bw[NTW];                                                                           \
    _Pragma("unroll") for (int t = 0; t < NTW; ++t)                                          \
        bw[t] = *reinterpret_cast<const uint4*>(B_ + boff + (brow(t) - brow(0)) * 64);      \
    uint4 afp[2][MT], bfp[2][NTW];                                                           \
    _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                        \
        afp[0][mt] = *reinterpret_cast<const uint4*>(A_ + aoff + mt * 16 * 256);             \
    _Pragma("unroll") for (int t = 0; t < NTW; ++t)                                          \
        bfp[0][t] = deq_nat(bw[t].x, dq_mask, dq_magic);                                     \
    __builtin_amdgcn_sched_barrier(0);                                                       \
    _Pragma("unroll") for (int s = 0; s < 4; ++s) {                                          \
      const int c_ = s & 1, n_ = c_ ^ 1;                                                     \
      if (s < 3) {                                                                           \
        _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                    \
            afp[n_][mt] =                                                                    \
                *reinterpret_cast<const uint4*>(A_ + (aoff ^ ((s + 1) * 16)) + mt * 16 * 256); \
        _Pragma("unroll") for (int t = 0; t < NTW; ++t) {                                    \
          const uint32_t p_ = s == 0 ? bw[t].y : s == 1 ? bw[t].z : bw[t].w;                 \
          bfp[n_][t] = deq_nat(p_, dq_mask, dq_magic);                                       \
        }                                                                                    \
      }                                                                                      \
      _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                      \
          _Pragma("unroll") for (int t = 0; t < NTW; ++t)                                    \
              acc[mt][t] = mfma16<BF>(afp[c_][mt], bfp[c_][t], acc[mt][t]);                  \
      if (s == 0) {                                                                          \
        PF;                                                                                  \
        tile_interleave_hint_vm<MT * NTW, MT, 9 * NTW, QA + QB + NTW + RSR>();               \
      } else if (s < 3) {                                                                    \
        tile_interleave_hint<MT * NTW, MT, 9 * NTW>();                                       \
      } else {                                                                               \
        /* each accumulator's scaling follows its last MFMA, under the later ones */         \
        _Pragma("unroll") for (int t = 0; t < NTW; ++t) {                                    \
          const float sc_ = f16_bits_to_f32(sc_raw[ST][t]);                                  \
          _Pragma("unroll") for (int mt = 0; mt < MT; ++mt) tot[mt][t] += sc_ * acc[mt][t];  \
        }                                                                                    \
        tile_scale_hint<MT * NTW, 4 * MT * NTW + NTW>();                                     \
      }                                                                                      \
      __builtin_amdgcn_sched_barrier(0);                                                     \
    }                                                                                        \
  } while (0)

  // Per chunk: wait for this wave's copies of the chunk (and its row sums),
  // set the accumulators to the chunk's base correction (registers only, so
  // before the barrier), then the barrier; the next chunk's copies go out
  // inside the first k-step, among its MFMAs.
  f32x4_t acc[MT][NTW];
  auto start_chunk = [&](int st) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4_t c_;
#pragma unroll
      for (int v_ = 0; v_ < 4; ++v_) c_[v_] = row_bcast(rs_raw[st][mt >> 2], (mt & 3) * 4 + v_);
#pragma unroll
      for (int t = 0; t < NTW; ++t) acc[mt][t] = c_;
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  prefetch(0, 0);
  for (int ch = 0; ch < nch; ch += 2) {
    start_chunk(0);
    EXQ_TILE_CHUNK(0, prefetch(1, ch + 1));
    if (ch + 1 >= nch) break;
    start_chunk(1);
    EXQ_TILE_CHUNK(1, prefetch(0, ch + 2));
  }
#undef EXQ_TILE_CHUNK
  wait_vm_all();  // the last (empty) prefetch has drained before the work-group ends

  tile_store<BF, MODE, MT, NTW, TN>(a, te, nt, wm, wn, r16, kq, tot);
}

// ---- INT4 experts, scaled weight operands ------------------------------------
// 128 sorted rows x 256 weight rows per work-group, four waves of 128 x 64
// (4 x 2 MFMA 32x32x16 tiles).  Each weight fragment is dequantised with its
// group scale applied, (n - 8) * s rounded once to the operand type (for f16
// operands this is the value the reference's kernel multiplies,
// moe_int4_kernel.py:211-233), so the fp32 accumulators run over the whole
// contraction: no per-group accumulator set, no base correction and no row-sum
// pass.  That halves the accumulator registers per output, which is what lets
// a wave hold 128 x 64 outputs at two waves per SIMD: every activation chunk
// copied into LDS feeds 256 weight rows, twice the 128 x 128 tile's reuse.
//
// Data movement: activations in 64-k chunks (128 rows x 128 B, 16 KiB), packed
// weights one scale group at a time (256 rows x 64 B, 16 KiB), both double
// buffered (64 KiB per work-group, two work-groups per CU): the next
// activation chunk is copied during the current one, the next group's weights
// during the first chunk of the current group, two chunks ahead of their use.
//
// MFMA 32x32x16 operands: lane l holds row / column l % 32 and 8 k values of
// half h = l / 32.  At k-step s (four per chunk) of chunk half c of a group,
// lane half h covers group-relative k = 64 c + 32 h + 8 s + i, so a lane's
// packed bytes for a whole chunk are 16 consecutive bytes (one ds_read_b128
// per weight tile and chunk), and its activation fragment for step s is 16
// consecutive bytes of the staged row.
constexpr int PS_KC = 64;                    // activation chunk (k)
constexpr int PS_A_STAGE = 128 * PS_KC * 2;  // 16 KiB
constexpr int PS_B_ROW = 64;                 // one 128-k group of a packed weight row

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Swizzles for the 32-lane operand rows (same bank-group rule as above: each
// group of 16 lanes served together covers 16 distinct 16-byte units).
//   activation rows (128 B, 8 columns): c ^ psa_swz(r)
//   packed weight rows (64 B, 4 columns): c ^ psb_swz(r)
__device__ __forceinline__ int psa_swz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int psb_swz(int r) { return (r >> 2) & 3; }

template <bool BF>
__device__ __forceinline__ f32x16_t mfma32(const uint4& a, const uint4& b, f32x16_t c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

// Per-lane scale constants of one weight row and group.
struct PsScale {
  float s, s16, c;  // bf16: s, s / 16, -8 s
  uint32_t s2;      // f16: s in both halves
};

template <bool BF>
__device__ __forceinline__ PsScale ps_scale(uint32_t raw) {
  PsScale p;
  if constexpr (BF) {
    p.s = f16_bits_to_f32(raw & 0xffffu);
    p.s16 = p.s * 0.0625f;
    p.c = -8.0f * p.s;
    p.s2 = 0;
  } else {
    p.s = p.s16 = p.c = 0.f;
    p.s2 = __builtin_amdgcn_perm(raw, raw, 0x01000100u);
  }
  return p;
}

// 8 packed nibbles (k offsets 0..7, low nibble = even k) -> the 8 operand
// values (n - 8) * s in natural k order.
//   bf16: the exact product in fp32 (n from v_cvt_f32_ubyte*, the high nibbles
//         as 16 n against s / 16), one rounding by v_cvt_pk_bf16_f32;
//   f16:  the exact 1024 + n pair (v_perm_b32 + v_and_or_b32), minus 1032
//         (exact), times s: one f16 rounding, the reference's product.
template <bool BF>
__device__ __forceinline__ uint4 deq_scaled(uint32_t p, const PsScale& sc, uint32_t mask,
                                            uint32_t magic) {
  uint4 o;
  if constexpr (BF) {
    uint32_t lo = p & 0x0F0F0F0Fu, hi = p & 0xF0F0F0F0u;
    asm volatile("" : "+v"(lo), "+v"(hi));  // keep whole-byte conversions (v_cvt_f32_ubyteN)
    auto pk = [](float a, float b) {
      const f32x2_t v = {a, b};
      return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    };
    o.x = pk(__builtin_fmaf((float)(lo & 0xffu), sc.s, sc.c),
             __builtin_fmaf((float)(hi & 0xffu), sc.s16, sc.c));
    o.y = pk(__builtin_fmaf((float)((lo >> 8) & 0xffu), sc.s, sc.c),
             __builtin_fmaf((float)((hi >> 8) & 0xffu), sc.s16, sc.c));
    o.z = pk(__builtin_fmaf((float)((lo >> 16) & 0xffu), sc.s, sc.c),
             __builtin_fmaf((float)((hi >> 16) & 0xffu), sc.s16, sc.c));
    o.w = pk(__builtin_fmaf((float)(lo >> 24), sc.s, sc.c),
             __builtin_fmaf((float)(hi >> 24), sc.s16, sc.c));
  } else {
    const uint4 e = deq_nat(p, mask, magic);  // 1024 + n
    const f16x2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const f16x2_t s2 = __builtin_bit_cast(f16x2_t, sc.s2);
    o.x = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2_t, e.x) + off) * s2);
    o.y = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2_t, e.y) + off) * s2);
    o.z = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2_t, e.z) + off) * s2);
    o.w = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2_t, e.w) + off) * s2);
  }
  return o;
}

// First LDS weight row of 32-row tile t (0, 1) of wave wn in a tile of TN
// weight rows.  GATEUP: tile 0 the gate rows j0 + 32 wn.., tile 1 the matching
// up rows (LDS rows TN / 2..).
template <int MODE, int TN>
__device__ __forceinline__ int ps_brow(int wn, int t) {
  if constexpr (MODE == MODE_GATEUP)
    return t * (TN / 2) + wn * 32;
  else
    return wn * 64 + t * 32;
}

// Four waves of 128 x 64, two work-groups per CU.  (Eight waves of 128 x 64 in
// one work-group per CU, each activation chunk feeding 512 weight rows,
// measured 8 % slower for Mixtral: every chunk's barrier then holds all the
// CU's waves.)
constexpr int PS_B_STAGE = TT * PS_B_ROW;     // weight rows of the tile x one group

template <bool BF, int MODE>
__device__ __forceinline__ void tile_ps_body(const GemmArgs& a, const TileArgs& ta, int bid,
                                             unsigned char* sA0, unsigned char* sA1,
                                             unsigned char* sB0, unsigned char* sB1) {
  constexpr int W = TT / 64;
  constexpr int MT = 4, NT = 2, TN = 64 * W;
  constexpr int QA = 16 / W;                    // activation copies per wave and chunk

  TgEntry te;
  int nt;
  if (!tile_unit(a, a.hdr[ta.h_lo], a.hdr[ta.h_hi] - a.hdr[ta.h_lo], ta.n_tiles, bid, te, nt))
    return;  // INT4 groups [hdr[h_lo], hdr[h_hi])
  const int cnt = te.cnt, pos0 = te.pos0;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;
  const int wn = wave;
  const int K = a.K;
  const int nch = K / PS_KC;  // activation chunks, two per scale group
  const int ngs = K / KC;     // scale groups (group_size == 128)

  const int widx = a.w.index ? a.w.index[te.e] : te.e;
  const int64_t ebase = (int64_t)widx * a.n_rows;
  const int rowbytes = K / 2;
  auto wrow = [&](int rho) { return tile_wrow<MODE, TN>(a, nt, rho); };
  auto x_row = [&](int m) { return tile_xrow<MODE>(a, te, m); };

  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(a.w.i4 + ebase * rowbytes, (int64_t)a.n_rows * rowbytes);
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(a.w.i4_scales + ebase * ngs, (int64_t)a.n_rows * ngs * 2);
  const __amdgpu_buffer_rsrc_t xr =
      MODE == MODE_GATEUP
          ? make_rsrc(a.x, ta.x_bytes)
          : make_rsrc(a.x + (int64_t)pos0 * a.x_stride, (int64_t)cnt * a.x_stride * 2);
  const __amdgpu_buffer_rsrc_t wnull = make_rsrc(a.w.i4, 0);
  const __amdgpu_buffer_rsrc_t snull = make_rsrc(a.w.i4_scales, 0);
  const __amdgpu_buffer_rsrc_t xnull = make_rsrc(a.x, 0);

  // ---- per-lane DMA offsets ------------------------------------------------
  // activations: instruction q fills LDS rows 8j..8j+7 (j = QA wave + q), 8 columns each;
  // weights: instruction q fills LDS rows 16j..16j+15 (j = 4 wave + q), 4 columns each.
  int voffA[QA], voffB[4];
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int m = (wave * QA + q) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ psa_swz(m);
    const int xrow = x_row(m);
    voffA[q] = (MODE == MODE_GATEUP ? xrow : xrow - pos0) * (int)a.x_stride * 2 + c * 16;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rho = (wave * 4 + q) * 16 + (lane >> 2);
    const int cb = (lane & 3) ^ psb_swz(rho);
    voffB[q] = wrow(rho) * rowbytes + cb * 16;
  }
  // Scale of weight row wrow(ps_brow(t) + r32): lane part + a wave-uniform delta.
  const int soffS = wrow(ps_brow<MODE, TN>(wn, 0) + r32) * ngs * 2;
  int sdel[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    sdel[t] = __builtin_amdgcn_readfirstlane(
        (wrow(ps_brow<MODE, TN>(wn, t) + r32) - wrow(ps_brow<MODE, TN>(wn, 0) + r32)) * ngs * 2);

  // LDS read offsets: A fragment of m-tile mt, k-step s = aoff ^ (16 s) + 4 KiB mt;
  // weight tile t, chunk half c = (boff + brow(t) * 64) ^ (32 c).
  const int aoff = r32 * 128 + ((4 * h) ^ psa_swz(r32)) * 16;
  const int boff = r32 * 64 + (h ^ psb_swz(r32)) * 16;
  uint32_t sc_raw[NT];

  auto prefetch_a = [&](int st, int ch) {
    const bool ok = ch < nch;
    const int chl = ok ? ch : 0;
    unsigned char* A = st ? sA1 : sA0;
#pragma unroll
    for (int q = 0; q < QA; ++q) dma16(ok ? xr : xnull, A + (wave * QA + q) * 1024, voffA[q], chl * 128);
  };
  auto prefetch_b = [&](int st, int g) {
    const bool ok = g < ngs;
    const int gl = ok ? g : 0;
    unsigned char* B = st ? sB1 : sB0;
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16(ok ? wr : wnull, B + (wave * 4 + q) * 1024, voffB[q], gl * 64);
  };
  auto prefetch_scales = [&](int g) {
    const bool ok = g < ngs;
    const int gl = ok ? g : 0;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      sc_raw[t] = __builtin_amdgcn_raw_buffer_load_b16(ok ? sr : snull, soffS, gl * 2 + sdel[t], 0);
  };
  // The next group's loads: its scales and the next activation chunk, then,
  // after an ordering fence, its 4 weight copies.  The fence (no memory access
  // and no instruction crosses it) makes those 4 copies the only loads issued
  // after the activation chunk's, whatever the compiler drops (the scales of
  // a group past the end are never used) or reorders before it.
  auto prefetch_group = [&](int st, int g, int ch) {
    prefetch_scales(g);
    prefetch_a(1, ch);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    prefetch_b(st, g);
  };

  const uint32_t dq_mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t dq_magic = 0x64006400u;
  asm volatile("" : "+v"(dq_magic));

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][t][v] = 0.f;

  // Copies in flight: the next activation chunk, and the weights and scales
  // of the next group from the first chunk of a group on (two chunks ahead).
  // A chunk's own copies have landed when none (first chunk of a group) or
  // only the next group's 4 weight copies (second chunk, issued after its
  // copies) of the wave's loads are outstanding.
  PsScale sc[NT];
  auto start_chunk = [&](int half) {
    if (half == 0)
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
    if (half == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) sc[t] = ps_scale<BF>(sc_raw[t]);
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // One 64-k chunk: activation stage AS, weight stage BS, half HF of the group.
#define EXQ_PS_CHUNK(AS, BS, HF, PF)                                                         \
  do {                                                                                       \
    const unsigned char* A_ = AS ? sA1 : sA0;                                                \
    const unsigned char* B_ = BS ? sB1 : sB0;                                                \
    uint4 bw[NT];                                                                            \
    _Pragma("unroll") for (int t = 0; t < NT; ++t)                                           \
        bw[t] = *reinterpret_cast<const uint4*>(                                             \
            B_ + ((boff + ps_brow<MODE, TN>(wn, t) * 64) ^ (32 * HF)));                      \
    uint4 af[2][MT], wf[2][NT];                                                              \
    _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                        \
        af[0][mt] = *reinterpret_cast<const uint4*>(A_ + aoff + mt * 32 * 128);              \
    _Pragma("unroll") for (int t = 0; t < NT; ++t)                                           \
        wf[0][t] = deq_scaled<BF>(bw[t].x, sc[t], dq_mask, dq_magic);                        \
    _Pragma("unroll") for (int s = 0; s < 4; ++s) {                                          \
      const int c_ = s & 1, n_ = c_ ^ 1;                                                     \
      if (s < 3) {                                                                           \
        _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                    \
            af[n_][mt] =                                                                     \
                *reinterpret_cast<const uint4*>(A_ + (aoff ^ ((s + 1) * 16)) + mt * 32 * 128); \
        _Pragma("unroll") for (int t = 0; t < NT; ++t) {                                     \
          const uint32_t p_ = s == 0 ? bw[t].y : s == 1 ? bw[t].z : bw[t].w;                 \
          wf[n_][t] = deq_scaled<BF>(p_, sc[t], dq_mask, dq_magic);                          \
        }                                                                                    \
      }                                                                                      \
      _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                      \
          _Pragma("unroll") for (int t = 0; t < NT; ++t)                                     \
              acc[mt][t] = mfma32<BF>(af[c_][mt], wf[c_][t], acc[mt][t]);                    \
      if (s == 0) { PF; }                                                                    \
      __builtin_amdgcn_sched_barrier(0);                                                     \
    }                                                                                        \
  } while (0)

  // One scale group = two activation chunks.  The weight stage is a constant
  // in each copy of the group body (two groups per iteration, an odd last
  // group after the loop) so that the compiler can tell the stages apart and
  // does not wait for the other stage's copies before reading this one.
#define EXQ_PS_GROUP(G, BS)                                                                  \
  do {                                                                                       \
    start_chunk(0);                                                                          \
    EXQ_PS_CHUNK(0, BS, 0, prefetch_group((BS) ^ 1, (G) + 1, 2 * (G) + 1));                  \
    start_chunk(1);                                                                          \
    EXQ_PS_CHUNK(1, BS, 1, prefetch_a(0, 2 * (G) + 2));                                      \
  } while (0)
  prefetch_scales(0);
  prefetch_a(0, 0);
  prefetch_b(0, 0);
  int g = 0;
  for (; g + 1 < ngs; g += 2) {
    EXQ_PS_GROUP(g, 0);
    EXQ_PS_GROUP(g + 1, 1);
  }
  if (g < ngs) EXQ_PS_GROUP(g, 0);
#undef EXQ_PS_GROUP
#undef EXQ_PS_CHUNK
  wait_vm_all();  // the last (empty) prefetch has drained before the work-group ends

  // Output: accumulator v of tile (mt, t) is row 32 mt + 8 (v / 4) + 4 h + v % 4,
  // column r32 of the tile.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = mt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
      if (m >= cnt) continue;
      const int pos = pos0 + m;
      if constexpr (MODE == MODE_GATEUP) {
        uint16_t* mid = reinterpret_cast<uint16_t*>(a.out) + (int64_t)pos * a.out_stride +
                        nt * (TN / 2) + wn * 32 + r32;
        *mid = (uint16_t)to_act_bits<BF>(silu_f32(acc[mt][0][v]) * acc[mt][1][v]);
      } else if constexpr (MODE == MODE_PLAIN) {
        uint16_t* c = reinterpret_cast<uint16_t*>(a.out) + (int64_t)pos * a.out_stride + nt * TN +
                      wn * 64 + r32;
#pragma unroll
        for (int t = 0; t < NT; ++t) c[t * 32] = (uint16_t)to_act_bits<BF>(acc[mt][t][v]);
      } else {
        const int slot = a.row_slot[pos];
        float* part = reinterpret_cast<float*>(a.out) + (int64_t)slot * a.out_stride + nt * TN +
                      wn * 64 + r32;
#pragma unroll
        for (int t = 0; t < NT; ++t) part[t * 32] = acc[mt][t][v];
      }
    }
  }
}

// ---- BF16 experts ------------------------------------------------------------
// Same tile and unit order over the BF16 token groups [0, hdr[2]); chunks of
// 64 k: activations and weights both 128 rows x 128 B per stage, swizzled in
// 16-byte columns with c ^ f(r), f(r) = (r ^ (r >> 3)) & 7 (measured free of
// bank conflicts for the operand reads).  Lane (r, q) at k-step s holds k = 16q + 8s .. +7 of both operands;
// the fp32 accumulators run over the whole contraction.
constexpr int KCB = 64;
constexpr int AB_STAGE = 128 * KCB * 2;  // 16 KiB per operand and stage

__device__ __forceinline__ int bf_swz(int r) { return (r ^ (r >> 3)) & 7; }

template <bool BF, int MODE>
__device__ __forceinline__ void tile_gemm_bf16_body(const GemmArgs& a, const TileArgs& ta, int bid,
                                                    unsigned char* sA0, unsigned char* sA1,
                                                    unsigned char* sB0, unsigned char* sB1) {
  constexpr int MT = 4, NTW = 4, WAVES_N = 2;

  TgEntry te;
  int nt;
  if (!tile_unit(a, 0, a.hdr[2], ta.n_tiles, bid, te, nt)) return;  // BF16 groups
  const int cnt = te.cnt, pos0 = te.pos0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int K = a.K;
  const int nch = K / KCB;
  const int widx = a.w.index ? a.w.index[te.e] : te.e;
  const int64_t ebase = (int64_t)widx * a.n_rows;
  const int rowbytes = K * 2;

  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(a.w.bf16 + ebase * K, (int64_t)a.n_rows * rowbytes);
  const __amdgpu_buffer_rsrc_t xr =
      MODE == MODE_GATEUP
          ? make_rsrc(a.x, ta.x_bytes)
          : make_rsrc(a.x + (int64_t)pos0 * a.x_stride, (int64_t)cnt * a.x_stride * 2);
  const __amdgpu_buffer_rsrc_t wnull = make_rsrc(a.w.bf16, 0);
  const __amdgpu_buffer_rsrc_t xnull = make_rsrc(a.x, 0);

  // DMA: instruction q of this wave fills LDS rows 8j..8j+7 (j = 4 wave + q),
  // 8 columns each.
  int voffA[4], voffB[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (wave * 4 + q) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ bf_swz(r & 15);
    const int xrow = tile_xrow<MODE>(a, te, r);
    voffA[q] = (MODE == MODE_GATEUP ? xrow : xrow - pos0) * (int)a.x_stride * 2 + c * 16;
    voffB[q] = tile_wrow<MODE>(a, nt, r) * rowbytes + c * 16;
  }
  // Fragment of k-step s: column (2 kq + s) ^ f(r16) of the row.
  const int colx = ((kq * 2) ^ bf_swz(r16)) * 16;
  const int aoff = (wm * MT * 16 + r16) * 128 + colx;
  const int boff = (tile_brow<MODE, NTW>(wn, 0) + r16) * 128 + colx;

  auto prefetch = [&](int st, int ch) {
    const bool ok = ch < nch;
    const int chl = ok ? ch : 0;
    unsigned char* A = st ? sA1 : sA0;
    unsigned char* B = st ? sB1 : sB0;
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16(ok ? xr : xnull, A + (wave * 4 + q) * 1024, voffA[q], chl * 128);
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16(ok ? wr : wnull, B + (wave * 4 + q) * 1024, voffB[q], chl * 128);
  };

  f32x4_t acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTW; ++t) acc[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#define EXQ_BF_CHUNK(ST)                                                                      \
  do {                                                                                        \
    const unsigned char* A_ = ST ? sA1 : sA0;                                                 \
    const unsigned char* B_ = ST ? sB1 : sB0;                                                 \
    _Pragma("unroll") for (int s = 0; s < 2; ++s) {                                           \
      uint4 af[MT], bf[NTW];                                                                  \
      _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                       \
          af[mt] = *reinterpret_cast<const uint4*>(A_ + (aoff ^ (s * 16)) + mt * 16 * 128);   \
      _Pragma("unroll") for (int t = 0; t < NTW; ++t)                                         \
          bf[t] = *reinterpret_cast<const uint4*>(                                            \
              B_ + (boff ^ (s * 16)) +                                                        \
              (tile_brow<MODE, NTW>(wn, t) - tile_brow<MODE, NTW>(wn, 0)) * 128);             \
      _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                       \
          _Pragma("unroll") for (int t = 0; t < NTW; ++t)                                     \
              acc[mt][t] = mfma16<BF>(af[mt], bf[t], acc[mt][t]);                             \
    }                                                                                         \
  } while (0)

  prefetch(0, 0);
  for (int ch = 0; ch < nch; ch += 2) {
    chunk_barrier();
    prefetch(1, ch + 1);
    __builtin_amdgcn_sched_barrier(0);
    EXQ_BF_CHUNK(0);
    if (ch + 1 >= nch) break;
    chunk_barrier();
    prefetch(0, ch + 2);
    __builtin_amdgcn_sched_barrier(0);
    EXQ_BF_CHUNK(1);
  }
#undef EXQ_BF_CHUNK
  wait_vm_all();
  tile_store<BF, MODE, MT, NTW>(a, te, nt, wm, wn, r16, kq, acc);
}

// out[g][r] = base * sum_{k in group g} x[r, k] (fp32 sums of the 16-bit
// values) for base = -136 (bf16) or -1032 (f16): the accumulator start of the
// tiled kernel.  One work-group per row; 16 lanes cover one 128-element block.
template <bool BF>
__global__ void __launch_bounds__(256) group_rowsum_kernel(const uint16_t* __restrict__ x,
                                                           int64_t stride, int R, int K, int gs,
                                                           float base, float* __restrict__ out) {
  __shared__ float bs[512];
  const int r = blockIdx.x;
  const uint16_t* row = x + (int64_t)r * stride;
  const int np = K / 8;  // 16-byte pieces, a multiple of 16
  for (int p0 = 0; p0 < np; p0 += 256) {
    const int p = p0 + (int)threadIdx.x;
    float s = 0.f;
    if (p < np) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + (int64_t)p * 8);
      const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (BF)
          s += __uint_as_float(d[i] << 16) + __uint_as_float(d[i] & 0xffff0000u);
        else
          s += f16_bits_to_f32(d[i] & 0xffffu) + f16_bits_to_f32(d[i] >> 16);
      }
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    s += __shfl_xor(s, 8, 64);
    if (p < np && (threadIdx.x & 15) == 0) bs[p >> 4] = s;
  }
  __syncthreads();
  const int ng = K / gs, nb = gs / 128;
  for (int g = threadIdx.x; g < ng; g += 256) {
    float s = 0.f;
    for (int i = 0; i < nb; ++i) s += bs[g * nb + i];
    out[(int64_t)g * R + r] = base * s;
  }
}

// The same sums for the expert-sorted rows of token groups [hdr[3], hdr[0])
// only (the 64 x 256 INT4 tiles' groups; the scaled-operand and BF16 tiles
// read none): work-group b takes rows 8 (b % 16) .. +7 of group b / 16 (<= 128
// rows per group), 16 lanes per (row, 128-k block) cell; a lane's loads for
// up to eight cells go out together.
constexpr int kRowsumTgRows = 8;
constexpr int kRowsumTgParts = kTokenGroupI4 / kRowsumTgRows;

template <bool BF>
__global__ void __launch_bounds__(256) group_rowsum_tg_kernel(const uint16_t* __restrict__ x,
                                                              int64_t stride, int K, float base,
                                                              const int* __restrict__ hdr,
                                                              const TgEntry* __restrict__ tg,
                                                              int rs_rows, float* __restrict__ out) {
  const int g = (int)(blockIdx.x / kRowsumTgParts);
  const int r0 = (int)(blockIdx.x % kRowsumTgParts) * kRowsumTgRows;
  const int lo = hdr[3];
  if (g >= hdr[0] - lo) return;
  const TgEntry te = tg[lo + g];
  const int nr = min(kRowsumTgRows, te.cnt - r0);
  if (nr <= 0) return;
  const int nblk = K / 128;  // 128-k blocks per row
  const int cells = nr * nblk;
  const int lane16 = threadIdx.x & 15, c0 = threadIdx.x >> 4;
  constexpr int U = 8;
  for (int cb = 0; cb < cells; cb += 16 * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * 16 + c0;
      v[u] = make_uint4(0u, 0u, 0u, 0u);
      if (c < cells) {
        const int r = c / nblk, kb = c - r * nblk;
        v[u] = *reinterpret_cast<const uint4*>(x + (int64_t)(te.pos0 + r0 + r) * stride +
                                               kb * 128 + lane16 * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t d[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (BF)
          sum += __uint_as_float(d[i] << 16) + __uint_as_float(d[i] & 0xffff0000u);
        else
          sum += f16_bits_to_f32(d[i] & 0xffffu) + f16_bits_to_f32(d[i] >> 16);
      }
      sum += __shfl_xor(sum, 1, 64);
      sum += __shfl_xor(sum, 2, 64);
      sum += __shfl_xor(sum, 4, 64);
      sum += __shfl_xor(sum, 8, 64);
      const int c = cb + u * 16 + c0;
      if (c < cells && lane16 == 0) {
        const int r = c / nblk, kb = c - r * nblk;
        out[(int64_t)kb * rs_rows + te.pos0 + r0 + r] = base * sum;
      }
    }
  }
}

// ---- kernels ------------------------------------------------------------------
// Each stage array is its own LDS object, so the compiler can tell that reading
// one stage cannot touch another's pending copy.
template <bool BF, int MODE, int MT, int NTW>
__global__ void __launch_bounds__(TT, 2) tile_gemm_kernel(GemmArgs a, TileArgs ta) {
  __shared__ __attribute__((aligned(1024))) unsigned char sA0[tile_a_stage<MT, NTW>()];
  __shared__ __attribute__((aligned(1024))) unsigned char sA1[tile_a_stage<MT, NTW>()];
  __shared__ __attribute__((aligned(1024))) unsigned char sB0[tile_b_stage<MT, NTW>()];
  __shared__ __attribute__((aligned(1024))) unsigned char sB1[tile_b_stage<MT, NTW>()];
  tile_gemm_body<BF, MODE, MT, NTW>(a, ta, blockIdx.x, sA0, sA1, sB0, sB1);
}

template <bool BF, int MODE>
__global__ void __launch_bounds__(TT, 2) tile_ps_kernel(GemmArgs a, TileArgs ta) {
  __shared__ __attribute__((aligned(1024))) unsigned char sA0[PS_A_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sA1[PS_A_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sB0[PS_B_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sB1[PS_B_STAGE];
  tile_ps_body<BF, MODE>(a, ta, blockIdx.x, sA0, sA1, sB0, sB1);
}

template <bool BF, int MODE>
__global__ void __launch_bounds__(TT, 2) tile_gemm_bf16_kernel(GemmArgs a, TileArgs ta) {
  __shared__ __attribute__((aligned(1024))) unsigned char sA0[AB_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sA1[AB_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sB0[AB_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sB1[AB_STAGE];
  tile_gemm_bf16_body<BF, MODE>(a, ta, blockIdx.x, sA0, sA1, sB0, sB1);
}

// Work-groups of tile_unit's unit range over n token groups (a multiple of
// eight groups times the weight tiles per group).
__device__ __forceinline__ int tile_unit_count(int n, int n_tiles) {
  return ((n + 7) >> 3) * 8 * n_tiles;
}

// The tiles of one projection in one grid, in three ranges whose sizes come
// from the token-group list on the device: 128 x 256 scaled-operand INT4 tiles
// over the big-group INT4 experts [hdr[1], hdr[3]), 64 x 256 INT4 tiles over
// the other INT4 experts [hdr[3], hdr[0]), then BF16 tiles over [0, hdr[2]).
// All three take 16 KiB per operand stage, so the LDS is shared.  The host
// sizes the grid from upper bounds; the work-groups past the three ranges
// return at once, after every real unit in dispatch order.  The longest units
// (the big experts' 128-row tiles) go first and the BF16 units fill the last,
// partly empty round of the INT4 ones (DeepSeek-V2-Lite's INT4 gate/up at
// 2048 tokens is several rounds of the 512 resident work-groups).
template <bool BF, int MODE>
__global__ void __launch_bounds__(TT, 2) tile_mix_kernel(GemmArgs a, TileArgs tps, TileArgs t64,
                                                         TileArgs tbf) {
  static_assert(tile_a_stage<4, 4>() == AB_STAGE && tile_b_stage<4, 4>() == AB_STAGE &&
                    PS_A_STAGE == AB_STAGE && PS_B_STAGE == AB_STAGE,
                "one LDS layout for the three tiles");
  __shared__ __attribute__((aligned(1024))) unsigned char sA0[AB_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sA1[AB_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sB0[AB_STAGE];
  __shared__ __attribute__((aligned(1024))) unsigned char sB1[AB_STAGE];
  int bid = (int)blockIdx.x;
  const int u_ps = tile_unit_count(a.hdr[3] - a.hdr[1], tps.n_tiles);
  if (bid < u_ps) {
    tile_ps_body<BF, MODE>(a, tps, bid, sA0, sA1, sB0, sB1);
    return;
  }
  bid -= u_ps;
  const int u_64 = tile_unit_count(a.hdr[0] - a.hdr[3], t64.n_tiles);
  if (bid < u_64) {
    tile_gemm_body<BF, MODE, 4, 4>(a, t64, bid, sA0, sA1, sB0, sB1);
    return;
  }
  bid -= u_64;
  if (tbf.n_tiles > 0) tile_gemm_bf16_body<BF, MODE>(a, tbf, bid, sA0, sA1, sB0, sB1);
}

}  // namespace

bool tile_gemm_applies(int tier, int mode, int n_rows, int inter, int K, int group_size) {
  if (K < KC || K % KC != 0 || K > 65536) return false;
  if (tier == 2 && group_size != KC) return false;  // one chunk = one scale group
  if (tier == 1) return false;
  if (mode == MODE_GATEUP) {
    if (inter % 64 != 0 || n_rows != 2 * inter) return false;
  } else if (n_rows % 128 != 0) {
    return false;
  }
  // 32-bit buffer offsets within one expert's weights
  if ((int64_t)n_rows * (tier == 2 ? K / 2 : K * 2) > 0x7fffffffLL) return false;
  return true;
}

int64_t tile_rowsum_floats(int64_t rows, int64_t K) { return rows * (K / KC); }

int launch_group_rowsum(bool bf, const uint16_t* x, int64_t stride, int64_t rows, int K, int gs,
                        float* out, hipStream_t s) {
  if (rows <= 0) return EXQ_SUCCESS;
  if (rows > INT32_MAX) return set_error(EXQ_ERROR_UNSUPPORTED, "group_rowsum: too many rows");
  if (bf)
    hipLaunchKernelGGL(group_rowsum_kernel<true>, dim3((unsigned)rows), dim3(256), 0, s, x, stride,
                       (int)rows, K, gs, -136.0f, out);
  else
    hipLaunchKernelGGL(group_rowsum_kernel<false>, dim3((unsigned)rows), dim3(256), 0, s, x,
                       stride, (int)rows, K, gs, -1032.0f, out);
  return check_launch("group_rowsum_kernel");
}

int launch_group_rowsum_tg(bool bf, const uint16_t* x, int64_t stride, int K, const int* hdr,
                           const TgEntry* tg, int64_t cap, int64_t rs_rows, float* out,
                           hipStream_t s) {
  const int64_t grid = kRowsumTgParts * cap;
  if (grid <= 0) return EXQ_SUCCESS;
  if (grid > INT32_MAX || rs_rows > INT32_MAX)
    return set_error(EXQ_ERROR_UNSUPPORTED, "group_rowsum_tg: too many rows");
  if (bf)
    hipLaunchKernelGGL(group_rowsum_tg_kernel<true>, dim3((unsigned)grid), dim3(256), 0, s, x,
                       stride, K, -136.0f, hdr, tg, (int)rs_rows, out);
  else
    hipLaunchKernelGGL(group_rowsum_tg_kernel<false>, dim3((unsigned)grid), dim3(256), 0, s, x,
                       stride, K, -1032.0f, hdr, tg, (int)rs_rows, out);
  return check_launch("group_rowsum_tg_kernel");
}

template <int MODE>
static int launch_tile_mode(int tier, bool bf, int shape, const GemmArgs& a, const TileArgs& t,
                            int64_t grid, hipStream_t s) {
  const dim3 g((unsigned)grid), b(TT);
  if (tier == 0) {
    if (bf)
      hipLaunchKernelGGL((tile_gemm_bf16_kernel<true, MODE>), g, b, 0, s, a, t);
    else
      hipLaunchKernelGGL((tile_gemm_bf16_kernel<false, MODE>), g, b, 0, s, a, t);
    return check_launch("tile_gemm_bf16_kernel");
  }
  if (shape == TILE_PS_128x256) {
    if (bf)
      hipLaunchKernelGGL((tile_ps_kernel<true, MODE>), g, b, 0, s, a, t);
    else
      hipLaunchKernelGGL((tile_ps_kernel<false, MODE>), g, b, 0, s, a, t);
    return check_launch("tile_ps_kernel");
  }
  if (shape == TILE_64x256) {
    if (bf)
      hipLaunchKernelGGL((tile_gemm_kernel<true, MODE, 4, 4>), g, b, 0, s, a, t);
    else
      hipLaunchKernelGGL((tile_gemm_kernel<false, MODE, 4, 4>), g, b, 0, s, a, t);
    return check_launch("tile_gemm_kernel");
  }
  if (bf)
    hipLaunchKernelGGL((tile_gemm_kernel<true, MODE, 8, 2>), g, b, 0, s, a, t);
  else
    hipLaunchKernelGGL((tile_gemm_kernel<false, MODE, 8, 2>), g, b, 0, s, a, t);
  return check_launch("tile_gemm_kernel");
}

bool tile_gemm_wide_applies(int mode, int n_rows, int inter) {
  return mode == MODE_GATEUP ? inter % 128 == 0 : n_rows % 256 == 0;
}

int launch_tile_gemm(int tier, int mode, bool bf, const GemmArgs& a, const float* rs,
                     int64_t rs_rows, int64_t x_bytes, int64_t tg_cap, hipStream_t s,
                     int shape) {
  TileArgs t;
  t.rs = rs;
  t.rs_rows = (int)rs_rows;
  t.x_bytes = x_bytes;
  t.h_lo = 1;  // every INT4 group (one tile shape)
  t.h_hi = 0;
  if (tier != 2) shape = TILE_128x128;
  const int tn = shape == TILE_128x128 ? 128 : 256;
  t.n_tiles = mode == MODE_GATEUP ? a.inter / (tn / 2) : a.n_rows / tn;
  const int64_t grid = 8 * cdiv(tg_cap, 8) * t.n_tiles;
  if (grid <= 0) return EXQ_SUCCESS;
  if (grid > INT32_MAX || rs_rows > INT32_MAX)
    return set_error(EXQ_ERROR_UNSUPPORTED, "tile_gemm: problem too large");
  if (mode == MODE_GATEUP) return launch_tile_mode<MODE_GATEUP>(tier, bf, shape, a, t, grid, s);
  if (mode == MODE_DOWN) return launch_tile_mode<MODE_DOWN>(tier, bf, shape, a, t, grid, s);
  return launch_tile_mode<MODE_PLAIN>(tier, bf, shape, a, t, grid, s);
}

template <int MODE>
static int launch_mix_mode(bool bf, const GemmArgs& a, const TileArgs& tps, const TileArgs& t64,
                           const TileArgs& tbf, int64_t grid, hipStream_t s) {
  const dim3 g((unsigned)grid), b(TT);
  if (bf)
    hipLaunchKernelGGL((tile_mix_kernel<true, MODE>), g, b, 0, s, a, tps, t64, tbf);
  else
    hipLaunchKernelGGL((tile_mix_kernel<false, MODE>), g, b, 0, s, a, tps, t64, tbf);
  return check_launch("tile_mix_kernel");
}

int launch_tile_mix(int mode, bool bf, const GemmArgs& a, const float* rs, int64_t rs_rows,
                    int64_t x_bytes, int64_t cap_ps, int64_t cap_64, int64_t cap_bf,
                    hipStream_t s) {
  if (mode != MODE_GATEUP && mode != MODE_DOWN)
    return set_error(EXQ_ERROR_UNSUPPORTED, "tile_mix: gate/up or down only");
  TileArgs tps, t64, tbf;
  tps.rs = nullptr;  // scaled weight operands: no row sums
  tps.rs_rows = 0;
  tps.x_bytes = x_bytes;
  tps.n_tiles = mode == MODE_GATEUP ? a.inter / 128 : a.n_rows / 256;  // 256-row INT4 tiles
  tps.h_lo = 1;
  tps.h_hi = 3;
  t64 = tps;
  t64.rs = rs;
  t64.rs_rows = (int)rs_rows;
  t64.h_lo = 3;
  t64.h_hi = 0;
  tbf.rs = nullptr;
  tbf.rs_rows = 0;
  tbf.x_bytes = x_bytes;
  tbf.n_tiles = cap_bf > 0 ? (mode == MODE_GATEUP ? a.inter / 64 : a.n_rows / 128) : 0;
  tbf.h_lo = 0;
  tbf.h_hi = 2;
  const int64_t grid = 8 * cdiv(cap_ps, 8) * tps.n_tiles + 8 * cdiv(cap_64, 8) * t64.n_tiles +
                       8 * cdiv(cap_bf, 8) * tbf.n_tiles;
  if (grid <= 0) return EXQ_SUCCESS;
  if (grid > INT32_MAX || rs_rows > INT32_MAX)
    return set_error(EXQ_ERROR_UNSUPPORTED, "tile_mix: problem too large");
  return mode == MODE_GATEUP ? launch_mix_mode<MODE_GATEUP>(bf, a, tps, t64, tbf, grid, s)
                             : launch_mix_mode<MODE_DOWN>(bf, a, tps, t64, tbf, grid, s);
}

}  // namespace exq
