// decode.hip -- the MoE layer for decode batches (T <= 64) in two launches.
//
//   gate/up kernel: unit = (active expert, 16 gate rows + the 16 matching up
//                   rows); SiLU(gate) * up -> `mid` rows.
//   down kernel:    unit = (active expert, ROWS_B output rows); fp32 partial
//                   rows per routed slot; the last unit to finish a column
//                   block of H combines it over each token's slots in fixed
//                   order (deterministic) and writes `out`.  From T = 32 or
//                   four k-splits on, that tail (one work-group per block)
//                   outlasts a separate launch, so decode_combine_kernel does
//                   the same combine as a third launch instead.
//
// Both kernels route for themselves: every work-group reads the (<= 1024)
// routed ids into LDS once, marks the active experts in a bitmap and counts
// them; unit u belongs to the (u / nb)-th active expert (ascending id; routed
// experts that received a slot, then the always-on shared experts).  The grid
// is one resident round of work-groups (CUs x occupancy), each taking units
// blockIdx.x, blockIdx.x + gridDim.x, ...  Each wave finds the expert's rows
// itself with one ballot per 64 ids (ascending slot order -- the canonical
// order of the reference's stable argsort), so no row table or barrier is
// needed before the activation loads.
//
// Per unit, the four waves split the contraction into contiguous k-block
// ranges.  INT4 weights take the LDS path when a wave's range fits its 8 KB
// region: the wave DMAs its whole slice with buffer_load ... lds, whole
// 128-byte lines per row, into XOR-swizzled slots, so the slice is in flight
// without occupying registers; measured, this streams better than 128-bit
// register loads in the MFMA operand layout (16 rows x 64 B per instruction,
// half lines).  Activation fragments (16-byte loads from L2) and the fp16
// group scales stream through a 2-deep register ring.  Other cases (INT8 and
// BF16 experts of a mixed bank, or a k-range too long for the region) stream
// weights through a register ring instead.  Nibbles become exact bf16/f16
// values (base + n) with one v_and_or_b32 per pair (the exponent-OR method of
// Kim et al., "Who Says Elephants Can't Run", 2022) and feed
// v_mfma_f32_16x16x32_{bf16,f16}; the constant base is removed by MFMAs of
// the same activations against a -base operand; the fp16 group scale
// multiplies each exact k-block sum in fp32.  The four waves' partial tiles
// are summed through LDS.  INT4 weights pair k-offsets (0,4),(1,5),(2,6),
// (3,7) inside each 8-group; the gate/up epilogue writes `mid` in that order
// so the down kernel reads INT4 experts' rows without a permute.
//
// The combine's fp32 partials are written and read with agent-coherent (sc1)
// accesses; every storing wave waits for its stores before its work-group
// bumps the column block's counter, so no whole-cache writeback or
// invalidate is needed (on this part agent-scope fences write back /
// invalidate the whole L2 of an XCD).  The gate/up kernel, which always runs
// first on the same stream, zeroes the down kernel's counters, so the
// workspace needs no zero fill and an interrupted call leaves nothing behind
// for the next one; the last combine zeroes them again as well.
#include <type_traits>

#include "exq_internal.h"

#include <hip/hip_ext.h>

#include "dev_util.h"

#include <map>
#include <mutex>
#include <tuple>

namespace exq {
namespace {

using namespace dev;

constexpr int DW = 4;              // waves per work-group
constexpr int DNT = DW * 64;
constexpr int MAX_SLOTS = 1024;    // T * (k + n_shared)
constexpr int MAX_BM_WORDS = 32;   // active-expert bitmap: E + shared <= 1024
constexpr int kCombineLaunchMinT = 32;     // down combine: own launch from this batch on,
constexpr int kCombineLaunchMinSplit = 4;  // or from this many k-splits on; else in-kernel
static_assert(kCombineLaunchMinSplit <= 4, "the in-kernel combine sums at most three k-splits");
// The down projection by output rows (decode_down_rows_kernel) up to this batch
// (measured on 48 streamed Qwen3 layers, µs per layer, rows / tiled down:
// T=1 15.2 / 19.5, T=2 20.1 / 22.6, T=3 24.1 / 23.6, T=4 28.3 / 25.2).
constexpr int kRowsDownMaxT = 2;
// The gate/up projection by output rows (decode_gateup_rows_kernel) up to this
// batch (same layers, with the rows down kernel, rows / tiled gate/up: T=1
// 14.5 / 15.2, T=2 21.0 / 20.1).
constexpr int kRowsGateUpMaxT = 1;

// Output rows of a down unit: 64 (four row sets), 32 when a pass holds two
// or four 16-row tiles (register budget of the accumulators).
__host__ __device__ constexpr int rows_b(int nt) { return nt == 1 ? 64 : 32; }

// 128-bit registers per lane for the weight + activation ring.
__host__ __device__ constexpr int ring_regs(int nt) { return nt == 1 ? 12 : 20; }

// LDS bytes per wave: the INT4 weight slice of the DMA path and, after a
// pass's k-loop, the wave's partial tiles (WAVE_W), then the unit's fp16
// group scales (WAVE_S).
constexpr int WAVE_W = 8192;
constexpr int WAVE_S = 1024;
constexpr int WAVE_LDS = WAVE_W + WAVE_S;
// Register-ring units keep their k-range's group scales behind the partial
// tiles (at most 4 KiB), in the rest of the wave's region.
constexpr int SCALE_OFF = 4096;
constexpr int RING_SCALE_BYTES = WAVE_LDS - SCALE_OFF;

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
  uint16_t* mid;                // [T * kp, I] activation dtype, MFMA k-order
  float* part;                  // [T * kp, H] fp32
  uint16_t* out;                // [T, H]
  int* sync;                    // combine counters, see sync_* below
  int* plan;                    // per-tile records for the down kernel, see kPlan* below
  int nbA, nbB;                 // units per expert: I / 16, H / rows_b(NT)
  int nsplit;                   // down: k-splits per (expert, row block), partial sets
  int combine;                  // down: 1 = the last unit of a column block combines it,
                                // 0 = decode_combine_kernel runs after the down kernel
};

// Counter layout of the sync region (fixed, independent of the problem size):
// one 128-byte line per counter.
constexpr int SYNC_INTS = 32;
__device__ __forceinline__ int* sync_c(const LayerArgs& a, int hb) {
  return a.sync + (kDecodeMaxBuckets + hb) * SYNC_INTS;
}
__device__ __forceinline__ int* sync_done(const LayerArgs& a) {
  return a.sync + (kDecodeMaxBuckets + kDecodeMaxHBlocks) * SYNC_INTS;
}

// Row field of a mixed bank's expert map entry (tier in the top two bits).
constexpr uint32_t kRowMask = 0x3fffffffu;

// The batch's routed ids and active-expert bitmap, per work-group.
struct Route {
  uint32_t bitmap[MAX_BM_WORDS];
  int16_t ids[MAX_SLOTS];  // routed id of slot t*k + j (-1: dropped)
  int multi;               // some expert has more than 16 rows
};

// Load the ids and build the bitmap (all threads); returns the number of
// active experts and leaves this lane's bitmap word and prefix for
// select_expert.
// Also counts each expert's rows into cntw (16 bits per expert, two per word;
// a count is at most T * k <= MAX_SLOTS, so no carry crosses a half).
// MAP (mixed banks): also writes emap[e] = (tier << 30) | row of expert e in
// its tier's bank, for every expert, from loads issued beside the id loads
// (tier 0 / 1 / 2 in the top two bits; a row below 2^30 in the rest: a bank of
// 2^30 experts would not fit any GPU's memory).
template <bool MAP = false>
__device__ __forceinline__ int route(const LayerArgs& a, Route& r, uint32_t* cntw, uint32_t& word,
                                     int& incl, int& c, int* emap = nullptr) {
  const int lane = threadIdx.x & 63;
  const int n = a.T * a.k;
  const int nw = (a.Ep + 31) >> 5;
  // this thread's ids (s = threadIdx.x + i * DNT), loaded as raw words before
  // the LDS clear and its barrier, all in flight at once (no dtype branch or
  // conversion between the loads)
  constexpr int RPT = MAX_SLOTS / DNT;
  const bool id64 = a.ids_dtype == EXQ_DTYPE_I64;
  const __amdgpu_buffer_rsrc_t ids_r = make_rsrc(a.ids, (int64_t)n * (id64 ? 8 : 4));
  uint32_t lo[RPT], hi[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int s = threadIdx.x + i * DNT;
    lo[i] = __builtin_amdgcn_raw_buffer_load_b32(ids_r, s < n ? s * (id64 ? 8 : 4) : OOB_OFF, 0, 0);
    hi[i] = __builtin_amdgcn_raw_buffer_load_b32(ids_r, s < n && id64 ? s * 8 + 4 : OOB_OFF, 0, 0);
  }
  constexpr int EPT = MAP ? kDecodeMaxBuckets / DNT : 1;  // experts per thread
  uint32_t mt[EPT], mi[EPT];
  if constexpr (MAP) {
    const __amdgpu_buffer_rsrc_t tier_r = make_rsrc(a.tier, a.Ep);
    const __amdgpu_buffer_rsrc_t idx_r = make_rsrc(a.index, a.index ? (int64_t)a.Ep * 4 : 0);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + i * DNT;
      mt[i] = __builtin_amdgcn_raw_buffer_load_b8(tier_r, e < a.Ep ? e : OOB_OFF, 0, 0);
      mi[i] = __builtin_amdgcn_raw_buffer_load_b32(idx_r, e < a.Ep ? e * 4 : OOB_OFF, 0, 0);
    }
  }
  if (threadIdx.x < MAX_BM_WORDS) r.bitmap[threadIdx.x] = 0u;
  if (threadIdx.x == 0) r.multi = a.T > 16 && a.Ep > a.E;  // shared experts take every token
  for (int i = threadIdx.x; i < (a.Ep + 1) >> 1; i += DNT) cntw[i] = 0u;
  __syncthreads();
  if constexpr (MAP) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + i * DNT;
      if (e < a.Ep)
        emap[e] = (int)(((mt[i] & 3u) << 30) | ((a.index ? mi[i] : (uint32_t)e) & kRowMask));
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int s = threadIdx.x + i * DNT;
    if (s < n) {
      const int64_t id = id64 ? (int64_t)(((uint64_t)hi[i] << 32) | lo[i]) : (int64_t)(int32_t)lo[i];
      const int v = (id >= 0 && id < a.E) ? (int)id : -1;
      r.ids[s] = (int16_t)v;
      if (v >= 0) {
        atomicOr(&r.bitmap[v >> 5], 1u << (v & 31));
        const uint32_t old = atomicAdd(&cntw[v >> 1], 1u << ((v & 1) * 16));
        if (((old >> ((v & 1) * 16)) & 0xffffu) >= 16u) r.multi = 1;
      }
    }
  }
  if (threadIdx.x < a.Ep - a.E && a.T > 0) {
    const int v = a.E + threadIdx.x;
    atomicOr(&r.bitmap[v >> 5], 1u << (v & 31));
    atomicAdd(&cntw[v >> 1], (uint32_t)a.T << ((v & 1) * 16));
  }
  __syncthreads();
  word = lane < nw ? r.bitmap[lane] : 0u;
  c = __popc(word);
  // inclusive prefix of the per-word counts (< 64 each) from bit-sliced ballots
  const uint64_t lt_or_eq = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
  incl = 0;
#pragma unroll
  for (int b = 0; b < 6; ++b) incl += __popcll(__ballot((c >> b) & 1) & lt_or_eq) << b;
  return __builtin_amdgcn_readlane(incl, 63);
}

// The ai-th active expert (ai < number of active experts).
__device__ __forceinline__ int select_expert(int ai, uint32_t word, int incl, int c) {
  const uint64_t hit = __ballot(incl - c <= ai && ai < incl);
  const int wl = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)hit) - 1);
  uint32_t wbits = __builtin_amdgcn_readlane(word, wl);
  const int q0 = ai - (__builtin_amdgcn_readlane(incl, wl) - __builtin_amdgcn_readlane(c, wl));
  for (int t = 0; t < q0; ++t) wbits &= wbits - 1u;
  return wl * 32 + (__ffs(wbits) - 1);
}

// Rows of expert e (after route()).
__device__ __forceinline__ int expert_rows(const uint32_t* cntw, int e) {
  return (int)((cntw[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
}

// Token tiles (16 rows each) of the active experts, as segments: segment t
// holds tile t of every expert with more than t tiles, in ascending expert
// order, so an expert's first tile comes first and its later tiles are
// spread over other work-groups.  Lane t of the result holds segment t's
// expert count (lanes past the last segment hold 0); *total = all tiles.
__device__ __forceinline__ int tile_segments(const LayerArgs& a, const uint32_t* cntw,
                                             const Route& rt, int* total) {
  const int lane = threadIdx.x & 63;
  int seg = 0;
  for (int e0 = 0; e0 < a.Ep; e0 += 64) {
    const int e = e0 + lane;
    const bool act = e < a.Ep && ((rt.bitmap[e >> 5] >> (e & 31)) & 1u);
    const int nt = act ? (expert_rows(cntw, e) + 15) >> 4 : 0;
    for (int t = 0; t < 64; ++t) {
      const uint64_t m = __ballot(nt > t);
      if (m == 0) break;
      if (lane == t) seg += __popcll(m);
    }
  }
  int tot = seg;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) tot += __shfl_xor(tot, o, 64);
  *total = __builtin_amdgcn_readfirstlane(tot);
  return seg;
}

// The j-th expert (ascending) with more than t tiles (t >= 1).
__device__ __forceinline__ int select_tiled_expert(const LayerArgs& a, const uint32_t* cntw,
                                                   const Route& rt, int t, int j) {
  const int lane = threadIdx.x & 63;
  for (int e0 = 0; e0 < a.Ep; e0 += 64) {
    const int e = e0 + lane;
    const bool act = e < a.Ep && ((rt.bitmap[e >> 5] >> (e & 31)) & 1u);
    const uint64_t m = __ballot(act && ((expert_rows(cntw, e) + 15) >> 4) > t);
    const int cm = __popcll(m);
    if (j < cm) return e0 + nth_set_bit(m, j);
    j -= cm;
  }
  return 0;  // not reached for j < the segment's count
}


// Expert e's rows (its routed slots t*kp + j in ascending order, the order of
// the reference's stable sort; every token for a shared expert), found by
// each wave on its own with one ballot per 64 ids: sl[tt] receives the slot
// of row r0 + tt*16 + r16, or of the last row when that is beyond the count.
// Returns the row count (wave-uniform).
template <int NT>
__device__ __forceinline__ int lane_slots(const LayerArgs& a, const Route& r, int e, int r0,
                                          int (&sl)[NT]) {
  const int lane = threadIdx.x & 63, r16 = lane & 15;
  if (e >= a.E) {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int q = r0 + tt * 16 + r16;
      sl[tt] = (q < a.T ? q : a.T - 1) * a.kp + a.k + (e - a.E);
    }
    return a.T;
  }
  const int n = a.T * a.k;
  int cnt = 0, last = 0, found[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) found[tt] = -1;
  for (int s0 = 0; s0 < n; s0 += 64) {
    const int s = s0 + lane;
    const uint64_t m = __ballot(s < n && r.ids[s] == e);
    const int c = __popcll(m);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int q = r0 + tt * 16 + r16;
      if (found[tt] < 0 && q >= cnt && q < cnt + c) found[tt] = s0 + nth_set_bit(m, q - cnt);
    }
    if (c) last = s0 + 63 - __clzll(m);
    cnt += c;
  }
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int f = found[tt] < 0 ? last : found[tt];
    const int t = f / a.k;
    sl[tt] = t * a.kp + (f - t * a.k);
  }
  return cnt;
}

// The down kernel's plan, written by the gate/up kernel of the same call
// (which has routed already): int plan[0] = the number of 16-row tiles, bit s
// of the words from plan[kPlanMaskOff] on = routed slot s (t * k + j) has an id
// in [0, E), then from int kPlanHdrInts on one 32-int (128-byte) record per
// tile, in unit order:
//   [0] expert | (tile << 16), [1] the expert's row count, [2] its mixed-bank
//   map entry (tier << 30 | row), [16 + r] the slot of the tile's row r
//   (tile * 16 + r, the last row past the count).
// A down unit then needs one load of its record before its weight copies go
// out, instead of routing again (loading every id, LDS histogram, barriers).
constexpr int kPlanHdrInts = 96;   // [0] tile count; [32, 66) the routed slots' validity bits
constexpr int kPlanMaskOff = 32;
constexpr int kPlanRecInts = 32;
constexpr int kPlanSlotOff = 16;
static_assert(kPlanMaskOff + MAX_SLOTS / 32 + 2 <= kPlanHdrInts, "validity bits fit the header");

// Row sources of a unit: the routed ids in LDS (gate/up), or the unit's plan
// record (down).  slots() gives lane r16 the slot of row r0 + r16 (the last
// row past the count) and returns the expert's row count.
struct RowsRoute {
  const Route& rt;
  template <int NT>
  __device__ __forceinline__ int slots(const LayerArgs& a, int e, int r0, int (&sl)[NT]) const {
    return lane_slots<NT>(a, rt, e, r0, sl);
  }
};
struct RowsPlan {
  int cnt;   // the expert's row count (wave-uniform)
  int slot;  // this lane's slot, from the record (lanes r16 hold rows r0 + r16)
  template <int NT>
  __device__ __forceinline__ int slots(const LayerArgs&, int, int, int (&sl)[NT]) const {
    static_assert(NT == 1, "a plan record holds one 16-row tile");
    sl[0] = slot;
    return cnt;
  }
};

// Compile-time geometry of a (tier, phase, tiles-per-pass) instantiation.
template <int TIER, int PH, int NT>
struct Geo {
  static constexpr int ROWS_B = rows_b(NT);
  static constexpr int RS = PH == 0 ? 2 : ROWS_B / 16;              // row sets of 16 rows
  static constexpr int QPK = TIER == 2 ? 1 : (TIER == 1 ? 2 : 4);   // uint4 per lane, k-block, row set
  static constexpr int WSLOT = RS * QPK;                            // weight registers per k-block
  static constexpr int SLOT = WSLOT + 4 * NT;                       // + activation fragments
  static constexpr int P0 = ring_regs(NT) / SLOT;
  static constexpr int P = P0 < 1 ? 1 : (P0 > 4 ? 4 : P0);          // ring depth (k-blocks)
  static constexpr int KBSTRIDE = TIER == 2 ? 64 : (TIER == 1 ? 128 : 256);  // row bytes per k-block
  static constexpr int CK = WAVE_W / (RS * 1024);                   // INT4 k-blocks a wave holds in LDS
  static_assert(RS * NT * 1024 <= WAVE_W, "partial tiles exceed the wave's LDS region");
};

// Per-unit quantities shared by both k-loop variants.
template <int TIER, int PH, int NT>
struct UnitCtx {
  using G = Geo<TIER, PH, NT>;
  int lane, wave, r16, kq, K, nkb, lo, nmy, ng, rowbytes;
  int64_t ebase;
  __amdgpu_buffer_rsrc_t wr, wnull, sr, snull, xr, xnull, part_r;
  float rowscale[G::RS];

  int split;  // down: this unit's k-split (its partial set)
  __device__ __forceinline__ UnitCtx(const LayerArgs& a, int e, int blk, int sp = 0,
                                     int widx_in = -1) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    r16 = lane & 15;
    kq = lane >> 4;
    K = PH == 0 ? a.H : a.I;
    nkb = K >> 7;
    split = sp;
    // the split's k-blocks [s0, s1), then this wave's quarter of them; the
    // longer ranges go to the first waves, so that with two k-blocks copied
    // per instruction the ranges start at even k-blocks where they can (six
    // k-blocks: 2, 2, 1, 1 from k-blocks 0, 2, 4, 5)
    const int ns = PH == 0 ? 1 : a.nsplit;
    const int s0 = (sp * nkb) / ns, s1 = ((sp + 1) * nkb) / ns;
    const int nq = (s1 - s0) >> 2, nx = (s1 - s0) & 3;
    lo = s0 + wave * nq + (wave < nx ? wave : nx);
    nmy = nq + (wave < nx ? 1 : 0);  // k-blocks of this wave
    const Proj& W = PH == 0 ? a.w13 : a.w2;
    const int n_rows = PH == 0 ? 2 * a.I : a.H;
    // the expert's row in its tier's bank (from the LDS map when the caller has it)
    const int widx = widx_in >= 0 ? widx_in : (a.index ? uni_i(a.index[uni_i(e)]) : e);
    ebase = (int64_t)widx * n_rows;
    rowbytes = TIER == 2 ? K / 2 : (TIER == 1 ? K : 2 * K);
    const unsigned char* wbase =
        TIER == 2 ? W.i4
                  : (TIER == 1 ? reinterpret_cast<const unsigned char*>(W.i8)
                               : reinterpret_cast<const unsigned char*>(W.bf16));
    wr = make_rsrc(wbase + ebase * rowbytes, (int64_t)n_rows * rowbytes);
    wnull = make_rsrc(wbase + ebase * rowbytes, 0);
    ng = nkb >> a.gshift;  // scale groups per row
    const uint16_t* sbase = TIER == 2 ? W.i4_scales + ebase * ng : nullptr;
    sr = make_rsrc(sbase, (int64_t)n_rows * ng * 2);
    snull = make_rsrc(sbase, 0);
    xr = PH == 0 ? make_rsrc(a.x, (int64_t)a.T * a.H * 2)
                 : make_rsrc(a.mid, (int64_t)a.T * a.kp * a.I * 2);
    xnull = make_rsrc(PH == 0 ? (const void*)a.x : (const void*)a.mid, 0);
    part_r = make_rsrc(a.part, (int64_t)a.nsplit * a.T * a.kp * a.H * 4);
#pragma unroll
    for (int rs = 0; rs < G::RS; ++rs) {
      rowscale[rs] = 1.f;
      if constexpr (TIER == 1) rowscale[rs] = f16_bits_to_f32(W.i8_scales[ebase + row(a, blk, rs * 16 + r16)]);
    }
  }
  // Weight row of row-set row rr (0 <= rr < RS*16) of row block blk.
  __device__ __forceinline__ int row(const LayerArgs& a, int blk, int rr) const {
    return PH == 0 ? (rr < 16 ? 0 : a.I - 16) + blk * 16 + rr : blk * G::ROWS_B + rr;
  }
  // Byte offset of this lane's activation row (slot sl) in its tile.
  __device__ __forceinline__ int xoff(const LayerArgs& a, int sl) const {
    const int xrow = PH == 0 ? sl / a.kp : sl;
    return (xrow * (PH == 0 ? a.H : a.I) + kq * 32) * 2;
  }
};

// A operand of one 16-row tile (four 16x32 pieces) from its raw fragments,
// and its -base sum (the exact correction for the +base in dequantised weights).
// The gate/up phase reads activations in natural k order; `mid` is stored in
// INT4 pairing order.
template <int TIER, bool BF, int PH>
__device__ __forceinline__ void make_a(const uint4* raw, uint4 (&xa)[4], f32x4_t& init) {
  const uint4 negb = neg_base_operand<TIER, BF>();
  init = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    xa[d] = raw[d];
    if constexpr (PH == 0 && TIER == 2) xa[d] = dperm(xa[d]);
    if constexpr (PH == 1 && TIER != 2) xa[d] = dperm_inv(xa[d]);
  }
  if constexpr (TIER != 0) {
#pragma unroll
    for (int d = 0; d < 4; ++d) init = dmfma<BF>(xa[d], negb, init);
  }
}

// After a pass's k-loop: the four waves' partial tiles sit in their LDS
// regions; sum them and write `mid` (gate/up: SiLU(gate) * up) or the fp32
// partial rows (down).
template <int TIER, bool BF, int PH, int NT, int WSTRIDE = WAVE_LDS>  // wave w's tiles at lds + w*WSTRIDE
__device__ __forceinline__ void finish_pass(const LayerArgs& a, const UnitCtx<TIER, PH, NT>& u,
                                            const unsigned char* lds, const int (&sl)[NT], int cc,
                                            int ntiles, int blk) {
  // slot of row tt*16 + 4*kq + i of the pass: held by lane 4*kq + i of tile tt
  auto slot_of = [&](int tt, int i) {
    int v = sl[0];
#pragma unroll
    for (int j = 1; j < NT; ++j)
      if (j == tt) v = sl[j];
    return __shfl(v, u.kq * 4 + i, 64);
  };
  using G = Geo<TIER, PH, NT>;
  constexpr int RS = G::RS, ROWS_B = G::ROWS_B;
  auto red = [&](int w, int rs, int tt) {
    return reinterpret_cast<const float4*>(lds + w * WSTRIDE)[(rs * NT + tt) * 64 + u.lane];
  };
  // lane (r16, kq) of tile tt holds rows tt*16 + 4*kq + i, column r16
  if constexpr (PH == 0) {
    const int tt = u.wave;
    if (tt < ntiles) {
      float g[4] = {0.f, 0.f, 0.f, 0.f}, v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const float4 pg = red(w, 0, tt);
        const float4 pu = red(w, 1, tt);
        g[0] += pg.x; g[1] += pg.y; g[2] += pg.z; g[3] += pg.w;
        v[0] += pu.x; v[1] += pu.y; v[2] += pu.z; v[3] += pu.w;
      }
      const int col = blk * 16 + (u.r16 & 8) + pair_pos(u.r16 & 7);  // INT4 pairing order
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = tt * 16 + u.kq * 4 + i;
        const int slot = slot_of(tt, i);
        if (q < cc) {
          const float y = silu_f32(g[i] * u.rowscale[0]) * (v[i] * u.rowscale[1]);
          a.mid[(int64_t)slot * a.I + col] = (uint16_t)to_act_bits<BF>(y);
        }
      }
    }
  } else {
    bool stored = false;
    for (int it = threadIdx.x; it < RS * ntiles * 64; it += DNT) {
      const int rtl = it >> 6;
      const int rs = rtl / ntiles, tt = rtl - rs * ntiles;
      float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const float4 pv = red(w, rs, tt);
        s[0] += pv.x; s[1] += pv.y; s[2] += pv.z; s[3] += pv.w;
      }
      float rsc = 1.f;
#pragma unroll
      for (int j = 0; j < RS; ++j)
        if (j == rs) rsc = u.rowscale[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = tt * 16 + u.kq * 4 + i;
        const int slot = slot_of(tt, i);
        if (q < cc)
          __builtin_amdgcn_raw_buffer_store_b32(
              __builtin_bit_cast(uint32_t, s[i] * rsc), u.part_r,
              ((u.split * a.T * a.kp + slot) * a.H + blk * ROWS_B + rs * 16 + u.r16) * 4, 0,
              CPOL_SC1);
      }
      stored = true;
    }
    if (stored && a.combine) wait_vm_all();  // this wave's partial rows have completed
  }
}

// Down phase: the last of a column block's units (by its counter) combines
// the block: out[t, h..h+3] = sum over the token's slots j (ascending) of
// weight * partial (the NS k-splits of a slot summed in split order first).
// Slots are taken 8 / NS at a time: all of a batch's partial loads and the
// raw router weights of its slots go out before any of them is used, so
// a batch is one memory round trip (NS and the weight width are template
// arguments, so every load lands in a register of its own with no branch
// between the loads and their use).
template <bool BF, int ROWS_B, int NS, bool WF32>  // WF32: fp32 router weights (else 16-bit)
__device__ __forceinline__ void combine_block_ns(const LayerArgs& a, int blk) {
  constexpr int SB = 8 / NS;  // slots per batch (eight slots: every k + shared of these configurations)
  constexpr bool wf32 = WF32;
  const int64_t set = (int64_t)a.T * a.kp * a.H;  // floats per partial set
  const __amdgpu_buffer_rsrc_t part_r = make_rsrc(a.part, a.nsplit * set * 4);
  const __amdgpu_buffer_rsrc_t w_r = make_rsrc(a.topk_w, (int64_t)a.T * a.k * (wf32 ? 4 : 2));
  const uint32_t* valid = reinterpret_cast<const uint32_t*>(a.plan + kPlanMaskOff);
  const int h0 = blk * ROWS_B;
  for (int idx = threadIdx.x; idx < a.T * (ROWS_B / 4); idx += DNT) {
    const int t = idx / (ROWS_B / 4);
    const int h = h0 + (idx - t * (ROWS_B / 4)) * 4;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < a.kp; j0 += SB) {
      float4 pv[SB][NS];
#pragma unroll
      for (int i = 0; i < SB; ++i)
#pragma unroll
        for (int sp = 0; sp < NS; ++sp)
          pv[i][sp] = __builtin_bit_cast(
              float4, __builtin_amdgcn_raw_buffer_load_b128(
                          part_r,
                          j0 + i < a.kp ? (int)((sp * set + (int64_t)(t * a.kp + j0 + i) * a.H + h) * 4)
                                        : OOB_OFF,
                          0, CPOL_SC1));
      // (the weights after the partial loads: converting them waits for
      // loads that are all in flight already)
      // raw weights of the routed slots (zeros otherwise), and the validity
      // bits of slots t*k + j0 .. (a 64-bit window holds the batch's SB <= 8)
      uint32_t wr[SB];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int q = t * a.k + j0 + i;
        const bool in = j0 + i < a.k;
        if constexpr (WF32)
          wr[i] = __builtin_amdgcn_raw_buffer_load_b32(w_r, in ? q * 4 : OOB_OFF, 0, 0);
        else
          wr[i] = __builtin_amdgcn_raw_buffer_load_b16(w_r, in ? q * 2 : OOB_OFF, 0, 0);
      }
      const int b0 = t * a.k + j0;
      const uint64_t vw = ((uint64_t)valid[(b0 >> 5) + 1] << 32 | valid[b0 >> 5]) >> (b0 & 31);
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int j = j0 + i;
        if (j < a.kp) {
          // a dropped slot (id outside [0, E)) never wrote its partial rows: zeros instead
          const bool ok = j >= a.k || ((vw >> i) & 1u);
          const float wf = j >= a.k                    ? 1.f
                           : wf32                      ? __builtin_bit_cast(float, wr[i])
                           : a.w_dtype == EXQ_DTYPE_BF16 ? bf16_bits_to_f32(wr[i])
                                                         : f16_bits_to_f32(wr[i]);
          const float wg = ok ? wf : 0.f;
          const float4 zero = float4{0.f, 0.f, 0.f, 0.f};
          float4 cur = ok ? pv[i][0] : zero;
#pragma unroll
          for (int sp = 1; sp < NS; ++sp) {  // further k-splits, in split order
            const float4 q = ok ? pv[i][sp] : zero;
            cur.x += q.x; cur.y += q.y; cur.z += q.z; cur.w += q.w;
          }
          acc[0] += wg * cur.x;
          acc[1] += wg * cur.y;
          acc[2] += wg * cur.z;
          acc[3] += wg * cur.w;
        }
      }
    }
    uint2 o;
    o.x = to_act_bits<BF>(acc[0]) | (to_act_bits<BF>(acc[1]) << 16);
    o.y = to_act_bits<BF>(acc[2]) | (to_act_bits<BF>(acc[3]) << 16);
    *reinterpret_cast<uint2*>(a.out + (int64_t)t * a.H + h) = o;
  }
}

template <bool BF, int ROWS_B>
__device__ __forceinline__ void combine_block(const LayerArgs& a, int blk) {
  // in-kernel combines run with fewer than kCombineLaunchMinSplit splits
  const bool wf32 = a.w_dtype == EXQ_DTYPE_F32;
  if (a.nsplit == 1)
    wf32 ? combine_block_ns<BF, ROWS_B, 1, true>(a, blk) : combine_block_ns<BF, ROWS_B, 1, false>(a, blk);
  else if (a.nsplit == 2)
    wf32 ? combine_block_ns<BF, ROWS_B, 2, true>(a, blk) : combine_block_ns<BF, ROWS_B, 2, false>(a, blk);
  else
    wf32 ? combine_block_ns<BF, ROWS_B, 3, true>(a, blk) : combine_block_ns<BF, ROWS_B, 3, false>(a, blk);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_store(sync_c(a, blk), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int d = __hip_atomic_fetch_add(sync_done(a), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == a.nbB - 1)  // every block is combined
      __hip_atomic_store(sync_done(a), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Down phase, after the unit's last pass: count the unit in for its column
// block (n_tiles units times the k-splits write each block); the last of the
// block's units combines the block.
template <bool BF, int ROWS_B>
__device__ __forceinline__ void publish_and_combine(const LayerArgs& a, int blk, int n_tiles,
                                                    int* s_flag) {
  if (threadIdx.x == 0) {
    const int old =
        __hip_atomic_fetch_add(sync_c(a, blk), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = old == n_tiles * a.nsplit - 1;
  }
  __syncthreads();
  if (*s_flag) combine_block<BF, ROWS_B>(a, blk);
}

// INT4 unit whose k-blocks fit the wave's LDS region (nmy <= CK): every
// wave DMAs its whole weight slice (RS*16 rows x nmy k-blocks) into LDS with
// buffer_load ... lds.  Each DMA instruction moves 64 16-byte pieces; a row's
// pieces are contiguous in memory (whole 128-byte lines whenever nmy >= 2)
// and land at slot rr*4*nmy + (c ^ (rr & xm)), an XOR swizzle that makes the
// MFMA-layout reads (16 rows, same column) conflict-free.  No registers hold
// the weights in flight, so a work-group's whole slice is requested at once.
// Activation fragments (and the fp16 group scales) stream through a 2-deep
// register ring.
template <bool BF, int PH, int NT, typename Rows>
__device__ __forceinline__ void run_unit_dma(const LayerArgs& a, const Rows& rows, int e, int blk,
                                             int sp, int tile, unsigned char* lds, int widx,
                                             bool once) {
  using G = Geo<2, PH, NT>;
  constexpr int RS = G::RS, CK = G::CK;
  constexpr int DA = NT == 4 ? 1 : 2;  // activation k-blocks in flight
  const UnitCtx<2, PH, NT> u(a, e, blk, sp, widx);
  unsigned char* region = lds + u.wave * WAVE_LDS;
  const int p4 = 4 * u.nmy;                 // 16-byte pieces per row in LDS
  const int xm = (u.nmy & 1) ? 3 : 7;       // swizzle mask keeps c ^ (rr & xm) < p4
  auto dma = [&]() {
    for (int j = 0; j < RS * u.nmy; ++j) {  // 64 pieces per instruction
      const int p = j * 64 + u.lane;
      const int rr = p / p4;
      const int c = (p - rr * p4) ^ (rr & xm);
      const int off = u.row(a, blk, rr) * u.rowbytes + u.lo * 64 + c * 16;
      if (once)  // a slice this unit alone reads: nontemporal
        dma16_nt(u.wr, region + j * 1024, off);
      else
        dma16(u.wr, region + j * 1024, off);
    }
  };
  auto wslot = [&](int kbl, int rs) {  // LDS byte offset of this lane's piece
    const int rr = rs * 16 + u.r16;
    const int c = kbl * 4 + u.kq;
    return kbl < u.nmy ? (rr * p4 + (c ^ (rr & xm))) * 16 : 0;
  };

  dma();
  // The unit's fp16 group scales in one instruction: its rows' scales are one
  // contiguous block (two for gate/up: the gate rows and the up rows), copied
  // whole into the wave's scale area (scattered 2-byte loads cost several
  // times a 1 KiB load in the vector-memory pipeline).
  {
    const int blk_bytes = 16 * u.ng * 2;  // 16 rows
    int goff;
    if constexpr (PH == 0) {
      const int half = u.lane * 16 < blk_bytes ? 0 : 1;
      goff = (half ? a.I + blk * 16 : blk * 16) * u.ng * 2 + u.lane * 16 - half * blk_bytes;
    } else {
      goff = blk * G::ROWS_B * u.ng * 2 + u.lane * 16;
    }
    const bool in = u.lane * 16 < RS * blk_bytes;
    dma16(u.sr, region + WAVE_W, in ? goff : OOB_OFF);
  }
  // this unit's rows: tile `tile` of the expert's rows (one pass)
  const int r_begin = tile * NT * 16;
  int sl[NT];
  const int cnt = __builtin_amdgcn_readfirstlane(rows.template slots<NT>(a, e, r_begin, sl));

  const uint32_t dq_mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(dq_magic));  // keep the magic in a VGPR: one v_and_or_b32 per pair
  const uint16_t* sc_lds = reinterpret_cast<const uint16_t*>(region + WAVE_W);

  for (int r0 = r_begin; r0 < cnt && r0 < r_begin + NT * 16; r0 += NT * 16) {
    const int cc = cnt - r0 < NT * 16 ? cnt - r0 : NT * 16;
    const int ntiles = (cc + 15) >> 4;
    int xo[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) xo[tt] = u.xoff(a, sl[tt]);
    uint4 areg[DA][4 * NT];
    auto load_a = [&](int p, int kbl) {  // zeros past the wave's range
      const bool ok = uni_b(kbl < u.nmy);
      const int kb = uni_i(ok ? u.lo + kbl : u.lo);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int d = 0; d < 4; ++d)
          areg[p][tt * 4 + d] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(ok ? u.xr : u.xnull, xo[tt] + d * 16,
                                                           kb * 256, 0));
    };
#pragma unroll
    for (int p = 0; p < DA; ++p) load_a(p, p);
    wait_vm_all();  // the weight slice has landed in LDS

    f32x4_t tot[RS][NT];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int t = 0; t < NT; ++t) tot[rs][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kbl = 0; kbl < CK; ++kbl) {
      const int p = kbl % DA;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        if (tt < ntiles) {
          uint4 xa[4];
          f32x4_t init;
          make_a<2, BF, PH>(&areg[p][tt * 4], xa, init);
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) {
            const uint4 w = *reinterpret_cast<const uint4*>(region + wslot(kbl, rs));
            f32x4_t acc = dmfma<BF>(xa[0], ddeq4(w.x, dq_mask, dq_magic), init);
            acc = dmfma<BF>(xa[1], ddeq4(w.y, dq_mask, dq_magic), acc);
            acc = dmfma<BF>(xa[2], ddeq4(w.z, dq_mask, dq_magic), acc);
            acc = dmfma<BF>(xa[3], ddeq4(w.w, dq_mask, dq_magic), acc);
            // past the wave's range the activations (and so acc) are zero
            const float sc =
                kbl < u.nmy
                    ? f16_bits_to_f32(sc_lds[(rs * 16 + u.r16) * u.ng + ((u.lo + kbl) >> a.gshift)])
                    : 0.f;
            tot[rs][tt] += sc * acc;
          }
        }
      }
      if (kbl + DA < CK) load_a(p, kbl + DA);
    }
    // partial tiles into this wave's own region (its weight reads are done)
    float4* red = reinterpret_cast<float4*>(region);
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (tt < ntiles)
          red[(rs * NT + tt) * 64 + u.lane] =
              float4{tot[rs][tt][0], tot[rs][tt][1], tot[rs][tt][2], tot[rs][tt][3]};
    __syncthreads();
    finish_pass<2, BF, PH, NT>(a, u, lds, sl, cc, ntiles, blk);
    __syncthreads();  // LDS regions free again
  }
}

// LDS-path unit with the slice copied a pair of k-blocks at a time into
// separate LDS arrays (one per pair position, all four waves' copies), so
// that the k-loop starts on the first pair while the second is still
// landing: the copies go out in the order scales, pair 0, activations 0-1,
// pair 1, and each k-block waits only for the loads issued up to it.  One
// copy instruction moves 8 rows x 128 bytes (two k-blocks of each row: whole
// cache lines, as a streaming read fetches them), into LDS rows of eight
// 16-byte pieces, piece c of row r at c ^ ((r >> 1) & 7) (conflict-free MFMA
// operand reads).  A wave always issues CK / 2 pair copies (through an empty
// buffer past its range, zeros for a range's odd last k-block), so those
// waits are fixed counts.  Separate arrays let the compiler see that reading
// one pair cannot touch another's pending copy.  A slice that only this unit
// reads (its expert has one 16-row tile) is copied with the nontemporal hint.
// The partial tiles go to pair 0's array once the loop is done.
template <bool BF, int PH, typename Rows>
__device__ __forceinline__ void run_unit_kb(const LayerArgs& a, const Rows& rows, int e, int blk,
                                            int sp, int tile, bool prio, bool once) {
  constexpr int NT = 1;
  using G = Geo<2, PH, NT>;
  constexpr int RS = G::RS, CK = G::CK;
  static_assert(CK == 2 || CK == 4, "k-block pairs");
  constexpr int KPB = 2 * RS * 1024;  // one pair of k-blocks of the wave's rows
  constexpr int NP = CK / 2;          // pair arrays
  __shared__ __attribute__((aligned(16))) unsigned char s_kp0[DW * KPB];
  __shared__ __attribute__((aligned(16))) unsigned char s_kp1[NP > 1 ? DW * KPB : 16];
  __shared__ __attribute__((aligned(16))) unsigned char s_sc[DW * WAVE_S];
  const UnitCtx<2, PH, NT> u(a, e, blk, sp);
  auto pbuf = [&](int pp) { return (pp == 0 ? s_kp0 : s_kp1) + u.wave * KPB; };
  // pair pp of the wave's range: 2 * RS instructions of 8 rows x 8 pieces
  const int prow = u.lane >> 3;
  auto copy_pair = [&](int pp) {
    const bool any = uni_b(2 * pp < u.nmy);
#pragma unroll
    for (int j = 0; j < 2 * RS; ++j) {
      const int r = j * 8 + prow;
      const int c = (u.lane & 7) ^ ((r >> 1) & 7);  // source piece of this LDS slot
      const bool in = 2 * pp + (c >> 2) < u.nmy;
      const int off = in ? u.row(a, blk, r) * u.rowbytes + (u.lo + 2 * pp) * 64 + c * 16 : OOB_OFF;
      if (once)
        dma16_nt(any ? u.wr : u.wnull, pbuf(pp) + j * 1024, any ? off : 0);
      else
        dma16(any ? u.wr : u.wnull, pbuf(pp) + j * 1024, any ? off : 0);
    }
  };
  unsigned char* scl = s_sc + u.wave * WAVE_S;
  // With three or more units per work-group, the copies go out at raised
  // wave priority, so a unit's loads are not queued behind other waves'
  // compute (measured: T=64 83.2 -> 80.7 us; slower at T <= 16, hence the
  // condition).
  if (prio) __builtin_amdgcn_s_setprio(2);
  {  // the unit's scale block (as run_unit_dma)
    const int blk_bytes = 16 * u.ng * 2;
    int goff;
    if constexpr (PH == 0) {
      const int half = u.lane * 16 < blk_bytes ? 0 : 1;
      goff = (half ? a.I + blk * 16 : blk * 16) * u.ng * 2 + u.lane * 16 - half * blk_bytes;
    } else {
      goff = blk * G::ROWS_B * u.ng * 2 + u.lane * 16;
    }
    const bool in = u.lane * 16 < RS * blk_bytes;
    dma16(u.sr, scl, in ? goff : OOB_OFF);
  }
  copy_pair(0);
  const int r_begin = tile * 16;
  int sl[NT];
  const int cnt = __builtin_amdgcn_readfirstlane(rows.template slots<NT>(a, e, r_begin, sl));
  const int xo = u.xoff(a, sl[0]);
  uint4 areg[2][4];
  auto load_a = [&](int p, int kbl) {  // zeros past the wave's range
    const bool ok = uni_b(kbl < u.nmy);
    const int kb = uni_i(ok ? u.lo + kbl : u.lo);
#pragma unroll
    for (int d = 0; d < 4; ++d)
      areg[p][d] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(ok ? u.xr : u.xnull, xo + d * 16,
                                                       kb * 256, 0));
  };
  load_a(0, 0);
  load_a(1, 1);
  if constexpr (NP > 1) copy_pair(1);
  if (prio) __builtin_amdgcn_s_setprio(0);

  const uint32_t dq_mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(dq_magic));
  const uint16_t* sc_lds = reinterpret_cast<const uint16_t*>(scl);
  const int cc = cnt - r_begin < 16 ? cnt - r_begin : 16;
  f32x4_t tot[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) tot[rs] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int pswz = (u.r16 >> 1) & 7;  // rows rs * 16 + r16 share it
  // Loads in flight behind k-block kbl's operands, in issue order: for kbl = 0
  // the second activation fragments and pair 1; for kbl = 1 pair 1 and k-block
  // 2's activations (issued in the loop after pair 1); for kbl = 2 k-block 3's
  // activations.
#pragma unroll
  for (int kbl = 0; kbl < CK; ++kbl) {
    const int p = kbl & 1;
    if (kbl == 0) {
      wait_vm_le<4 + (NP > 1 ? 2 * RS : 0)>();
    } else if (kbl == 1 && NP > 1) {
      wait_vm_le<2 * RS + 4>();
    } else if (kbl == 2) {
      wait_vm_le<4>();
    } else {
      wait_vm_all();
    }
    uint4 xa[4];
    f32x4_t init;
    make_a<2, BF, PH>(areg[p], xa, init);
    const unsigned char* kp_lds = pbuf(kbl >> 1);
    const int poff = ((((kbl & 1) * 4 + u.kq) ^ pswz)) * 16;
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
      const uint4 w = *reinterpret_cast<const uint4*>(kp_lds + (rs * 16 + u.r16) * 128 + poff);
      f32x4_t acc = dmfma<BF>(xa[0], ddeq4(w.x, dq_mask, dq_magic), init);
      acc = dmfma<BF>(xa[1], ddeq4(w.y, dq_mask, dq_magic), acc);
      acc = dmfma<BF>(xa[2], ddeq4(w.z, dq_mask, dq_magic), acc);
      acc = dmfma<BF>(xa[3], ddeq4(w.w, dq_mask, dq_magic), acc);
      // past the wave's range the activations (and so acc) are zero
      const float sc =
          kbl < u.nmy ? f16_bits_to_f32(sc_lds[(rs * 16 + u.r16) * u.ng + ((u.lo + kbl) >> a.gshift)])
                      : 0.f;
      tot[rs] += sc * acc;
    }
    if (kbl + 2 < CK) load_a(p, kbl + 2);
  }
  // partial tiles into pair 0's array (this wave's reads of it are done)
  wave_lds_fence();
  float4* red = reinterpret_cast<float4*>(pbuf(0));
#pragma unroll
  for (int rs = 0; rs < RS; ++rs)
    red[rs * 64 + u.lane] = float4{tot[rs][0], tot[rs][1], tot[rs][2], tot[rs][3]};
  __syncthreads();
  finish_pass<2, BF, PH, NT, KPB>(a, u, s_kp0, sl, cc, 1, blk);
  __syncthreads();  // LDS arrays free again
}

// INT4 gate/up unit whose k-range is longer than the wave's LDS region
// holds (large hidden sizes): the range is copied and consumed in chunks of
// CK k-blocks, each a whole-slice LDS DMA like run_unit_dma's, accumulating
// in registers across chunks.  A wave's region is its own, so a chunk's copy
// only waits for the wave's own reads of the previous chunk.  Twice the bytes
// of the register ring are in flight per wave (8 KiB, 32 rows x 4 k-blocks).
// The group scales of the whole k-range are copied once with 4-byte LDS DMA
// (row r's groups g_lo.. as nd dwords from its aligned start).
template <bool BF, int NT>
__device__ __forceinline__ void run_unit_dma_chunked(const LayerArgs& a, const Route& rt, int e,
                                                     int blk, int tile, unsigned char* lds,
                                                     bool once) {
  constexpr int PH = 0;
  using G = Geo<2, PH, NT>;
  constexpr int RS = G::RS, CK = G::CK;
  constexpr int DA = NT == 4 ? 1 : 2;  // activation k-blocks in flight
  const UnitCtx<2, PH, NT> u(a, e, blk, 0);
  unsigned char* region = lds + u.wave * WAVE_LDS;

  const int g_lo = u.lo >> a.gshift;
  const int ngw = u.nmy > 0 ? ((u.lo + u.nmy - 1) >> a.gshift) - g_lo + 1 : 1;
  const int nd = (ngw * 2 + 2 + 3) >> 2;  // dwords per row (2 bytes of alignment slack)
  {
    unsigned char* dst = region + WAVE_W;
    const int nflat = RS * 16 * nd;
    for (int i0 = 0; i0 < nflat; i0 += 64) {  // wave-uniform trip count
      const int f = i0 + u.lane;
      const int rr = f / nd, d = f - (f / nd) * nd;
      const bool in = f < nflat;
      const int b0 = (u.row(a, blk, in ? rr : 0) * u.ng + g_lo) * 2;
      dma4(u.sr, dst + i0 * 4, in ? (b0 & ~3) + d * 4 : OOB_OFF);
    }
  }
  const uint16_t* sc_lds = reinterpret_cast<const uint16_t*>(region + WAVE_W);
  auto scale_at = [&](int rs, int kb) {
    const int row = u.row(a, blk, rs * 16 + u.r16);
    const int e0 = ((row * u.ng + g_lo) * 2) & 2;
    return f16_bits_to_f32(sc_lds[((rs * 16 + u.r16) * nd * 4 + e0) / 2 + ((kb >> a.gshift) - g_lo)]);
  };

  const int r_begin = tile * NT * 16;
  int sl[NT];
  const int cnt = __builtin_amdgcn_readfirstlane(lane_slots<NT>(a, rt, e, r_begin, sl));
  const uint32_t dq_mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(dq_magic));

  for (int r0 = r_begin; r0 < cnt && r0 < r_begin + NT * 16; r0 += NT * 16) {
    const int cc = cnt - r0 < NT * 16 ? cnt - r0 : NT * 16;
    const int ntiles = (cc + 15) >> 4;
    int xo[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) xo[tt] = u.xoff(a, sl[tt]);
    f32x4_t tot[RS][NT];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int t = 0; t < NT; ++t) tot[rs][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int c0 = 0; c0 < u.nmy; c0 += CK) {  // wave-uniform
      const int nc = u.nmy - c0 < CK ? u.nmy - c0 : CK;
      const int p4 = 4 * nc;               // 16-byte pieces per row in LDS
      const int xm = (nc & 1) ? 3 : 7;     // swizzle mask keeps c ^ (rr & xm) < p4
      if (c0 > 0) wave_lds_fence();        // this wave's reads of the last chunk are done
      for (int j = 0; j < RS * nc; ++j) {  // 64 pieces per instruction
        const int p = j * 64 + u.lane;
        const int rr = p / p4;
        const int c = (p - rr * p4) ^ (rr & xm);
        const int off = u.row(a, blk, rr) * u.rowbytes + (u.lo + c0) * 64 + c * 16;
        if (once)  // a slice this unit alone reads: nontemporal
          dma16_nt(u.wr, region + j * 1024, off);
        else
          dma16(u.wr, region + j * 1024, off);
      }
      uint4 areg[DA][4 * NT];
      auto load_a = [&](int p, int kbl) {  // zeros past the chunk
        const bool ok = uni_b(kbl < nc);
        const int kb = uni_i(ok ? u.lo + c0 + kbl : u.lo);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int d = 0; d < 4; ++d)
            areg[p][tt * 4 + d] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(ok ? u.xr : u.xnull,
                                                             xo[tt] + d * 16, kb * 256, 0));
      };
#pragma unroll
      for (int p = 0; p < DA; ++p) load_a(p, p);
      wait_vm_all();  // the chunk (and, the first time, the scales) has landed
#pragma unroll
      for (int kbl = 0; kbl < CK; ++kbl) {
        const int p = kbl % DA;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
          if (tt < ntiles) {
            uint4 xa[4];
            f32x4_t init;
            make_a<2, BF, PH>(&areg[p][tt * 4], xa, init);
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) {
              const int rr = rs * 16 + u.r16;
              const int cpos = kbl * 4 + u.kq;
              const int off = kbl < nc ? (rr * p4 + (cpos ^ (rr & xm))) * 16 : 0;
              const uint4 w = *reinterpret_cast<const uint4*>(region + off);
              f32x4_t acc = dmfma<BF>(xa[0], ddeq4(w.x, dq_mask, dq_magic), init);
              acc = dmfma<BF>(xa[1], ddeq4(w.y, dq_mask, dq_magic), acc);
              acc = dmfma<BF>(xa[2], ddeq4(w.z, dq_mask, dq_magic), acc);
              acc = dmfma<BF>(xa[3], ddeq4(w.w, dq_mask, dq_magic), acc);
              // past the chunk the activations (and so acc) are zero
              const float sc = kbl < nc ? scale_at(rs, u.lo + c0 + kbl) : 0.f;
              tot[rs][tt] += sc * acc;
            }
          }
        }
        if (kbl + DA < CK) load_a(p, kbl + DA);
      }
    }
    wave_lds_fence();  // the last chunk's reads are done before the partial tiles
    float4* red = reinterpret_cast<float4*>(region);
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (tt < ntiles)
          red[(rs * NT + tt) * 64 + u.lane] =
              float4{tot[rs][tt][0], tot[rs][tt][1], tot[rs][tt][2], tot[rs][tt][3]};
    __syncthreads();
    finish_pass<2, BF, PH, NT>(a, u, lds, sl, cc, ntiles, blk);
    __syncthreads();  // LDS regions free again
  }
}

// General unit (any tier, any K): each wave streams k-blocks lo .. lo+nmy-1
// through a register ring of P k-blocks.  Every ring slot is refilled
// unconditionally: a k-block beyond the wave's range is read through a
// zero-length buffer resource, which returns zeros without a memory access
// (and contributes exactly zero), so the number of loads in flight is the
// same on every path and each slot waits only for its own loads.  The first
// ring fill of weights is issued before the expert's rows are gathered.
template <int TIER, bool BF, int PH, int NT, typename Rows>
__device__ __forceinline__ void run_unit_ring(const LayerArgs& a, const Rows& rows, int e, int blk,
                                              int sp, int tile, unsigned char* lds, int widx = -1) {
  using G = Geo<TIER, PH, NT>;
  constexpr int RS = G::RS, QPK = G::QPK, P = G::P;
  // BF16 and INT8 down units take their 64 rows in two passes of 32, so that
  // a ring slot holds half the weight registers (32 instead of 64 for BF16)
  constexpr int RSP = (TIER != 2 && PH == 1) ? RS / 2 : RS;  // row sets per pass
  constexpr int NPASS = RS / RSP;
  using pass0_t = std::integral_constant<int, 0>;
  const UnitCtx<TIER, PH, NT> u(a, e, blk, sp, widx);
  // A lane's 16-byte weight loads of a k-block: INT4 (one) at kq * 16; BF16 /
  // INT8 (four / two) at kq * 16 + h * 64, so that each load instruction reads
  // 64 contiguous bytes of every row and the lane holds, for MFMA step d, k
  // = 32 d + 8 kq .. (BF16) or 64 (d / 2) + 16 kq + 8 (d % 2) .. (INT8); the
  // activation fragments are read in the same k order (a_off below).
  constexpr int WSTEP = TIER == 2 ? 16 : 64;
  int voff[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs)
    voff[rs] = u.row(a, blk, rs * 16 + u.r16) * u.rowbytes + u.kq * 16;
  const uint32_t dq_mask = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(dq_magic));

  // INT4 group scales of the wave's k-range, copied into LDS behind the
  // partial-tile area with 4-byte LDS-DMA instructions (row r's groups
  // g_lo.. as nd dwords from its aligned start) before the ring loads, so the
  // k-loop reads them from LDS instead of issuing scattered 2-byte loads.
  const int g_lo = u.lo >> a.gshift;
  const int ngw = u.nmy > 0 ? ((u.lo + u.nmy - 1) >> a.gshift) - g_lo + 1 : 1;
  const int nd = (ngw * 2 + 2 + 3) >> 2;  // dwords per row (2 bytes of alignment slack)
  const uint16_t* sc_lds = reinterpret_cast<const uint16_t*>(lds + u.wave * WAVE_LDS + SCALE_OFF);
  if constexpr (TIER == 2) {
    unsigned char* dst = lds + u.wave * WAVE_LDS + SCALE_OFF;
    const int nflat = RS * 16 * nd;
    for (int i0 = 0; i0 < nflat; i0 += 64) {  // wave-uniform trip count
      const int f = i0 + u.lane;
      const int rr = f / nd, d = f - (f / nd) * nd;
      const bool in = f < nflat;
      const int b0 = (u.row(a, blk, in ? rr : 0) * u.ng + g_lo) * 2;
      dma4(u.sr, dst + i0 * 4, in ? (b0 & ~3) + d * 4 : OOB_OFF);
    }
    __builtin_amdgcn_sched_barrier(0);  // the copies go out before the ring loads
  }
  // scale of row-set row rs*16 + r16, k-block kb (in the wave's range)
  auto scale_at = [&](int rs, int kb) {
    const int row = u.row(a, blk, rs * 16 + u.r16);
    const int e0 = ((row * u.ng + g_lo) * 2) & 2;
    return f16_bits_to_f32(
        sc_lds[((rs * 16 + u.r16) * nd * 4 + e0) / 2 + ((kb >> a.gshift) - g_lo)]);
  };

  uint4 wreg[P][RSP * QPK];
  uint4 areg[P][4 * NT];
  int xo[NT];
  auto load_w = [&](int p, int kbl, auto rs0c) {  // row sets rs0 .. rs0 + RSP - 1
    constexpr int rs0 = decltype(rs0c)::value;
    const bool ok = uni_b(kbl < u.nmy);
    const __amdgpu_buffer_rsrc_t r = ok ? u.wr : u.wnull;
    const int kb = uni_i(ok ? u.lo + kbl : u.lo);
#pragma unroll
    for (int rs = 0; rs < RSP; ++rs) {
#pragma unroll
      for (int h = 0; h < QPK; ++h)
        wreg[p][rs * QPK + h] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff[rs0 + rs] + h * WSTEP, kb * G::KBSTRIDE, 0));
    }
  };
  // byte offset of step d's activation fragment from the lane's row start
  // (u.xoff puts lane kq at k = 32 kq, the INT4 order)
  auto a_off = [&](int d) {
    if constexpr (TIER == 2) return d * 16;
    else if constexpr (TIER == 0) return d * 64 - u.kq * 48;
    else return (d >> 1) * 128 + (d & 1) * 16 - u.kq * 32;
  };
  auto load_a = [&](int p, int kbl) {
    const bool ok = uni_b(kbl < u.nmy);
    const int kb = uni_i(ok ? u.lo + kbl : u.lo);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int d = 0; d < 4; ++d)
        areg[p][tt * 4 + d] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(ok ? u.xr : u.xnull, xo[tt] + a_off(d),
                                                         kb * 256, 0));
  };

#pragma unroll
  for (int p = 0; p < P; ++p) load_w(p, p, pass0_t{});
  // this unit's rows: tile `tile` of the expert's rows (one pass)
  const int r_begin = tile * NT * 16;
  int sl[NT];
  const int cnt = __builtin_amdgcn_readfirstlane(rows.template slots<NT>(a, e, r_begin, sl));

  for (int r0 = r_begin; r0 < cnt && r0 < r_begin + NT * 16; r0 += NT * 16) {
    const int cc = cnt - r0 < NT * 16 ? cnt - r0 : NT * 16;
    const int ntiles = (cc + 15) >> 4;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) xo[tt] = u.xoff(a, sl[tt]);
#pragma unroll
    for (int p = 0; p < P; ++p) load_a(p, p);

    f32x4_t tot[RS][NT];
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int t = 0; t < NT; ++t) tot[rs][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // the scale copies were issued before every ring load now outstanding
    if constexpr (TIER == 2) {
      if (r0 == 0) wait_vm_le<P * (RS * QPK + 4 * NT)>();
    }

    // the k-loop over row sets rs0 .. rs0 + RSP - 1 (ring already filled)
    auto kloop = [&](auto rs0c) {
    constexpr int rs0 = decltype(rs0c)::value;
    for (int kb0 = 0; kb0 < u.nmy; kb0 += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        // One row set's weights as MFMA B operands (exact base + q values).
        auto dequant = [&](int rs, uint4 (&bfr)[4], float& sc) {
          sc = 1.f;
          if constexpr (TIER == 2) {
            const uint4 w = wreg[p][rs];
            bfr[0] = ddeq4(w.x, dq_mask, dq_magic);
            bfr[1] = ddeq4(w.y, dq_mask, dq_magic);
            bfr[2] = ddeq4(w.z, dq_mask, dq_magic);
            bfr[3] = ddeq4(w.w, dq_mask, dq_magic);
            // past the wave's range the activations (so acc) are zero
            sc = kb0 + p < u.nmy ? scale_at(rs0 + rs, u.lo + kb0 + p) : 0.f;
          } else if constexpr (TIER == 1) {
            const uint4 w0 = wreg[p][rs * QPK + 0], w1 = wreg[p][rs * QPK + 1];
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
            for (int h = 0; h < 4; ++h) bfr[h] = wreg[p][rs * QPK + h];
          }
        };
        if constexpr (NT == 1) {
          // A operand first, then one row set at a time
          uint4 xa[4];
          f32x4_t init;
          make_a<TIER, BF, PH>(&areg[p][0], xa, init);
#pragma unroll
          for (int rs = 0; rs < RSP; ++rs) {
            uint4 bfr[4];
            float sc;
            dequant(rs, bfr, sc);
            f32x4_t acc = init;
#pragma unroll
            for (int d = 0; d < 4; ++d) acc = dmfma<BF>(xa[d], bfr[d], acc);
            tot[rs0 + rs][0] += sc * acc;
          }
        } else {
          // several tiles: one tile's A operand at a time (fewer live registers)
#pragma unroll
          for (int tt = 0; tt < NT; ++tt) {
            if (tt < ntiles) {
              uint4 xa[4];
              f32x4_t init;
              make_a<TIER, BF, PH>(&areg[p][tt * 4], xa, init);
#pragma unroll
              for (int rs = 0; rs < RSP; ++rs) {
                uint4 bfr[4];
                float sc;
                dequant(rs, bfr, sc);
                f32x4_t acc = init;
#pragma unroll
                for (int d = 0; d < 4; ++d) acc = dmfma<BF>(xa[d], bfr[d], acc);
                tot[rs0 + rs][tt] += sc * acc;
              }
            }
          }
        }
        load_w(p, kb0 + p + P, rs0c);  // refill this ring slot (zeros past the range)
        load_a(p, kb0 + p + P);
        // keep the ring order: slot p's refill is issued before slot p+1 is consumed
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    };
    kloop(pass0_t{});
    if constexpr (NPASS == 2) {  // the second half of the rows: fill the ring again
#pragma unroll
      for (int p = 0; p < P; ++p) {
        load_w(p, p, std::integral_constant<int, RSP>{});
        load_a(p, p);
      }
      kloop(std::integral_constant<int, RSP>{});
    }
    float4* red = reinterpret_cast<float4*>(lds + u.wave * WAVE_LDS);
#pragma unroll
    for (int rs = 0; rs < RS; ++rs)
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (tt < ntiles)
          red[(rs * NT + tt) * 64 + u.lane] =
              float4{tot[rs][tt][0], tot[rs][tt][1], tot[rs][tt][2], tot[rs][tt][3]};
    __syncthreads();
    finish_pass<TIER, BF, PH, NT>(a, u, lds, sl, cc, ntiles, blk);
    __syncthreads();  // LDS regions free again
  }
}

// One unit of either phase: the tier (mixed banks) and the INT4 path pick its
// routine.  `rt` is the work-group's routing (only the chunked gate/up path
// reads it directly).
template <bool BF, int PH, int NT, bool MIXED, int PATH, typename Rows>
__device__ __forceinline__ void run_unit_any(const LayerArgs& a, const Rows& rows, const Route* rt,
                                             int e, int blk, int sp, int t, uint32_t ev,
                                             unsigned char* dyn_lds, bool prio, bool once) {
  const int tier = (int)(ev >> 30);
  const int widx = MIXED ? (int)(ev & kRowMask) : -1;
  if (!MIXED || tier == 2) {
    if constexpr (PATH == 1 && NT == 1 && !MIXED)
      run_unit_kb<BF, PH>(a, rows, e, blk, sp, t, prio, once);
    else if constexpr (PATH == 1)
      run_unit_dma<BF, PH, NT>(a, rows, e, blk, sp, t, dyn_lds, widx, once);
    else if constexpr (PATH == 2 && PH == 0)
      run_unit_dma_chunked<BF, NT>(a, *rt, e, blk, t, dyn_lds, once);
    else
      run_unit_ring<2, BF, PH, NT>(a, rows, e, blk, sp, t, dyn_lds, widx);
  } else if constexpr (MIXED) {
    if (tier == 1)
      run_unit_ring<1, BF, PH, NT>(a, rows, e, blk, sp, t, dyn_lds, widx);
    else
      run_unit_ring<0, BF, PH, NT>(a, rows, e, blk, sp, t, dyn_lds, widx);
  }
}

// Gate/up (PH 0): a grid of at most one resident round of work-groups; each
// routes once and then takes units blockIdx.x, blockIdx.x + gridDim.x, ...
// (unit u is row block u % nb of the (u / nb)-th tile), and finally writes
// its share of the down kernel's plan.  Down (PH 1): each unit's tile record
// comes from that plan.
// Four waves per SIMD (four work-groups per CU, at most 128 VGPRs), the
// mixed-tier down kernel included: its BF16 and INT8 units hold their 64
// weight rows in two passes of 32 (run_unit_ring), which keeps it within 128
// registers without spills (at two waves per SIMD it left half the resident
// slots empty: DeepSeek-V2-Lite T=64 120.5 -> 118.0 us, the mixed OLMoE
// stack at T=32 88.9 -> 87.0).
// The down kernel's plan (see kPlanHdrInts), written by wave 0 of the
// gate/up work-groups from their routing: tile j's record by work-group
// gridDim.x - 1 - (j % gridDim.x), the tile count and the validity bits by the
// last work-group.
template <bool MIXED>
__device__ __forceinline__ void write_plan(const LayerArgs& a, const Route& rt, const uint32_t* cntw,
                                        const int* emap, uint32_t word, int incl, int c,
                                        int incl_u, int n_tiles, int nb) {
  const int lane = threadIdx.x & 63;
  const int w_last = (int)gridDim.x - 1 - (int)blockIdx.x;
  for (int j = w_last; j < n_tiles; j += gridDim.x) {
    const int u = j * nb;  // the tile's first unit
    const int t = __popcll(__ballot(incl_u <= u));
    const int v = u - (t > 0 ? __builtin_amdgcn_readlane(incl_u, t - 1) : 0);
    const int ai = v / nb;
    const int e = t == 0 ? select_expert(ai, word, incl, c) : select_tiled_expert(a, cntw, rt, t, ai);
    int sl[1];
    const int cnt = lane_slots<1>(a, rt, e, t * 16, sl);
    int* rec = a.plan + kPlanHdrInts + j * kPlanRecInts;
    if (lane < 16) rec[kPlanSlotOff + lane] = sl[0];
    if (lane == 0) {
      rec[0] = e | (t << 16);
      rec[1] = cnt;
      rec[2] = MIXED ? emap[e] : 0;
    }
  }
  if (w_last == 0) {
    // validity bits of the routed slots, for the down kernel's combine
    const int n = a.T * a.k;
    for (int s0 = 0; s0 < n; s0 += 64) {
      const uint64_t m = __ballot(s0 + lane < n && rt.ids[s0 + lane] >= 0);
      if (lane < 2) a.plan[kPlanMaskOff + (s0 >> 5) + lane] = (int)(uint32_t)(m >> (32 * lane));
    }
    if (lane == 0) a.plan[0] = n_tiles;
  }
}

template <bool BF, int NT, bool MIXED, int PATH>
__device__ __forceinline__ void decode_gateup(const LayerArgs& a, unsigned char* dyn_lds) {
  constexpr int PH = 0;
  __shared__ Route rt;
  // rows per expert, behind the per-wave regions (the k-block LDS path keeps
  // its slices in static arrays and has only this in dynamic LDS)
  uint32_t* cntw =
      reinterpret_cast<uint32_t*>(dyn_lds + (PATH == 1 && NT == 1 && !MIXED ? 0 : DW * WAVE_LDS));
  // the down launch that follows on this stream starts from zero counters,
  // whatever an earlier call (or the caller's fill) left in the workspace
  for (int i = blockIdx.x * DNT + threadIdx.x; i <= kDecodeMaxHBlocks; i += gridDim.x * DNT)
    __hip_atomic_store(sync_c(a, i), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // mixed banks: every expert's (tier << 30) | row, behind the row counts
  int* emap = reinterpret_cast<int*>(cntw + ((a.Ep + 1) >> 1));
  uint32_t word;
  int incl, c;
  const int n_active = route<MIXED>(a, rt, cntw, word, incl, c, emap);
  const int w_last = (int)gridDim.x - 1 - (int)blockIdx.x;  // 0 for the last work-group
  if (n_active == 0) {  // nothing routed: the down kernel writes a zero output
    if (w_last == 0 && threadIdx.x == 0) a.plan[0] = 0;
    return;
  }
  // Unit u = (token tile, row block); tiles in segments (tile 0 of every
  // active expert, then tile 1 of the experts with more than 16 rows, ...),
  // so a busy expert's tiles run side by side.
  const int nb = a.nbA;
  int n_tiles = n_active;
  int incl_u = n_active * nb;  // inclusive prefix of the segments' unit counts, lane t = segment t
  if (rt.multi) {              // (otherwise every expert is one tile: segment 0 only)
    const int seg = tile_segments(a, cntw, rt, &n_tiles);
    incl_u = seg * nb;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl_u, o, 64);
      if (lane >= o) incl_u += v;
    }
  }
  const int n_units = n_tiles * nb;
  // unit u -> (expert, row block, tile); uniform across the work-group
  auto decode = [&](int u, int& e, int& blk, int& t) {
    t = __popcll(__ballot(incl_u <= u));  // segment = tile index
    const int v = u - (t > 0 ? __builtin_amdgcn_readlane(incl_u, t - 1) : 0);
    const int ai = v / nb;
    blk = v - ai * nb;
    e = t == 0 ? select_expert(ai, word, incl, c) : select_tiled_expert(a, cntw, rt, t, ai);
  };
  const RowsRoute rows{rt};
  for (int u = blockIdx.x; u < n_units; u += gridDim.x) {
    int e, blk, t;
    decode(u, e, blk, t);
    const uint32_t ev = MIXED ? (uint32_t)__builtin_amdgcn_readfirstlane(emap[e]) : (2u << 30);
    // the expert's only 16-row tile reads its slice once
    const bool once = expert_rows(cntw, e) <= 16;
    run_unit_any<BF, PH, NT, MIXED, PATH>(a, rows, &rt, e, blk, 0, t, ev, dyn_lds,
                                         n_units > 2 * (int)gridDim.x, once);
  }
  // The down kernel's plan, after this work-group's own units (the last
  // work-groups of the grid hold the fewest units); the routing state in LDS
  // is untouched by the units (they use the per-wave regions and the k-block
  // arrays).
  if (threadIdx.x < 64) write_plan<MIXED>(a, rt, cntw, emap, word, incl, c, incl_u, n_tiles, nb);
}

template <bool BF, int NT, bool MIXED, int PATH>
__device__ __forceinline__ void decode_down(const LayerArgs& a, unsigned char* dyn_lds) {
  constexpr int PH = 1;
  __shared__ int s_flag;
  const int lane = threadIdx.x & 63;
  const int ns = a.nsplit;
  const int nb = a.nbB * ns;  // units per tile: row blocks x k-splits, the split fastest
  // The first unit's record goes out beside the tile count (the grid has at
  // most one work-group per unit of the largest plan, so the record index is
  // inside the plan even before the count is known).
  const int* recs = a.plan + kPlanHdrInts;
  int u = blockIdx.x;
  int j = u / nb;
  int4 h = *reinterpret_cast<const int4*>(recs + j * kPlanRecInts);
  int slot = recs[j * kPlanRecInts + kPlanSlotOff + (lane & 15)];
  const int n_tiles = __builtin_amdgcn_readfirstlane(a.plan[0]);
  if (n_tiles == 0) {  // nothing routed: the output is zero
    uint4* o = reinterpret_cast<uint4*>(a.out);
    const int64_t n16 = (int64_t)a.T * a.H / 8;
    for (int64_t i = (int64_t)blockIdx.x * DNT + threadIdx.x; i < n16; i += (int64_t)gridDim.x * DNT)
      o[i] = uint4{0u, 0u, 0u, 0u};
    return;
  }
  const int n_units = n_tiles * nb;
  while (u < n_units) {
    const int bs = u - j * nb;
    const int blk = bs / ns, sp = bs - blk * ns;
    const int e = __builtin_amdgcn_readfirstlane(h.x & 0xffff);
    const int t = __builtin_amdgcn_readfirstlane(h.x >> 16);
    const RowsPlan rows{__builtin_amdgcn_readfirstlane(h.y), slot};
    const uint32_t ev = MIXED ? (uint32_t)__builtin_amdgcn_readfirstlane(h.z) : (2u << 30);
    run_unit_any<BF, PH, NT, MIXED, PATH>(a, rows, nullptr, e, blk, sp, t, ev, dyn_lds,
                                         n_units > 2 * (int)gridDim.x, rows.cnt <= 16);
    if (a.combine) publish_and_combine<BF, rows_b(NT)>(a, blk, n_tiles, &s_flag);
    u += gridDim.x;
    if (u < n_units) {
      j = u / nb;
      h = *reinterpret_cast<const int4*>(recs + j * kPlanRecInts);
      slot = recs[j * kPlanRecInts + kPlanSlotOff + (lane & 15)];
    }
  }
}

template <bool BF, int PH, int NT, bool MIXED, int PATH>  // INT4 path: 0 ring, 1 LDS, 2 chunked LDS
__global__ void __launch_bounds__(DNT, 4) moe_decode_kernel(LayerArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn_lds[];
  if constexpr (PH == 0)
    decode_gateup<BF, NT, MIXED, PATH>(a, dyn_lds);
  else
    decode_down<BF, NT, MIXED, PATH>(a, dyn_lds);
}

// The down phase's combine as a launch of its own (LayerArgs::combine == 0):
// out[t, h..h+3] = sum over the token's slots j (ascending) of weight * the
// slot's partial row (its k-splits summed in split order first), fp32,
// rounded once -- the same order and arithmetic as combine_block.  One thread
// per four consecutive h, in 64-thread work-groups so that even one token's
// row spreads over several CUs; the kernel boundary makes every partial row
// visible.  Slots are taken kCombineBatch at a time: their ids and weights
// are loaded as raw bits, then the first kCombineBatch (slot, split) partial
// loads go out, and only then are the ids and weights converted (so the
// partial loads do not wait behind them: Mixtral's two slots x eight splits
// at one token are one memory round trip).  A dropped slot's rows were never
// written: its loads are replaced by zeros.
constexpr int kCombineThreads = 64;
constexpr int kCombineBatch = 16;

template <bool BF, bool ID64, int WDT>  // ids int64 / int32; weights EXQ_DTYPE_F32 / _BF16 / _F16
__global__ void __launch_bounds__(kCombineThreads) decode_combine_kernel(LayerArgs a) {
  constexpr int CB = kCombineBatch;
  constexpr bool wf32 = WDT == EXQ_DTYPE_F32;
  __shared__ float s_w[CB][kCombineThreads];  // this thread's slot weights (0: dropped)
  const int hq = a.H >> 2;
  const int idx = blockIdx.x * kCombineThreads + threadIdx.x;
  if (idx >= a.T * hq) return;
  const int t = idx / hq;
  const int h = (idx - t * hq) * 4;
  const int64_t set = (int64_t)a.T * a.kp * a.H;  // floats per partial set
  const __amdgpu_buffer_rsrc_t part_r = make_rsrc(a.part, a.nsplit * set * 4);
  const __amdgpu_buffer_rsrc_t ids_r = make_rsrc(a.ids, (int64_t)a.T * a.k * (ID64 ? 8 : 4));
  const __amdgpu_buffer_rsrc_t w_r = make_rsrc(a.topk_w, (int64_t)a.T * a.k * (wf32 ? 4 : 2));
  const float4 zero = float4{0.f, 0.f, 0.f, 0.f};
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < a.kp; j0 += CB) {
    const int nsl = a.kp - j0 < CB ? a.kp - j0 : CB;  // slots of this batch
    // raw ids and weights of slots j0.. (one load each; zeros past the
    // routed slots)
    uint32_t lo[CB], hi[CB], wr[CB];
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int q = t * a.k + j0 + i;
      const bool in = i < nsl && j0 + i < a.k;
      if constexpr (ID64) {
        const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(ids_r, in ? q * 8 : OOB_OFF, 0, 0);
        lo[i] = v[0];
        hi[i] = v[1];
      } else {
        lo[i] = __builtin_amdgcn_raw_buffer_load_b32(ids_r, in ? q * 4 : OOB_OFF, 0, 0);
        hi[i] = 0u;
      }
      if constexpr (wf32)
        wr[i] = __builtin_amdgcn_raw_buffer_load_b32(w_r, in ? q * 4 : OOB_OFF, 0, 0);
      else
        wr[i] = __builtin_amdgcn_raw_buffer_load_b16(w_r, in ? q * 2 : OOB_OFF, 0, 0);
    }
    const int n_it = nsl * a.nsplit;  // item q: slot j0 + q / nsplit, split q % nsplit
    uint32_t okm = 0u;                // bit i: slot j0 + i is routed
    int jj = 0, sp = 0;               // slot (from j0) and split of the next item
    float4 cur = zero;                // the current slot's splits so far
    float cw = 0.f;
    float4 pv[CB];
    // items q0.. of the batch: every partial load in flight at once
    auto issue = [&](int q0) {
      int js = jj, ss = sp;
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const int off = q0 + i < n_it
                            ? (int)((ss * set + (int64_t)(t * a.kp + j0 + js) * a.H + h) * 4)
                            : OOB_OFF;
        pv[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(part_r, off, 0, 0));
        if (++ss == a.nsplit) {
          ss = 0;
          ++js;
        }
      }
    };
    auto accumulate = [&](int q0) {
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        if (q0 + i < n_it) {
          if (sp == 0) {
            const bool ok = (okm >> jj) & 1u;
            cw = s_w[jj][threadIdx.x];
            cur = ok ? pv[i] : zero;
          } else if ((okm >> jj) & 1u) {  // further k-splits, in split order
            cur.x += pv[i].x; cur.y += pv[i].y; cur.z += pv[i].z; cur.w += pv[i].w;
          }
          if (sp == a.nsplit - 1) {
            acc[0] += cw * cur.x;
            acc[1] += cw * cur.y;
            acc[2] += cw * cur.z;
            acc[3] += cw * cur.w;
          }
          if (++sp == a.nsplit) {
            sp = 0;
            ++jj;
          }
        }
      }
    };
    issue(0);
    // the slots' ids and weights, converted after the partial loads are out
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int j = j0 + i;
      const int64_t id = ID64 ? (int64_t)(((uint64_t)hi[i] << 32) | lo[i]) : (int64_t)(int32_t)lo[i];
      const bool ok = j >= a.k || (id >= 0 && id < a.E);  // shared experts: weight 1
      const float wf = j >= a.k                  ? 1.f
                       : wf32                    ? __builtin_bit_cast(float, wr[i])
                       : WDT == EXQ_DTYPE_BF16 ? bf16_bits_to_f32(wr[i])
                                                 : f16_bits_to_f32(wr[i]);
      okm |= (ok ? 1u : 0u) << i;
      s_w[i][threadIdx.x] = ok ? wf : 0.f;
    }
    accumulate(0);
    for (int q0 = CB; q0 < n_it; q0 += CB) {
      issue(q0);
      accumulate(q0);
    }
  }
  uint2 o;
  o.x = to_act_bits<BF>(acc[0]) | (to_act_bits<BF>(acc[1]) << 16);
  o.y = to_act_bits<BF>(acc[2]) | (to_act_bits<BF>(acc[3]) << 16);
  *reinterpret_cast<uint2*>(a.out + (int64_t)t * a.H + h) = o;
}

// ---- few tokens: the down projection by output rows ------------------------
// For a few tokens (T * (k + shared) <= ROWS_MAX_SLOTS) a work-group owns
// rows_r(NCH) output rows across all of the batch's routed slots and sums each
// token's slots itself: no fp32 partial rows, no counters, no combine tail
// (at T = 1 that tail is most of the down kernel's time).  A slot's weights
// are read per slot, so an expert routed by several tokens is read again (from
// L2).  Half-wave hw of slot group s0 takes slot s0 + hw (token s / kp); its
// 32 lanes take the 32-k chunks c = lane, lane + 32, ... of the slot's `mid`
// row (stored in INT4 pairing order: pairs (k, k + 4) of each
// 8-group) and, for each of the rows, the matching 16 packed bytes.  Nibbles
// become exact 16-bit floats base + n with one v_and_or_b32 per pair, in the
// same pairing order, and v_dot2 multiplies and adds them in fp32; the
// constant base is removed once per chunk (a v_dot2 of `mid` against ones),
// and the fp16 group scale multiplies the chunk's sum.  Each half-wave's 32
// lane sums are folded in a fixed order (DPP inside 16-lane rows, then the
// two rows), and each token's weighted slot rows are summed in ascending slot
// order: the result does not depend on scheduling.
// Output rows per work-group: 4, or 2 when each lane holds two or more
// 32-k chunks of a row (I > 1024), which keeps a lane's loads few and the
// grid twice as wide (DeepSeek-V2-Lite-shaped layer, I = 1408: T=1 17.8 ->
// 17.1 us per layer, T=2 26.0 -> 24.4; at I <= 1024 two rows were 0.3 us
// slower).
constexpr int rows_r(int nch) { return nch >= 2 ? 2 : 4; }
constexpr int ROWS_MAX_SLOTS = 64;  // T * (k + shared)

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

template <bool BF>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (BF)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
}

// The gate/up projection for the same batches, by output rows: work-group
// (x, y) takes routed slot y and the GU_PAIRS (gate j, up I + j) row pairs
// j = x * GU_PAIRS + w, one per wave.  A slot's expert is one load of its id
// (no active-expert list is needed).  Lanes take the 32-k chunks c = lane,
// lane + 64, ... of the token's row of x, permuted into the nibbles' pairing
// order, and dot2 both rows' dequantised nibbles against it (as in
// decode_down_rows_kernel); the folded gate and up sums give SiLU(g) * u, stored
// in `mid` in INT4 pairing order.
constexpr int GU_PAIRS = 4;            // = waves per work-group
constexpr int GU_THREADS = GU_PAIRS * 64;

template <bool BF, int NCH>  // NCH >= ceil(H / 2048): 32-k chunks per lane, all loads issued first
__global__ void __launch_bounds__(GU_THREADS) decode_gateup_rows_kernel(LayerArgs a) {
  const int s = blockIdx.y;  // routed slot t * kp + j
  const int t = s / a.kp, js = s - t * a.kp;
  int e;
  if (js < a.k) {
    const int64_t id = load_index(a.ids, a.ids_dtype, (int64_t)t * a.k + js);
    if (id < 0 || id >= a.E) return;  // dropped slot: no mid row (the down kernel skips it)
    e = (int)id;
  } else {
    e = a.E + (js - a.k);  // shared expert
  }
  const int lane = threadIdx.x & 63, l = lane;
  const int j = blockIdx.x * GU_PAIRS + (threadIdx.x >> 6);  // gate row j, up row I + j
  const int C = a.H >> 5;
  const int gch = 4 << a.gshift;
  const int ng = a.H >> (7 + a.gshift);
  const int rowb = a.H >> 1;
  const uint32_t dq_mask = 0x000F000Fu;
  const uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  const uint32_t ones = BF ? 0x3F803F80u : 0x3C003C00u;
  const float base = BF ? 136.f : 1032.f;
  const int64_t rg = (int64_t)(a.index ? a.index[e] : e) * 2 * a.I + j;  // gate row
  const int64_t ru = rg + a.I;                                            // up row
  const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.w13.i4 + rg * rowb, rowb);
  const __amdgpu_buffer_rsrc_t ur = make_rsrc(a.w13.i4 + ru * rowb, rowb);
  const __amdgpu_buffer_rsrc_t gsr = make_rsrc(a.w13.i4_scales + rg * ng, (int64_t)ng * 2);
  const __amdgpu_buffer_rsrc_t usr = make_rsrc(a.w13.i4_scales + ru * ng, (int64_t)ng * 2);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + (int64_t)t * a.H, (int64_t)a.H * 2);
  uint4 xv[NCH][4], gw[NCH], uw[NCH];
  uint32_t gs[NCH], us[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {  // chunk c = l + 64 i; past C the loads return zero
    const int c = l + 64 * i;
    const bool ok = c < C;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      xv[i][d] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? (c * 32 + d * 8) * 2 : OOB_OFF, 0, 0));
    // one token: every weight row is read once, nontemporal (aux 2)
    gw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(gr, ok ? c * 16 : OOB_OFF, 0, 2));
    uw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ur, ok ? c * 16 : OOB_OFF, 0, 2));
    gs[i] = __builtin_amdgcn_raw_buffer_load_b16(gsr, ok ? (c / gch) * 2 : OOB_OFF, 0, 0);
    us[i] = __builtin_amdgcn_raw_buffer_load_b16(usr, ok ? (c / gch) * 2 : OOB_OFF, 0, 0);
  }
  float g = 0.f, u = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    float xsum = 0.f;  // the chunk's sum of x (any order)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      xsum = dot2<BF>(xv[i][d].x, ones, xsum);
      xsum = dot2<BF>(xv[i][d].y, ones, xsum);
      xsum = dot2<BF>(xv[i][d].z, ones, xsum);
      xsum = dot2<BF>(xv[i][d].w, ones, xsum);
      xv[i][d] = dperm(xv[i][d]);  // pairs (k_q, k_q+4), the nibbles' order
    }
    float ag = 0.f, au = 0.f;
    const uint32_t pg[4] = {gw[i].x, gw[i].y, gw[i].z, gw[i].w};
    const uint32_t pu[4] = {uw[i].x, uw[i].y, uw[i].z, uw[i].w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      ag = dot2<BF>((pg[d] & dq_mask) | dq_magic, xv[i][d].x, ag);
      ag = dot2<BF>(((pg[d] >> 4) & dq_mask) | dq_magic, xv[i][d].y, ag);
      ag = dot2<BF>(((pg[d] >> 8) & dq_mask) | dq_magic, xv[i][d].z, ag);
      ag = dot2<BF>(((pg[d] >> 12) & dq_mask) | dq_magic, xv[i][d].w, ag);
      au = dot2<BF>((pu[d] & dq_mask) | dq_magic, xv[i][d].x, au);
      au = dot2<BF>(((pu[d] >> 4) & dq_mask) | dq_magic, xv[i][d].y, au);
      au = dot2<BF>(((pu[d] >> 8) & dq_mask) | dq_magic, xv[i][d].z, au);
      au = dot2<BF>(((pu[d] >> 12) & dq_mask) | dq_magic, xv[i][d].w, au);
    }
    // a chunk past C read zeros: its sums and scale are zero
    g += f16_bits_to_f32(gs[i]) * (ag - base * xsum);
    u += f16_bits_to_f32(us[i]) * (au - base * xsum);
  }
  // fold each half-wave's 32 lanes (fixed order), as decode_down_rows_kernel
  auto fold = [&](float v, float& lo, float& hi) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    const int vi = __builtin_bit_cast(int, v);
    lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 16));
    hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 48));
  };
  float g_lo, g_hi, u_lo, u_hi;
  fold(g, g_lo, g_hi);
  fold(u, u_lo, u_hi);
  if (lane == 0) {  // this wave's row pair: both half-waves' sums
    uint16_t* mrow = a.mid + (int64_t)s * a.I;
    mrow[(j & ~7) + pair_pos(j & 7)] = (uint16_t)to_act_bits<BF>(silu_f32(g_lo + g_hi) * (u_lo + u_hi));
  }
}

// MIXED: the bank's tiers per expert (INT4 as above; BF16 rows are multiplied
// as stored, against `mid` put back in natural order; INT8 bytes become exact
// 16-bit pairs and the row's fp16 scale multiplies the sum).  NCH: 32-k chunks
// per lane (all of a lane's loads are issued before its arithmetic).
template <bool BF, bool MIXED, int NCH, bool ONCE>  // ONCE: one token, each weight row read once
__global__ void __launch_bounds__(256) decode_down_rows_kernel(LayerArgs a) {
  constexpr int R = rows_r(NCH);
  __shared__ float red[ROWS_MAX_SLOTS][R];
  const int h0 = blockIdx.x * R;
  const int lane = threadIdx.x & 63, hw = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int C = a.I >> 5;                  // 32-k chunks per row
  const int gch = 4 << a.gshift;           // chunks per scale group
  const int ng = a.I >> (7 + a.gshift);    // scale groups per row
  const int rowb = a.I >> 1;               // packed bytes per INT4 row
  const uint32_t dq_mask = 0x000F000Fu;
  const uint32_t dq_magic = BF ? 0x43004300u : 0x64006400u;
  const uint32_t ones = BF ? 0x3F803F80u : 0x3C003C00u;
  const float base = BF ? 136.f : 1032.f;  // base + 8: (base + n) - (base + 8) = n - 8
  const int n_slots = a.T * a.kp;
  const __amdgpu_buffer_rsrc_t mid_r = make_rsrc(a.mid, (int64_t)n_slots * a.I * 2);
  for (int s0 = 0; s0 < n_slots; s0 += 8) {
    const int s = s0 + hw;
    int e = -1;
    float wt = 0.f;
    if (s < n_slots) {
      const int t = s / a.kp, j = s - t * a.kp;
      if (j < a.k) {
        const int64_t id = load_index(a.ids, a.ids_dtype, (int64_t)t * a.k + j);
        if (id >= 0 && id < a.E) {
          e = (int)id;
          wt = load_as_f32(a.topk_w, a.w_dtype, (int64_t)t * a.k + j);
        }
      } else {
        e = a.E + (j - a.k);  // shared expert, weight 1
        wt = 1.f;
      }
    }
    float part[R];
#pragma unroll
    for (int r = 0; r < R; ++r) part[r] = 0.f;
    if (e >= 0) {
      const int idx = a.index ? a.index[e] : e;  // row of the expert in its tier's bank
      const int tier = MIXED ? (int)a.tier[e] : 2;
      const int64_t row0 = (int64_t)idx * a.H + h0;
      uint4 m[NCH][4];  // mid chunks c = l + 32 i (zeros past C)
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = l + 32 * i;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          m[i][d] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 mid_r, c < C ? (s * a.I + c * 32 + d * 8) * 2 : OOB_OFF, 0, 0));
      }
      if (tier == 2) {
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w2.i4 + row0 * rowb, (int64_t)R * rowb);
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.w2.i4_scales + row0 * ng, (int64_t)R * ng * 2);
        uint4 w[NCH][R];
        uint32_t sc[NCH][R];
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          const int c = l + 32 * i;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            // at one token each weight row is read once: nontemporal (aux 2)
            w[i][r] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, c < C ? r * rowb + c * 16 : OOB_OFF,
                                                             0, ONCE ? 2 : 0));
            sc[i][r] = __builtin_amdgcn_raw_buffer_load_b16(sr, c < C ? (r * ng + c / gch) * 2 : OOB_OFF, 0, 0);
          }
        }
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          float msum = 0.f;  // the chunk's sum of mid values
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            msum = dot2<BF>(m[i][d].x, ones, msum);
            msum = dot2<BF>(m[i][d].y, ones, msum);
            msum = dot2<BF>(m[i][d].z, ones, msum);
            msum = dot2<BF>(m[i][d].w, ones, msum);
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float acc = 0.f;
            const uint32_t pw[4] = {w[i][r].x, w[i][r].y, w[i][r].z, w[i][r].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {  // word d: k = 8d .. 8d + 7; pair q = (k_q, k_q+4)
              const uint32_t p = pw[d];
              acc = dot2<BF>((p & dq_mask) | dq_magic, m[i][d].x, acc);
              acc = dot2<BF>(((p >> 4) & dq_mask) | dq_magic, m[i][d].y, acc);
              acc = dot2<BF>(((p >> 8) & dq_mask) | dq_magic, m[i][d].z, acc);
              acc = dot2<BF>(((p >> 12) & dq_mask) | dq_magic, m[i][d].w, acc);
            }
            // a chunk past C read zeros: its scale is zero
            part[r] += f16_bits_to_f32(sc[i][r]) * (acc - base * msum);
          }
        }
      } else if constexpr (MIXED) {
#pragma unroll
        for (int i = 0; i < NCH; ++i)
#pragma unroll
          for (int d = 0; d < 4; ++d) m[i][d] = dperm_inv(m[i][d]);  // natural k order
        if (tier == 0) {  // 16-bit weights as stored: rows of I values
          const __amdgpu_buffer_rsrc_t wr =
              make_rsrc(a.w2.bf16 + row0 * a.I, (int64_t)R * a.I * 2);
#pragma unroll
          for (int i = 0; i < NCH; ++i) {
            const int c = l + 32 * i;
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float acc = 0.f;
#pragma unroll
              for (int d = 0; d < 4; ++d) {
                const uint4 wv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                    wr, c < C ? (r * a.I + c * 32 + d * 8) * 2 : OOB_OFF, 0, 0));
                acc = dot2<BF>(wv.x, m[i][d].x, acc);
                acc = dot2<BF>(wv.y, m[i][d].y, acc);
                acc = dot2<BF>(wv.z, m[i][d].z, acc);
                acc = dot2<BF>(wv.w, m[i][d].w, acc);
              }
              part[r] += acc;
            }
          }
        } else {  // INT8 rows of I bytes, fp16 scale per row
          const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w2.i8 + row0 * a.I, (int64_t)R * a.I);
          auto pair16 = [&](uint32_t wd, int b) {  // bytes b, b+1 of wd -> exact 16-bit pair
            const float lo = (float)(int8_t)(wd >> (8 * b));
            const float hi = (float)(int8_t)(wd >> (8 * b + 8));
            if constexpr (BF)
              return (__builtin_bit_cast(uint32_t, lo) >> 16) |
                     (__builtin_bit_cast(uint32_t, hi) & 0xffff0000u);
            else
              return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
          };
#pragma unroll
          for (int i = 0; i < NCH; ++i) {
            const int c = l + 32 * i;
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float acc = 0.f;
#pragma unroll
              for (int h = 0; h < 2; ++h) {  // 16 bytes: k = 16 h .. 16 h + 15
                const uint4 wv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                    wr, c < C ? r * a.I + c * 32 + h * 16 : OOB_OFF, 0, 0));
                const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
                const uint4& m0 = m[i][2 * h];
                const uint4& m1 = m[i][2 * h + 1];
                const uint32_t mm[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  acc = dot2<BF>(pair16(ww[q], 0), mm[2 * q], acc);
                  acc = dot2<BF>(pair16(ww[q], 2), mm[2 * q + 1], acc);
                }
              }
              part[r] += f16_bits_to_f32(a.w2.i8_scales[row0 + r]) * acc;
            }
          }
        }
      }
    }
    // fold each half-wave's 32 lanes: DPP sums inside 16-lane rows, then the rows
    const float w_lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), 0));
    const float w_hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), 32));
    const int sw = s0 + 2 * (threadIdx.x >> 6);  // this wave's first slot
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v = part[r];
      v += dpp_f32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
      v += dpp_f32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
      v += dpp_f32<0x124>(v);  // row_ror 4
      v += dpp_f32<0x128>(v);  // row_ror 8
      const int vi = __builtin_bit_cast(int, v);
      const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0)) +
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 16));
      const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 32)) +
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 48));
      if (lane == 0) {
        if (sw < n_slots) red[sw][r] = w_lo * lo;
        if (sw + 1 < n_slots) red[sw + 1][r] = w_hi * hi;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < a.T * R) {  // out[t, row] = sum over the token's slots, ascending
    const int t = threadIdx.x / R, r = threadIdx.x - t * R;
    float o = 0.f;
    for (int j = 0; j < a.kp; ++j) o += red[t * a.kp + j][r];
    a.out[(int64_t)t * a.H + h0 + r] = (uint16_t)to_act_bits<BF>(o);
  }
}

typedef void (*decode_kernel_t)(LayerArgs);

template <bool BF, int PH>
decode_kernel_t pick_ph(bool mixed, int path) {
  if (mixed) return path == 1 ? moe_decode_kernel<BF, PH, 1, true, 1> : moe_decode_kernel<BF, PH, 1, true, 0>;
  if (PH == 0 && path == 2) return moe_decode_kernel<BF, 0, 1, false, 2>;
  return path == 1 ? moe_decode_kernel<BF, PH, 1, false, 1> : moe_decode_kernel<BF, PH, 1, false, 0>;
}

template <bool BF, bool ID64>
decode_kernel_t pick_combine_w(int w_dtype) {
  return w_dtype == EXQ_DTYPE_F32    ? decode_combine_kernel<BF, ID64, EXQ_DTYPE_F32>
         : w_dtype == EXQ_DTYPE_BF16 ? decode_combine_kernel<BF, ID64, EXQ_DTYPE_BF16>
                                     : decode_combine_kernel<BF, ID64, EXQ_DTYPE_F16>;
}
decode_kernel_t pick_combine(bool bf, bool id64, int w_dtype) {
  if (bf) return id64 ? pick_combine_w<true, true>(w_dtype) : pick_combine_w<true, false>(w_dtype);
  return id64 ? pick_combine_w<false, true>(w_dtype) : pick_combine_w<false, false>(w_dtype);
}

// One 16-row tile per pass: units with more rows take further passes (each
// re-reads its weight slice, from L2), which measured faster at T = 32 and 64
// than kernels holding two or four tiles per pass (higher register use, lower
// occupancy; Mixtral's chunked gate/up with two tiles per pass at three waves
// per SIMD: T=32 199.1 -> 226.1 us, T=64 286.1 -> 288.2).
decode_kernel_t pick_kernel(bool bf, int ph, bool mixed, int path) {
  if (bf) return ph == 0 ? pick_ph<true, 0>(mixed, path) : pick_ph<true, 1>(mixed, path);
  return ph == 0 ? pick_ph<false, 0>(mixed, path) : pick_ph<false, 1>(mixed, path);
}

}  // namespace

// Work-groups of `kern` that fit on the device at once (CUs x per-CU
// occupancy), cached per (device, kernel, LDS bytes).
int resident_work_groups(const void* kern, int threads, size_t lds, int* out) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, size_t>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(EXQ_ERROR_HIP, "decode: hipGetDevice failed");
  const auto key = std::make_tuple(dev, kern, lds);
  {
    std::lock_guard<std::mutex> g(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) {
      *out = it->second;
      return EXQ_SUCCESS;
    }
  }
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, threads, lds) != hipSuccess)
    return set_error(EXQ_ERROR_HIP, "decode: occupancy query failed");
  const int n = cus * per > 0 ? cus * per : 1;
  std::lock_guard<std::mutex> g(mu);
  cache[key] = n;
  *out = n;
  return EXQ_SUCCESS;
}

size_t decode_plan_bytes(int64_t T, int64_t k, int64_t E, int64_t n_shared) {
  // tiles: one per active expert, plus one per further 16 rows of any expert
  const int64_t active = (T * k < E ? T * k : E) + n_shared;
  const int64_t tiles = active + (T * (k + n_shared) + 15) / 16;
  return (size_t)(kPlanHdrInts + tiles * kPlanRecInts) * 4;
}

bool decode_path_supported(int64_t T, int64_t k, int64_t Ep, int64_t n_shared, int64_t H,
                           int64_t I, int64_t group_size) {
  const int64_t gkb = group_size / 128;  // k-blocks per scale group: a power of two
  if (H % 128 || I % 128 || group_size % 128) return false;
  if (!(T >= 1 && T <= 64 && T * k <= MAX_SLOTS && Ep <= kDecodeMaxBuckets && n_shared <= 64 &&
        H / 32 <= kDecodeMaxHBlocks && H % 64 == 0 && gkb >= 1 && (gkb & (gkb - 1)) == 0))
    return false;
  // the partial rows (every split) stay below the out-of-range offset
  if ((int64_t)kDecodeMaxSplit * T * (k + n_shared) * H * 4 >= OOB_OFF) return false;
  // a register-ring unit's scales (rows x dwords of its widest k-range) fit in LDS
  auto ring_scales_fit = [&](int64_t K, int64_t rows) {
    const int64_t nkb = K / 128, span = (nkb + 3) / 4;
    const int64_t ngw = (span + gkb - 1) / gkb + 1;
    return rows * ((ngw * 2 + 2 + 3) / 4) * 4 <= RING_SCALE_BYTES;
  };
  return ring_scales_fit(H, 32) && ring_scales_fit(I, rows_b(1));
}

// decode_down_rows_kernel for nch 32-k chunks per lane (1 or 2), nontemporal
// weight loads when every weight row is read once (one token).
template <bool BF, bool MIXED>
static decode_kernel_t pick_down_rows(int nch, bool once) {
  if (nch <= 1)
    return once ? decode_down_rows_kernel<BF, MIXED, 1, true> : decode_down_rows_kernel<BF, MIXED, 1, false>;
  return once ? decode_down_rows_kernel<BF, MIXED, 2, true> : decode_down_rows_kernel<BF, MIXED, 2, false>;
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
  a.plan = d.plan;
  const bool mixed = d.tier != nullptr;
  const int nt = 1;
  a.nbA = d.I / 16;
  a.nbB = d.H / rows_b(nt);
  a.nsplit = 1;

  const int64_t max_active = (int64_t)(d.T * d.k < d.E ? d.T * d.k : d.E) + (d.Ep - d.E);
  // Tiles: at most one per active expert plus one per further 16 rows.  The
  // grid is sized for one tile per expert up to T = 16 (more tiles there
  // need repeated ids; the work-groups then stride over the extra units).
  const int64_t max_tiles = d.T <= 16 ? max_active : max_active + ((int64_t)d.T * d.kp + 15) / 16;
  const bool rows = d.T <= kRowsDownMaxT && d.kp >= 4 && d.T * d.kp <= ROWS_MAX_SLOTS && d.I <= 2048;
  const bool rows_gu = rows && !mixed && d.T <= kRowsGateUpMaxT && d.I % GU_PAIRS == 0 && d.H <= 4096;
  for (int ph = 0; ph < 2; ++ph) {
    const hipEvent_t* ev = stage_events();
    if (ph == 0 && rows_gu) {
      // few tokens: the gate/up projection by output rows
      const dim3 g0((unsigned)(d.I / GU_PAIRS), (unsigned)(d.T * d.kp));
      const int nch = (d.H / 32 + 63) / 64;  // chunks per lane
      const auto k0 = nch <= 1 ? (d.bf ? decode_gateup_rows_kernel<true, 1> : decode_gateup_rows_kernel<false, 1>)
                    : nch <= 2 ? (d.bf ? decode_gateup_rows_kernel<true, 2> : decode_gateup_rows_kernel<false, 2>)
                               : (d.bf ? decode_gateup_rows_kernel<true, 4> : decode_gateup_rows_kernel<false, 4>);
      if (ev)
        hipExtLaunchKernelGGL(k0, g0, dim3(GU_THREADS), 0, s, ev[0], ev[1], 0, a);
      else
        hipLaunchKernelGGL(k0, g0, dim3(GU_THREADS), 0, s, a);
      const int st = check_launch("decode_gateup_rows_kernel");
      if (st) return st;
      continue;
    }
    if (ph == 1 && rows) {
      // few tokens: the down projection by output rows, summed in-kernel
      const dim3 g1((unsigned)(d.H / rows_r((d.I / 32 + 31) / 32)));
      const int nch = (d.I / 32 + 31) / 32;  // chunks per lane
      const decode_kernel_t k1 =
          mixed ? (d.bf ? pick_down_rows<true, true>(nch, d.T == 1) : pick_down_rows<false, true>(nch, d.T == 1))
                : (d.bf ? pick_down_rows<true, false>(nch, d.T == 1)
                        : pick_down_rows<false, false>(nch, d.T == 1));
      if (ev)
        hipExtLaunchKernelGGL(k1, g1, dim3(256), 0, s, ev[2], ev[3], 0, a);
      else
        hipLaunchKernelGGL(k1, g1, dim3(256), 0, s, a);
      return check_launch("decode_down_rows_kernel");
    }
    // per-wave weight slices / partial tiles, then the per-expert row counts
    const size_t lds = (size_t)DW * WAVE_LDS + (((size_t)(d.Ep + 1) / 2 * 4 + 15) & ~(size_t)15) +
                       (mixed ? (size_t)d.Ep * 4 : 0);  // (+ the mixed bank's expert map)
    if (ph == 1) {
      // Few down units (large experts, few active): split each (expert, row
      // block) contraction over up to kDecodeMaxSplit work-groups, each with
      // at least four k-blocks, to fill the resident round.
      int resident = 0;
      const int st = resident_work_groups(
          reinterpret_cast<const void*>(pick_kernel(d.bf, 1, mixed, 0)), DNT, lds, &resident);
      if (st) return st;
      const int64_t u1 = max_tiles * a.nbB;
      int64_t sp = u1 > 0 ? resident / u1 : 1;
      const int64_t cap = (d.I / 128) / 4;
      if (sp > cap) sp = cap;
      if (sp > kDecodeMaxSplit) sp = kDecodeMaxSplit;
      a.nsplit = sp < 1 ? 1 : (int)sp;
      // The last unit of each column block combines it inside the down
      // kernel for small batches; from kCombineLaunchMinT tokens or
      // kCombineLaunchMinSplit k-splits on, that tail (one work-group per
      // block reading T x kp x nsplit partial rows) outlasts a separate, fully
      // parallel combine launch (measured: Qwen3 T=64 81.2 -> 73.5 µs/layer,
      // Mixtral T=1 66.7 -> 63.2; T <= 16 with few splits 0.5-1 µs better
      // in-kernel).
      a.combine = d.T < kCombineLaunchMinT && a.nsplit < kCombineLaunchMinSplit ? 1 : 0;
    }
    // INT4 slices go through LDS when every wave's k-range fits its region
    const int rs = ph == 0 ? 2 : rows_b(nt) / 16;
    const int nkb = (ph == 0 ? d.H : d.I) / 128;
    const int ns = ph == 0 ? 1 : a.nsplit;
    const int nkb_split = (nkb + ns - 1) / ns;  // the widest split
    const int ng = nkb >> a.gshift;             // the unit's whole scale rows are copied
    // the wave's k-range fits its weight region and the unit's scales its scale area
    const bool dma = (nkb_split + 3) / 4 <= WAVE_W / (rs * 1024) && rs * 16 * ng * 2 <= WAVE_S;
    // Gate/up with a longer k-range (all INT4): chunked LDS copies, when the
    // k-range's scale dwords (rows x nd, whole 256-byte DMA steps) fit the
    // scale area.
    bool chunked = false;
    if (ph == 0 && !mixed && !dma) {
      const int gkb = 1 << a.gshift, span = (nkb_split + 3) / 4;
      const int ngw = (span + gkb - 1) / gkb + 1, nd = (ngw * 2 + 2 + 3) / 4;
      chunked = ((rs * 16 * nd + 63) / 64) * 256 <= WAVE_S;
    }
    const decode_kernel_t kern = pick_kernel(d.bf, ph, mixed, dma ? 1 : (chunked ? 2 : 0));
    // (the all-INT4 LDS path keeps its slices in static arrays)
    const size_t klds = dma && !mixed ? lds - (size_t)DW * WAVE_LDS : lds;
    const int64_t units = max_tiles * (ph == 0 ? a.nbA : (int64_t)a.nbB * a.nsplit);
    int resident = 0;
    const int st0 = resident_work_groups(reinterpret_cast<const void*>(kern), DNT, klds, &resident);
    if (st0) return st0;
    const int64_t grid = units < resident ? units : resident;
    const dim3 g((unsigned)(grid > 0 ? grid : 1));
    // stage events: start / stop of exactly this kernel (the down stage ends
    // after the combine launch when there is one)
    const bool tail = ph == 1 && !a.combine;
    if (ev)
      hipExtLaunchKernelGGL(kern, g, dim3(DNT), klds, s, ev[2 * ph],
                            tail ? nullptr : ev[2 * ph + 1], 0, a);
    else
      hipLaunchKernelGGL(kern, g, dim3(DNT), klds, s, a);
    int st = check_launch(ph == 0 ? "moe_decode_kernel<gate/up>" : "moe_decode_kernel<down>");
    if (st) return st;
    if (tail) {
      const dim3 cg((unsigned)cdiv((int64_t)d.T * (d.H / 4), kCombineThreads));
      const decode_kernel_t ck = pick_combine(d.bf, d.ids_dtype == EXQ_DTYPE_I64, d.w_dtype);
      if (ev)
        hipExtLaunchKernelGGL(ck, cg, dim3(kCombineThreads), 0, s, nullptr, ev[3], 0, a);
      else
        hipLaunchKernelGGL(ck, cg, dim3(kCombineThreads), 0, s, a);
      st = check_launch("decode_combine_kernel");
      if (st) return st;
    }
  }
  return EXQ_SUCCESS;
}

}  // namespace exq
