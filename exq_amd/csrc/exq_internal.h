// exq_internal.h -- declarations shared between the translation units of
// libexq_hip.so.  Not part of the C ABI.
#pragma once

#include "exq_common.h"

namespace exq {

// Tokens of one expert are processed in groups of at most this many rows:
// four 16-row MFMA tiles on the grouped kernel and on the 64 x 256 INT4 tiles
// of the prefill kernels, eight on the 128 x 128 tiles.
constexpr int kTokenGroup = 64;
constexpr int kTokenGroupI4 = 128;
// On the 64 x 256 INT4 prefill tiles, an INT4 expert with at least this many
// routed rows takes 128-row token groups on the 128 x 256 scaled-operand tiles.
constexpr int kI4BigMinRows = 384;

// One work item of the grouped kernels: rows [pos0, pos0 + cnt) of the
// expert-sorted order, all routed to expert `e` whose precision tier is
// `tier` (0 BF16, 1 INT8, 2 INT4).
struct TgEntry {
  int e;
  int pos0;
  int cnt;
  int tier;
};

// Upper bound on the number of token groups for n routed rows over nb experts.
inline int64_t tg_capacity(int64_t n_rows, int64_t n_buckets) {
  int64_t a = n_rows < n_buckets ? n_rows : n_buckets;
  return a + cdiv(n_rows, kTokenGroup) + 1;
}

// Grouped-GEMM modes: gate/up + SiLU into `mid`, plain C = A x W^T, down
// projection into fp32 partial rows per slot.
enum Mode { MODE_GATEUP = 0, MODE_PLAIN = 1, MODE_DOWN = 2 };

// Weights of one projection (w13 or w2) for every precision tier.
struct Bank {
  const int8_t* tier;     // per-expert tier or null (all INT4)
  const int32_t* index;   // per-expert row in the tier bank or null (identity)
  const uint16_t* bf16;   // [nb, rows, K] activation dtype
  const int8_t* i8;       // [n8, rows, K]
  const uint16_t* i8_scales;  // [n8, rows]
  const uint8_t* i4;      // [n4, rows, K/2]
  const uint16_t* i4_scales;  // [n4, rows, K/g]
};

struct GemmArgs {
  const int* hdr;          // [0] token groups, [1] first INT4 group, [2] first INT8 group,
                           // [3] first INT4 group of the small-group experts
  const TgEntry* tg;
  int n_blocks;            // row blocks per token group
  const uint16_t* x;       // activations (f16/bf16 bits)
  int64_t x_stride;        // elements per activation row
  const int* row_slot;     // expert-sorted position -> slot (GATEUP input, DOWN output)
  int slot_div;            // slots per token (kp)
  int K;                   // contraction length, multiple of 128
  Bank w;
  int n_rows;              // weight rows per expert
  int inter;               // I: offset of the up rows (GATEUP)
  int group_size;          // INT4 group size, multiple of 128
  void* out;               // GATEUP mid [n, I] act | PLAIN C [rows, N] act | DOWN partial [n, H] f32
  int64_t out_stride;
  int H;
  int skip_i4;             // INT4 token groups belong to the tiled kernel: skip them
  int skip_bf;             // BF16 token groups belong to the tiled kernel: skip them
};

// Tiled prefill GEMMs (prefill.hip): work-group tile = 128 expert-sorted rows
// x 128 weight rows over the token groups of one tier (cnt <= kTokenGroupI4):
// INT4 groups are entries [hdr[1], hdr[0]) of the list, BF16 groups [0,
// hdr[2]).  The INT4 kernel needs the per-row group sums of its activations,
// scaled by the nibble base, from launch_group_rowsum (rs [K / 128][rs_rows];
// GATEUP rows are tokens, DOWN / PLAIN rows are expert-sorted positions).
bool tile_gemm_applies(int tier, int mode, int n_rows, int inter, int K, int group_size);
// The INT4 tiles can be 64 expert-sorted rows x 256 weight rows instead (token
// groups of kTokenGroup rows): GATEUP needs I % 128 == 0, DOWN / PLAIN rows % 256.
bool tile_gemm_wide_applies(int mode, int n_rows, int inter);
// INT4 tile shapes: 128 x 128 and 64 x 256 (per-group accumulators, base
// corrections from launch_group_rowsum), and 128 x 256 with scaled weight
// operands (token groups of kTokenGroupI4 rows, same row conditions as 64 x
// 256; needs no row sums).
enum TileShape { TILE_128x128 = 0, TILE_64x256 = 1, TILE_PS_128x256 = 2 };
int64_t tile_rowsum_floats(int64_t rows, int64_t K);
int launch_group_rowsum(bool bf, const uint16_t* x, int64_t stride, int64_t rows, int K, int gs,
                        float* out, hipStream_t s);
// The same sums for the expert-sorted rows of the token groups [hdr[3],
// hdr[0]) only (the rows the 64 x 256 and 128 x 128 INT4 tiles read in the
// down projection); cap bounds that group count, groups hold <= 128 rows.
int launch_group_rowsum_tg(bool bf, const uint16_t* x, int64_t stride, int K, const int* hdr,
                           const TgEntry* tg, int64_t cap, int64_t rs_rows, float* out,
                           hipStream_t s);
int launch_tile_gemm(int tier, int mode, bool bf, const GemmArgs& a, const float* rs,
                     int64_t rs_rows, int64_t x_bytes, int64_t tg_cap, hipStream_t s,
                     int shape = TILE_128x128);
// The tiles of one projection in one launch (tile_mix_kernel): 128 x 256
// scaled-operand INT4 tiles over token groups [hdr[1], hdr[3]), 64 x 256 INT4
// tiles over [hdr[3], hdr[0]) (row sums from launch_group_rowsum), then BF16
// tiles over [0, hdr[2]).  cap_* bound each range's token groups (0: the range
// is empty); the grid is sized from them and each range's real size is read
// on the device.
int launch_tile_mix(int mode, bool bf, const GemmArgs& a, const float* rs, int64_t rs_rows,
                    int64_t x_bytes, int64_t cap_ps, int64_t cap_64, int64_t cap_bf,
                    hipStream_t s);

// INT4 grouped GEMMs for the shapes outside the tiled / grouped kernels
// (general.hip): K % 32 == 0, a group size that is a multiple of 32 dividing
// K, any number of weight rows.  Token groups [hdr[1], hdr[0]) (<= 64 rows),
// n_blocks = ceil(output columns / 16).
bool general_shape(int64_t K, int64_t group_size);
int launch_general_gemm(int mode, bool bf, const GemmArgs& a, int64_t tg_cap, hipStream_t s);

// Parameters of the routing-plan kernel (one work-group).
struct RoutePlanParams {
  const void* ids;
  int ids_dtype;
  int T, k, kp, E, Ep;  // kp = k + n_shared, Ep = E + n_shared
  int n;                // T * kp
  const int8_t* tier;   // [Ep] or null (all INT4)
  int* hdr;             // [0] token groups, [1] first INT4 group, [2] first INT8 group,
                        // [3] first INT4 group of an expert below i4_big_rows
  int* ends;            // [Ep + 1]
  int* sorted;          // [n] slot ids in expert-sorted order
  TgEntry* tg;          // [tg_cap]
  int tg_cap;
  int i4_group;         // rows per INT4 token group (kTokenGroup or kTokenGroupI4)
  int bf_group;         // rows per BF16 token group (kTokenGroup or kTokenGroupI4)
  // INT4 experts with at least i4_big_rows routed rows (none when 0) take
  // groups of i4_big_group rows and are listed before the other INT4 experts;
  // hdr[3] = the first group of those others (hdr[0] when there are none)
  int i4_big_rows;
  int i4_big_group;
  int* counters;        // combine arrival counters, zeroed here
  int n_counters;
  int64_t* sort_order_out;  // optional [T*k]
  int32_t* ends_out;        // optional [E+1]
  void* out;                // zero-filled when no row is routed
  int64_t out_bytes;
  int* blk_cnt;             // [route_plan_blocks(n) * Ep] scratch, or null (one block)
};

// Batches above this many slots are planned by several work-groups, which
// need route_plan_blocks(n) * Ep ints of scratch (blk_cnt).
constexpr int kRoutePlanOneBlock = 2048;
int64_t route_plan_blocks(int64_t n);
int launch_route_plan(const RoutePlanParams& p, hipStream_t stream);

// Token groups from user-provided expert boundaries (sorted-row GEMM API).
int launch_tg_from_ends(const int32_t* ends, int E, const int32_t* expert_mask, int tier,
                        int group, int* hdr, TgEntry* tg, int tg_cap, hipStream_t stream);

// Decode layer (decode.hip, T <= 64): a gate/up + SiLU kernel and a down
// kernel that route for themselves, the down kernel combining in-kernel or
// through a third, combine launch.  `sync` points at the combine counters
// (kDecodeSyncBytes at the start of the fused workspace); the gate/up kernel
// clears them, so the region needs no zero fill.
constexpr int kDecodeMaxBuckets = 1024;   // routed + shared experts
constexpr int kDecodeMaxHBlocks = 512;    // H / 64
constexpr size_t kDecodeSyncBytes = (size_t)(kDecodeMaxBuckets + kDecodeMaxHBlocks + 2) * 128;
// The down kernel may split each contraction over this many work-groups; the
// fused workspace holds one fp32 partial set per split.
constexpr int kDecodeMaxSplit = 8;

struct DecodeLaunch {
  const void* ids;
  int ids_dtype;
  const void* topk_w;
  int w_dtype;
  int T, k, kp, E, Ep;
  const uint16_t* x;
  const uint16_t* w13_bf16;
  const int8_t* w13_i8;
  const uint16_t* w13_i8_scales;
  const uint8_t* w13_i4;
  const uint16_t* w13_i4_scales;
  const uint16_t* w2_bf16;
  const int8_t* w2_i8;
  const uint16_t* w2_i8_scales;
  const uint8_t* w2_i4;
  const uint16_t* w2_i4_scales;
  const int8_t* tier;      // [Ep] or null (all INT4)
  const int32_t* index;    // [Ep] or null
  int H, I, group_size;
  uint16_t* mid;           // [T * kp, I]
  float* part;             // [kDecodeMaxSplit][T * kp, H]
  uint16_t* out;           // [T, H]
  int* sync;
  int* plan;               // the down kernel's per-tile records (decode_plan_bytes)
  bool bf;
};

// Bytes of the decode plan: a 128-byte header line, then one 128-byte record
// per 16-row tile (at most one per active expert plus one per further 16
// routed rows).
size_t decode_plan_bytes(int64_t T, int64_t k, int64_t E, int64_t n_shared);

bool decode_path_supported(int64_t T, int64_t k, int64_t Ep, int64_t n_shared, int64_t H,
                           int64_t I, int64_t group_size);
int launch_decode_layer(const DecodeLaunch& d, hipStream_t s);

// The four stage events installed with exq_set_stage_events for the current
// call on this thread, or nullptr.
const hipEvent_t* stage_events();

}  // namespace exq
