// exq_internal.h -- declarations shared between the translation units of
// libexq_hip.so.  Not part of the C ABI.
#pragma once

#include "exq_common.h"

namespace exq {

// Tokens of one expert are processed in groups of at most this many rows
// (four 16-row MFMA tiles).
constexpr int kTokenGroup = 64;

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

// Parameters of the routing-plan kernel (one work-group).
struct RoutePlanParams {
  const void* ids;
  int ids_dtype;
  int T, k, kp, E, Ep;  // kp = k + n_shared, Ep = E + n_shared
  int n;                // T * kp
  const int8_t* tier;   // [Ep] or null (all INT4)
  int* hdr;             // hdr[0] = number of token groups
  int* ends;            // [Ep + 1]
  int* sorted;          // [n] slot ids in expert-sorted order
  TgEntry* tg;          // [tg_cap]
  int tg_cap;
  int* counters;        // combine arrival counters, zeroed here
  int n_counters;
  int64_t* sort_order_out;  // optional [T*k]
  int32_t* ends_out;        // optional [E+1]
  void* out;                // zero-filled when no row is routed
  int64_t out_bytes;
};

int launch_route_plan(const RoutePlanParams& p, hipStream_t stream);

// Token groups from user-provided expert boundaries (sorted-row GEMM API).
int launch_tg_from_ends(const int32_t* ends, int E, const int32_t* expert_mask, int tier,
                        int* hdr, TgEntry* tg, int tg_cap, hipStream_t stream);

// One-launch decode layer (decode.hip): routing, gate/up + SiLU, down and the
// combine in a single persistent kernel.  `sync` points at the zero-filled
// counter region (kDecodeSyncBytes at the start of the fused workspace).
constexpr int kDecodeMaxBuckets = 1024;   // routed + shared experts
constexpr int kDecodeMaxHBlocks = 512;    // H / 64
constexpr size_t kDecodeSyncBytes = (size_t)(kDecodeMaxBuckets + kDecodeMaxHBlocks + 2) * 128;

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
  float* part;             // [T * kp, H]
  uint16_t* out;           // [T, H]
  int* sync;
  bool bf;
};

bool decode_path_supported(int64_t T, int64_t k, int64_t Ep, int64_t n_shared, int64_t H,
                           int64_t group_size);
int launch_decode_layer(const DecodeLaunch& d, hipStream_t s);

// The four stage events installed with exq_set_stage_events for the current
// call on this thread, or nullptr.
const hipEvent_t* stage_events();

}  // namespace exq
