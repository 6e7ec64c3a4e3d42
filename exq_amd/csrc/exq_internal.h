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

// Self-routing decode kernels (decode.hip).  mode 0: gate/up + SiLU into mid
// rows indexed by slot t*kp + j; mode 1: down projection into fp32 partial
// rows indexed the same way.
bool decode_path_supported(int64_t T, int64_t k, int64_t Ep, int64_t n_shared,
                           int64_t group_size);
int launch_decode(bool bf, int mode, const void* ids, int ids_dtype, int T, int k, int kp,
                  int E, int Ep, const uint16_t* x, int64_t x_stride, int K,
                  const int8_t* tier, const int32_t* index, const uint16_t* bf16,
                  const int8_t* i8, const uint16_t* i8_scales, const uint8_t* i4,
                  const uint16_t* i4_scales, int n_rows, int inter, int group_size, void* out,
                  int64_t out_stride, int n_blocks, hipStream_t s);

}  // namespace exq
