// routing.hip -- routing preparation.
//
// Decode batches route at most a few thousand slots, so a single 1024-thread
// work-group does the whole job out of LDS: an LDS-atomic histogram, a
// wave-shuffle block scan, and a stable scatter whose rank comes from
// per-bucket slot bitmasks (popcount of the lower bits), so the order inside
// a bucket is deterministic and ascending -- the canonical order of the
// reference's stable argsort (exq/kernels/moe_grouped_gemm.py:156-157).
// Larger calls run over many work-groups: the fused layer's plan in three
// launches through its workspace, the standalone entry points in one launch
// that needs no scratch (each block recounts every item's bucket).  Nothing
// here uses global atomics, hipCUB or temporary allocations.
#include <stdarg.h>
#include <stdio.h>

#include "exq_internal.h"

namespace exq {
namespace {

constexpr int RT = 1024;            // threads of the routing work-group
constexpr int RT_WAVES = RT / 64;
constexpr int MAX_BUCKETS = 1024;   // experts (+ shared / shifted bucket)
constexpr int MASK_WORDS = 16384;   // 64 KiB of chunk bitmasks

struct RouteLds {
  int cnt[MAX_BUCKETS];
  int start[MAX_BUCKETS + 1];
  int run[MAX_BUCKETS];
  int wsum[RT_WAVES];
  uint32_t masks[MASK_WORDS];
};

// Exclusive scan of one value per thread over the work-group.
__device__ int block_excl_scan(int v, int* wsum, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < RT_WAVES ? wsum[lane] : 0;
#pragma unroll
    for (int d = 1; d < RT_WAVES; d <<= 1) {
      int y = __shfl_up(w, d, 64);
      if (lane >= d) w += y;
    }
    if (lane < RT_WAVES) wsum[lane] = w;
  }
  __syncthreads();
  const int prefix = wave > 0 ? wsum[wave - 1] : 0;
  *total = wsum[RT_WAVES - 1];
  __syncthreads();
  return prefix + x - v;
}

template <typename KeyFn>
__device__ void histogram(int n, int nb, KeyFn key, int* cnt) {
  for (int b = threadIdx.x; b < nb; b += RT) cnt[b] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += RT) {
    int b = key(i);
    if (b >= 0) atomicAdd(&cnt[b], 1);
  }
  __syncthreads();
}

// Stable scatter: element i with bucket b = key(i) >= 0 is emitted at
// run[b] + (number of earlier elements in bucket b).  run[] advances.
template <typename KeyFn, typename EmitFn>
__device__ void stable_scatter(int n, int nb, KeyFn key, int* run, uint32_t* masks,
                               EmitFn emit) {
  const int tid = threadIdx.x;
  int wpb = MASK_WORDS / (nb > 0 ? nb : 1);
  if (wpb > RT / 32) wpb = RT / 32;
  const int chunk = wpb * 32;
  for (int base = 0; base < n; base += chunk) {
    for (int w = tid; w < nb * wpb; w += RT) masks[w] = 0u;
    __syncthreads();
    const int i = base + tid;
    const int b = (tid < chunk && i < n) ? key(i) : -1;
    if (b >= 0) atomicOr(&masks[b * wpb + (tid >> 5)], 1u << (tid & 31));
    __syncthreads();
    if (b >= 0) {
      const uint32_t* m = masks + b * wpb;
      int r = __popc(m[tid >> 5] & ((1u << (tid & 31)) - 1u));
      for (int w = 0; w < (tid >> 5); ++w) r += __popc(m[w]);
      emit(i, b, run[b] + r);
    }
    __syncthreads();
    if (tid < nb) {
      int c = 0;
      for (int w = 0; w < wpb; ++w) c += __popc(masks[tid * wpb + w]);
      run[tid] += c;
    }
    __syncthreads();
  }
}

// ---- exq_dispatch -----------------------------------------------------------
__global__ void __launch_bounds__(RT) dispatch_kernel(const void* ids, int ids_dtype, int n,
                                                      int E, int64_t* sort_order,
                                                      int64_t* sorted_ids, int32_t* ends) {
  __shared__ RouteLds s;
  // Ids outside [0, E) go to a trailing bucket E so sort_order stays a permutation.
  auto key = [&](int i) -> int {
    int64_t v = load_index(ids, ids_dtype, i);
    return (v >= 0 && v < E) ? (int)v : E;
  };
  const int nb = E + 1;  // <= RT, so one scan pass covers every bucket
  histogram(n, nb, key, s.cnt);
  const int b = threadIdx.x;
  int t;
  int ex = block_excl_scan(b < nb ? s.cnt[b] : 0, s.wsum, &t);
  if (b < nb) {
    s.start[b] = ex;
    s.run[b] = ex;
  }
  if (threadIdx.x == 0) s.start[nb] = t;
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += RT) ends[e] = s.start[e];
  stable_scatter(n, nb, key, s.run, s.masks, [&](int i, int b, int pos) {
    sort_order[pos] = i;
    sorted_ids[pos] = load_index(ids, ids_dtype, i);
  });
}

// ---- exq_build_ends_from_slots ---------------------------------------------
__global__ void __launch_bounds__(RT) build_ends_kernel(const int32_t* sid, int em,
                                                        const int32_t* fr, int n_active, int E,
                                                        int32_t* ends, int64_t* sort_order) {
  __shared__ RouteLds s;
  auto key = [&](int i) -> int {
    int slot = sid[i];
    if (slot < 0 || slot >= n_active) return -1;
    int e = fr[slot];
    return (e >= 0 && e < E) ? e : -1;
  };
  histogram(em, E, key, s.cnt);
  int b = threadIdx.x;
  int t;
  int ex = block_excl_scan(b < E ? s.cnt[b] : 0, s.wsum, &t);
  if (b < E) {
    s.start[b] = ex;
    s.run[b] = ex;
  }
  if (threadIdx.x == 0) s.start[E] = t;
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += RT) ends[e] = s.start[e];
  // A slot listed twice would overflow sort_order; such entries are dropped.
  stable_scatter(em, E, key, s.run, s.masks, [&](int i, int, int pos) {
    if (pos < n_active) sort_order[pos] = sid[i];
  });
}

// ---- exq_moe_align_block_size ----------------------------------------------
__global__ void __launch_bounds__(RT) align_kernel(const void* ids, int ids_dtype, int numel,
                                                   int nb, int B, int32_t* sorted_ids, int cap,
                                                   int32_t* expert_ids, int cap_blocks,
                                                   int32_t* ntpp, int32_t* cumsum, int pad) {
  __shared__ RouteLds s;
  auto key = [&](int i) -> int {
    int64_t v = load_index(ids, ids_dtype, i) + 1;  // bucket 0 holds id == -1
    return (v >= 0 && v < nb) ? (int)v : -1;
  };
  histogram(numel, nb, key, s.cnt);
  const int b = threadIdx.x;
  const int padded = b < nb ? ((s.cnt[b] + B - 1) / B) * B : 0;
  int t;
  int ex = block_excl_scan(padded, s.wsum, &t);
  if (b < nb) {
    s.start[b] = ex;
    s.run[b] = ex;
  }
  if (threadIdx.x == 0) s.start[nb] = t;
  __syncthreads();
  for (int i = threadIdx.x; i <= nb; i += RT) cumsum[i] = s.start[i];
  if (threadIdx.x == 0) ntpp[0] = t;
  if (pad) {
    for (int i = threadIdx.x; i < cap; i += RT) sorted_ids[i] = numel;
  }
  // Block -> bucket by binary search over the padded starts.
  for (int blk = threadIdx.x; blk < cap_blocks; blk += RT) {
    const int p = blk * B;
    int val = -1;
    if (p < t) {
      int lo = 0, hi = nb - 1;
      while (lo < hi) {  // last bucket with start <= p
        int mid = (lo + hi + 1) >> 1;
        if (s.start[mid] <= p) lo = mid; else hi = mid - 1;
      }
      val = lo - 1;
    }
    expert_ids[blk] = val;
  }
  __syncthreads();  // padding fill must land before the scatter overwrites
  stable_scatter(numel, nb, key, s.run, s.masks,
                 [&](int i, int, int pos) { sorted_ids[pos] = i; });
}

// ---- standalone entry points above one work-group ---------------------------
// A device-wide stable counting sort that needs no scratch memory: block b owns
// items [lo, hi) and counts the buckets of ALL n items itself, split into the
// items before lo and all items.  An exclusive scan of the totals gives every
// bucket's start; start + (items of the bucket before lo) is where block b's
// first item of that bucket goes, and a stable scatter of its own items
// follows.  No block waits for another and nothing is written outside the
// outputs; the recount costs each block n / RT loads per thread, so the grid
// is capped at kWideMaxGrid blocks (larger ranges per block past that).
// Results are identical to the one-work-group kernels (the same stable
// ascending order inside a bucket).
constexpr int kWideMaxBuckets = 4096;  // experts + the trailing or shifted bucket
constexpr int kWideMaxGrid = 128;
constexpr int kWideVPT = kWideMaxBuckets / RT;  // buckets per thread in the scan

struct WideLds {
  int tot[kWideMaxBuckets];        // bucket totals over all items
  int run[kWideMaxBuckets];        // items before lo, then this block's cursors
  int start[kWideMaxBuckets + 1];  // exclusive starts, start[nb] = total
  int wsum[RT_WAVES];
  uint32_t masks[MASK_WORDS];
};

// tot[] (all n items) and before[] (the items before lo) per bucket; each
// item costs one LDS atomic (the items from lo on count into tot, which then
// adds before).  Sixteen keys per thread are loaded before their atomics, so
// up to 16,384 items take one memory round trip.  *own receives the key of
// item lo + threadIdx.x when lo is a multiple of RT (-1 past n), for a
// scatter of [lo, lo + RT) that then needs no second load.
template <typename KeyFn>
__device__ void wide_count(int n, int lo, int nb, KeyFn key, int* tot, int* before,
                           int* own = nullptr) {
  for (int b = threadIdx.x; b < nb; b += RT) {
    tot[b] = 0;
    before[b] = 0;
  }
  __syncthreads();
  constexpr int U = 16;
  int mine = -1;
  for (int64_t i0 = 0; i0 < n; i0 += (int64_t)RT * U) {
    int kv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u * RT + (int)threadIdx.x;
      kv[u] = i < n ? key((int)i) : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i0u = i0 + u * RT;
      if (i0u == lo) mine = kv[u];
      if (kv[u] >= 0) atomicAdd(i0u + (int)threadIdx.x < lo ? &before[kv[u]] : &tot[kv[u]], 1);
    }
  }
  if (own) *own = mine;
  __syncthreads();
  for (int b = threadIdx.x; b < nb; b += RT) tot[b] += before[b];
  __syncthreads();
}

// start[b] = sum of val(b') for b' < b (b < nb), start[nb] = total; thread t
// takes buckets t*kWideVPT .. (consecutive), so the order is the bucket order.
template <typename ValFn>
__device__ int wide_excl_scan(int nb, ValFn val, int* start, int* wsum) {
  const int b0 = (int)threadIdx.x * kWideVPT;
  int loc[kWideVPT];
  int sum = 0;
#pragma unroll
  for (int j = 0; j < kWideVPT; ++j) {
    loc[j] = b0 + j < nb ? val(b0 + j) : 0;
    sum += loc[j];
  }
  int total;
  int ex = block_excl_scan(sum, wsum, &total);
#pragma unroll
  for (int j = 0; j < kWideVPT; ++j) {
    if (b0 + j < nb) start[b0 + j] = ex;
    ex += loc[j];
  }
  if (threadIdx.x == 0) start[nb] = total;
  __syncthreads();
  return total;
}

// Stable scatter of items [lo, hi): item i of bucket b goes to run[b] + (its
// rank among the range's earlier items of bucket b), in chunks whose per-bucket
// slot bitmasks fit the mask area; run[] advances after each chunk.
template <typename KeyFn, typename EmitFn>
__device__ void wide_scatter(int lo, int hi, int nb, KeyFn key, int* run, uint32_t* masks,
                             EmitFn emit) {
  const int tid = threadIdx.x;
  int wpb = MASK_WORDS / nb;
  if (wpb > RT / 32) wpb = RT / 32;
  const int chunk = wpb * 32;
  for (int base = lo; base < hi; base += chunk) {
    for (int w = tid; w < nb * wpb; w += RT) masks[w] = 0u;
    __syncthreads();
    const int i = base + tid;
    const int b = (tid < chunk && i < hi) ? key(i) : -1;
    if (b >= 0) atomicOr(&masks[b * wpb + (tid >> 5)], 1u << (tid & 31));
    __syncthreads();
    if (b >= 0) {
      const uint32_t* m = masks + b * wpb;
      int r = __popc(m[tid >> 5] & ((1u << (tid & 31)) - 1u));
      for (int w = 0; w < (tid >> 5); ++w) r += __popc(m[w]);
      emit(i, b, run[b] + r);
    }
    __syncthreads();
    for (int bb = tid; bb < nb; bb += RT) {
      int c = 0;
      for (int w = 0; w < wpb; ++w) c += __popc(masks[bb * wpb + w]);
      run[bb] += c;
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(RT) wide_dispatch_kernel(const void* ids, int ids_dtype, int n,
                                                           int E, int per, int64_t* sort_order,
                                                           int64_t* sorted_ids, int32_t* ends) {
  __shared__ WideLds s;
  auto key = [&](int i) -> int {
    const int64_t v = load_index(ids, ids_dtype, i);
    return (v >= 0 && v < E) ? (int)v : E;  // ids outside [0, E): trailing bucket E
  };
  const int nb = E + 1;
  const int lo = blockIdx.x * per, hi = min(n, lo + per);
  wide_count(n, lo, nb, key, s.tot, s.run);
  wide_excl_scan(nb, [&](int b) { return s.tot[b]; }, s.start, s.wsum);
  for (int b = threadIdx.x; b < nb; b += RT) s.run[b] += s.start[b];
  if (blockIdx.x == 0)
    for (int e = threadIdx.x; e <= E; e += RT) ends[e] = s.start[e];
  __syncthreads();
  wide_scatter(lo, hi, nb, key, s.run, s.masks, [&](int i, int, int pos) {
    sort_order[pos] = i;
    sorted_ids[pos] = load_index(ids, ids_dtype, i);
  });
}

__global__ void __launch_bounds__(RT) wide_build_ends_kernel(const int32_t* sid, int em,
                                                             const int32_t* fr, int n_active,
                                                             int E, int per, int32_t* ends,
                                                             int64_t* sort_order) {
  __shared__ WideLds s;
  auto key = [&](int i) -> int {
    const int slot = sid[i];
    if (slot < 0 || slot >= n_active) return -1;
    const int e = fr[slot];
    return (e >= 0 && e < E) ? e : -1;
  };
  const int lo = blockIdx.x * per, hi = min(em, lo + per);
  wide_count(em, lo, E, key, s.tot, s.run);
  wide_excl_scan(E, [&](int b) { return s.tot[b]; }, s.start, s.wsum);
  for (int b = threadIdx.x; b < E; b += RT) s.run[b] += s.start[b];
  if (blockIdx.x == 0)
    for (int e = threadIdx.x; e <= E; e += RT) ends[e] = s.start[e];
  __syncthreads();
  // a slot listed twice would overflow sort_order; such entries are dropped
  wide_scatter(lo, hi, E, key, s.run, s.masks, [&](int i, int, int pos) {
    if (pos < n_active) sort_order[pos] = sid[i];
  });
}

__global__ void __launch_bounds__(RT) wide_align_kernel(const void* ids, int ids_dtype, int numel,
                                                        int nb, int B, int per,
                                                        int32_t* sorted_ids, int cap,
                                                        int32_t* expert_ids, int cap_blocks,
                                                        int32_t* ntpp, int32_t* cumsum, int pad) {
  __shared__ WideLds s;
  auto key = [&](int i) -> int {
    const int64_t v = load_index(ids, ids_dtype, i) + 1;  // bucket 0 holds id == -1
    return (v >= 0 && v < nb) ? (int)v : -1;
  };
  const int lo = blockIdx.x * per, hi = min(numel, lo + per);
  wide_count(numel, lo, nb, key, s.tot, s.run);
  const int t = wide_excl_scan(nb, [&](int b) { return ((s.tot[b] + B - 1) / B) * B; }, s.start,
                               s.wsum);
  for (int b = threadIdx.x; b < nb; b += RT) s.run[b] += s.start[b];
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i <= nb; i += RT) cumsum[i] = s.start[i];
    if (threadIdx.x == 0) ntpp[0] = t;
  }
  // bucket of padded position p < t: the last bucket whose start is <= p
  auto bucket_of = [&](int p) {
    int a = 0, z = nb - 1;
    while (a < z) {
      const int mid = (a + z + 1) >> 1;
      if (s.start[mid] <= p) a = mid; else z = mid - 1;
    }
    return a;
  };
  const int gtid = blockIdx.x * RT + threadIdx.x, gstride = gridDim.x * RT;
  for (int blk = gtid; blk < cap_blocks; blk += gstride)
    expert_ids[blk] = blk * B < t ? bucket_of(blk * B) - 1 : -1;
  // padding entries only (a bucket's tail past its count, and everything past
  // t), so no block writes where another block's scatter does
  if (pad) {
    for (int p = gtid; p < cap; p += gstride) {
      bool fill = p >= t;
      if (!fill) {
        const int b = bucket_of(p);
        fill = p - s.start[b] >= s.tot[b];
      }
      if (fill) sorted_ids[p] = numel;
    }
  }
  __syncthreads();
  wide_scatter(lo, hi, nb, key, s.run, s.masks, [&](int i, int, int pos) { sorted_ids[pos] = i; });
}

// Blocks and items per block of the wide kernels for n items.
__host__ __forceinline__ void wide_grid(int64_t n, int* grid, int* per) {
  int64_t g = (n + RT - 1) / RT;
  if (g > kWideMaxGrid) g = kWideMaxGrid;
  if (g < 1) g = 1;
  *grid = (int)g;
  *per = (int)((n + g - 1) / g);
}

// ---- fused-path routing plan -----------------------------------------------
// Bucket of slot t*kp + j: routed id (dropped: -1) for j < k, shared expert
// E + (j - k) otherwise.
__device__ __forceinline__ int plan_key(const RoutePlanParams& p, int slot) {
  // slot / kp from a float reciprocal and one correction step: slot < 2^24
  // (validated), so the estimate is off by at most one
  int t = (int)((float)slot * (1.0f / (float)p.kp));
  int j = slot - t * p.kp;
  if (j >= p.kp) {
    ++t;
    j -= p.kp;
  } else if (j < 0) {
    --t;
    j += p.kp;
  }
  if (j < p.k) {
    int64_t v = load_index(p.ids, p.ids_dtype, (int64_t)t * p.k + j);
    return (v >= 0 && v < p.E) ? (int)v : -1;
  }
  return p.E + (j - p.k);
}

// Flat routed slot t*k + j of plan slot t*kp + j (j < k): the index space of
// sort_order_out, which lists the routed experts' slots only.
__device__ __forceinline__ int64_t routed_slot(const RoutePlanParams& p, int slot) {
  const int t = slot / p.kp;
  return (int64_t)t * p.k + (slot - t * p.kp);
}

// Everything after the sort that needs only the bucket counts s.cnt and
// starts s.start (one work-group): boundaries, token groups (tier order BF16,
// INT8, INT4, so long work items start early), header, combine counters, and
// the zero output of a layer with no routed row.
__device__ void plan_tail(const RoutePlanParams& p, RouteLds& s) {
  const int nb = p.Ep;
  const int b = threadIdx.x;
  for (int e = threadIdx.x; e <= nb; e += RT) p.ends[e] = s.start[e];
  if (p.ends_out) {
    for (int e = threadIdx.x; e <= p.E; e += RT) p.ends_out[e] = s.start[e];
  }
  const int c = b < nb ? s.cnt[b] : 0;
  const int my_tier = (b < nb) ? (p.tier ? (int)p.tier[b] : 2) : -1;
  // list class of the bucket's groups: 0 BF16, 1 INT8, 2 INT4 experts with at
  // least i4_big_rows rows, 3 the other INT4 experts
  const int my_cls =
      my_tier == 2 ? (p.i4_big_rows > 0 && c >= p.i4_big_rows ? 2 : 3) : my_tier;
  const int gsz = my_cls == 2   ? p.i4_big_group
                  : my_cls == 3 ? p.i4_group
                  : my_cls == 0 ? p.bf_group
                                : kTokenGroup;
  const int ng = (c + gsz - 1) / gsz;
  int base = 0, first_i4 = 0, first_i8 = 0, first_i4s = 0;
  for (int cl = (p.tier ? 0 : 2); cl <= 3; ++cl) {
    if (cl == 1) first_i8 = base;
    if (cl == 2) first_i4 = base;
    if (cl == 3) first_i4s = base;
    if (cl == 2 && p.i4_big_rows <= 0) continue;  // no big INT4 experts (uniform)
    int tot;
    int off = block_excl_scan(my_cls == cl ? ng : 0, s.wsum, &tot);
    if (my_cls == cl) {
      for (int g = 0; g < ng; ++g) {
        const int slot = base + off + g;
        if (slot < p.tg_cap) {
          TgEntry te;
          te.e = b;
          te.pos0 = s.start[b] + g * gsz;
          te.cnt = min(gsz, c - g * gsz);
          te.tier = my_tier;
          p.tg[slot] = te;
        }
      }
    }
    base += tot;
  }
  if (threadIdx.x == 0) {
    p.hdr[0] = base < p.tg_cap ? base : p.tg_cap;
    p.hdr[1] = first_i4 < p.tg_cap ? first_i4 : p.tg_cap;
    p.hdr[2] = first_i8 < p.tg_cap ? first_i8 : p.tg_cap;
    p.hdr[3] = first_i4s < p.tg_cap ? first_i4s : p.tg_cap;
  }
  for (int i = threadIdx.x; i < p.n_counters; i += RT) p.counters[i] = 0;
  if (base == 0 && p.out) {
    uint32_t* o = reinterpret_cast<uint32_t*>(p.out);
    for (int64_t i = threadIdx.x; i < p.out_bytes / 4; i += RT) o[i] = 0u;
  }
}

// One work-group: histogram, scan, stable scatter, tail.
__global__ void __launch_bounds__(RT) route_plan_kernel(RoutePlanParams p) {
  __shared__ RouteLds s;
  auto key = [&](int slot) { return plan_key(p, slot); };
  const int nb = p.Ep;
  histogram(p.n, nb, key, s.cnt);
  const int b = threadIdx.x;
  int t;
  int ex = block_excl_scan(b < nb ? s.cnt[b] : 0, s.wsum, &t);
  if (b < nb) {
    s.start[b] = ex;
    s.run[b] = ex;
  }
  if (threadIdx.x == 0) s.start[nb] = t;
  __syncthreads();
  stable_scatter(p.n, nb, key, s.run, s.masks, [&](int i, int b, int pos) {
    p.sorted[pos] = i;
    if (p.sort_order_out && b < p.E) p.sort_order_out[pos] = routed_slot(p, i);
  });
  plan_tail(p, s);
}

// Large batches up to kRecountMaxSlots: the same plan in one launch with no
// scratch, as the standalone sort does it -- every block counts all n slots'
// buckets (split into the slots before its range and all), scans, and stably
// scatters its own range; one more block (the last) only counts and runs the
// tail from the totals, off the scatter blocks' path.
constexpr int kRecountMaxSlots = 65536;

__global__ void __launch_bounds__(RT) route_plan_recount_kernel(RoutePlanParams p, int per) {
  __shared__ RouteLds s;
  auto key = [&](int slot) { return plan_key(p, slot); };
  const int nb = p.Ep;
  const bool tail = blockIdx.x == gridDim.x - 1;
  const int lo = tail ? p.n : blockIdx.x * per, hi = min(p.n, lo + per);
  int own;  // key of slot lo + threadIdx.x (per == RT: lo is a multiple of RT)
  wide_count(p.n, lo, nb, key, s.cnt, s.run, &own);
  const int b = threadIdx.x;
  int t;
  const int ex = block_excl_scan(b < nb ? s.cnt[b] : 0, s.wsum, &t);
  if (b < nb) {
    s.start[b] = ex;
    s.run[b] += ex;
  }
  if (threadIdx.x == 0) s.start[nb] = t;
  __syncthreads();
  if (tail) {
    plan_tail(p, s);
    return;
  }
  const bool cached = per == RT;
  auto key_or_own = [&](int slot) {
    return cached && slot == lo + (int)threadIdx.x ? own : plan_key(p, slot);
  };
  wide_scatter(lo, hi, nb, key_or_own, s.run, s.masks, [&](int i, int bk, int pos) {
    p.sorted[pos] = i;
    if (p.sort_order_out && bk < p.E) p.sort_order_out[pos] = routed_slot(p, i);
  });
}

// Larger batches: the same plan over RB-slot blocks in three launches --
// per-block bucket counts, one work-group that turns them into per-block
// bucket offsets (block order keeps every bucket in ascending slot order)
// and runs the tail, and a per-block stable scatter from those offsets.
constexpr int RB = 1024;  // slots per block

__global__ void __launch_bounds__(RT) route_count_kernel(RoutePlanParams p) {
  __shared__ int cnt[MAX_BUCKETS];
  const int lo = blockIdx.x * RB;
  const int m = min(RB, p.n - lo);
  const int nb = p.Ep;
  histogram(m, nb, [&](int i) { return plan_key(p, lo + i); }, cnt);
  for (int e = threadIdx.x; e < nb; e += RT) p.blk_cnt[(int64_t)blockIdx.x * nb + e] = cnt[e];
}

__global__ void __launch_bounds__(RT) route_scan_kernel(RoutePlanParams p, int nblk) {
  __shared__ RouteLds s;
  const int nb = p.Ep;
  const int b = threadIdx.x;
  // the bucket's per-block counts, 16 loads in flight at a time (a loop of
  // single loads would wait out one memory latency per block)
  constexpr int CB = 16;
  int tot_b = 0;
  if (b < nb) {
    for (int k0 = 0; k0 < nblk; k0 += CB) {
      int cv[CB];
#pragma unroll
      for (int j = 0; j < CB; ++j) cv[j] = k0 + j < nblk ? p.blk_cnt[(int64_t)(k0 + j) * nb + b] : 0;
#pragma unroll
      for (int j = 0; j < CB; ++j) tot_b += cv[j];
    }
    s.cnt[b] = tot_b;
  }
  int t;
  const int ex = block_excl_scan(b < nb ? tot_b : 0, s.wsum, &t);
  if (b < nb) {
    s.start[b] = ex;
    int run = ex;
    for (int k0 = 0; k0 < nblk; k0 += CB) {  // counts -> offsets, in place
      int cv[CB];
#pragma unroll
      for (int j = 0; j < CB; ++j) cv[j] = k0 + j < nblk ? p.blk_cnt[(int64_t)(k0 + j) * nb + b] : 0;
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        if (k0 + j < nblk) p.blk_cnt[(int64_t)(k0 + j) * nb + b] = run;
        run += cv[j];
      }
    }
  }
  if (threadIdx.x == 0) s.start[nb] = t;
  __syncthreads();
  plan_tail(p, s);
}

__global__ void __launch_bounds__(RT) route_scatter_kernel(RoutePlanParams p) {
  __shared__ RouteLds s;
  const int lo = blockIdx.x * RB;
  const int m = min(RB, p.n - lo);
  const int nb = p.Ep;
  for (int e = threadIdx.x; e < nb; e += RT) s.run[e] = p.blk_cnt[(int64_t)blockIdx.x * nb + e];
  __syncthreads();
  stable_scatter(m, nb, [&](int i) { return plan_key(p, lo + i); }, s.run, s.masks,
                 [&](int i, int b, int pos) {
                   p.sorted[pos] = lo + i;
                   if (p.sort_order_out && b < p.E) p.sort_order_out[pos] = routed_slot(p, lo + i);
                 });
}

// ---- token groups from user boundaries ------------------------------------------
__global__ void __launch_bounds__(RT) tg_from_ends_kernel(const int32_t* ends, int E,
                                                          const int32_t* mask, int tier,
                                                          int gsz, int* hdr, TgEntry* tg,
                                                          int tg_cap) {
  __shared__ int wsum[RT_WAVES];
  int base = 0;
  for (int e0 = 0; e0 < E; e0 += RT) {
    const int e = e0 + (int)threadIdx.x;
    int lo = 0, c = 0;
    if (e < E && (!mask || mask[e] != 0)) {
      lo = ends[e];
      c = ends[e + 1] - lo;
      if (c < 0) c = 0;
    }
    const int ng = (c + gsz - 1) / gsz;
    int tot;
    int off = block_excl_scan(ng, wsum, &tot);
    for (int g = 0; g < ng; ++g) {
      const int slot = base + off + g;
      if (slot < tg_cap) {
        TgEntry te;
        te.e = e;
        te.pos0 = lo + g * gsz;
        te.cnt = min(gsz, c - g * gsz);
        te.tier = tier;
        tg[slot] = te;
      }
    }
    base += tot;
  }
  if (threadIdx.x == 0) {
    hdr[0] = base < tg_cap ? base : tg_cap;
    hdr[1] = tier == 2 ? 0 : hdr[0];
    hdr[2] = tier == 0 ? hdr[0] : 0;
    hdr[3] = hdr[1];  // one group size: no big-group INT4 experts
  }
}

}  // namespace

int64_t route_plan_blocks(int64_t n) { return n > kRoutePlanOneBlock ? cdiv(n, RB) : 0; }

int launch_route_plan(const RoutePlanParams& p, hipStream_t stream) {
  const int64_t nblk = route_plan_blocks(p.n);
  if (nblk == 0 || p.blk_cnt == nullptr) {
    hipLaunchKernelGGL(route_plan_kernel, dim3(1), dim3(RT), 0, stream, p);
    return check_launch("route_plan_kernel");
  }
  if (p.n <= kRecountMaxSlots) {
    int grid, per;
    wide_grid(p.n, &grid, &per);
    hipLaunchKernelGGL(route_plan_recount_kernel, dim3(grid + 1), dim3(RT), 0, stream, p, per);
    return check_launch("route_plan_recount_kernel");
  }
  hipLaunchKernelGGL(route_count_kernel, dim3((unsigned)nblk), dim3(RT), 0, stream, p);
  int st = check_launch("route_count_kernel");
  if (st) return st;
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(RT), 0, stream, p, (int)nblk);
  st = check_launch("route_scan_kernel");
  if (st) return st;
  hipLaunchKernelGGL(route_scatter_kernel, dim3((unsigned)nblk), dim3(RT), 0, stream, p);
  return check_launch("route_scatter_kernel");
}

int launch_tg_from_ends(const int32_t* ends, int E, const int32_t* expert_mask, int tier,
                        int group, int* hdr, TgEntry* tg, int tg_cap, hipStream_t stream) {
  hipLaunchKernelGGL(tg_from_ends_kernel, dim3(1), dim3(RT), 0, stream, ends, E, expert_mask,
                     tier, group, hdr, tg, tg_cap);
  return check_launch("tg_from_ends_kernel");
}

// ---------------------------------------------------------------------------
// Router: fp32 softmax over a token's expert logits, the top-k experts, and
// optionally their weights renormalised to sum to one.  One wave per token;
// lane l holds logits l, l + 64, ...  The top-k is taken on the rounded fp32
// probabilities (largest first, equal probabilities to the lower expert id),
// as torch.topk over the softmax ranks them.  The denominator is a
// fixed-order wave reduction (deterministic).
// Wave-wide reductions with DPP (gfx9 row forms): quad swaps, rotations by 4
// and 8 inside each 16-lane row, then rows folded into row 3 by the row-15 and
// row-31 broadcasts; lane 63 ends with the result, read back as a scalar.
// `ID` is the operation's identity, returned by lanes a step does not write.
template <int CTRL, int ROWS, uint32_t ID>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)ID, (int)v, CTRL, ROWS, 0xf, false);
}
template <uint32_t ID, typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, Op op) {
  v = op(v, dpp_u32<0xB1, 0xf, ID>(v));   // quad_perm [1, 0, 3, 2]
  v = op(v, dpp_u32<0x4E, 0xf, ID>(v));   // quad_perm [2, 3, 0, 1]
  v = op(v, dpp_u32<0x124, 0xf, ID>(v));  // row_ror 4
  v = op(v, dpp_u32<0x128, 0xf, ID>(v));  // row_ror 8
  v = op(v, dpp_u32<0x142, 0xa, ID>(v));  // row_bcast 15 -> rows 1, 3
  v = op(v, dpp_u32<0x143, 0xc, ID>(v));  // row_bcast 31 -> rows 2, 3
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  return __uint_as_float(wave_reduce_u32<0u>(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(__uint_as_float(x) + __uint_as_float(y));
  }));
}

// Order-preserving key of a logit (larger logit, larger key; -0 and +0 share
// one, as they compare equal); key 0 lies below every logit and marks an
// expert that is taken or absent.
__device__ __forceinline__ uint32_t logit_key(float x) {
  uint32_t b = __float_as_uint(x);
  if ((b << 1) == 0u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// One wave per token: lane l holds logits l, l + 64, ...  The ranking is the
// reference's, torch.topk over the fp32 softmax (triton_emitter.py:273-277):
// every expert's probability p = exp(l - max) / sum is computed first (IEEE
// division, as numpy's and torch's `/`), and each of the k rounds takes the
// largest remaining p, equal p to the lower id.  Two different logits whose
// probabilities round to the same fp32 value are a tie, exactly as in the
// reference; ranking on the logits would split it.  A round is one DPP maximum
// over the lanes' best keys, plus a DPP minimum over the ids only when several
// lanes hold that key.  Key = bits(p) + 1 (p >= 0, so the bits are ordered);
// key 0 marks an expert that is taken or absent.
template <int MAXC>
__global__ void __launch_bounds__(256) topk_softmax_kernel(const void* logits, int ldt, int T,
                                                          int E, int k, int renorm, void* ids,
                                                          int idt, void* wts, int wdt) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;  // (wave-uniform)
  const auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  const auto umin = [](uint32_t x, uint32_t y) { return x < y ? x : y; };
  uint32_t key[MAXC];
  uint32_t kmax = 0u;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int e = lane + 64 * c;
    key[c] = e < E ? logit_key(load_as_f32(logits, ldt, (int64_t)row * E + e)) : 0u;
    kmax = umax(kmax, key[c]);
  }
  const float m = key_logit(wave_reduce_u32<0u>(kmax, umax));
  float ex[MAXC];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    ex[c] = lane + 64 * c < E ? expf(key_logit(key[c]) - m) : 0.f;
    sum += ex[c];
  }
  const float S = wave_sum_f32(sum);
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
    key[c] = lane + 64 * c < E ? __float_as_uint(ex[c] / S) + 1u : 0u;
  float mine = 0.f;  // lane j < k: weight of the j-th choice
  int my_id = 0;     // lane j < k: id of the j-th choice
  float ws = 0.f;    // sum of the chosen weights, in choice order
  for (int j = 0; j < k; ++j) {
    uint32_t bk = 0u;
    int bc = 0;
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (key[c] > bk) {  // strict: the lower c (lower id) keeps a tie
        bk = key[c];
        bc = c;
      }
    const uint32_t K = wave_reduce_u32<0u>(bk, umax);
    const uint64_t at = __ballot(bk == K);
    int be;
    if (__popcll(at) == 1) {
      const int l = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)at) - 1);
      be = __builtin_amdgcn_readlane(lane + 64 * bc, l);
    } else {
      be = (int)wave_reduce_u32<0xffffffffu>(bk == K ? (uint32_t)(lane + 64 * bc) : 0xffffffffu, umin);
    }
    if ((be & 63) == lane) {
#pragma unroll
      for (int c = 0; c < MAXC; ++c)
        if (c == (be >> 6)) key[c] = 0u;
    }
    const float w = __uint_as_float(K - 1u);
    ws += w;
    if (lane == j) {
      mine = w;
      my_id = be;
    }
  }
  if (renorm) mine = mine / ws;
  if (lane < k) {
    if (idt == EXQ_DTYPE_I64)
      reinterpret_cast<int64_t*>(ids)[(int64_t)row * k + lane] = my_id;
    else
      reinterpret_cast<int32_t*>(ids)[(int64_t)row * k + lane] = my_id;
    store_from_f32(wts, wdt, (int64_t)row * k + lane, mine);
  }
}

}  // namespace exq

using namespace exq;

extern "C" int exq_dispatch(const void* router_indices, int ids_dtype, int64_t n,
                            int64_t n_experts, int64_t* sort_order, int64_t* sorted_expert_ids,
                            int32_t* expert_ends, exq_stream stream) {
  EXQ_REQUIRE(is_index_dtype(ids_dtype), "exq_dispatch: ids dtype must be i32 or i64");
  EXQ_REQUIRE(n >= 0 && n <= INT32_MAX, "exq_dispatch: n=%lld out of range", (long long)n);
  EXQ_REQUIRE(n_experts >= 1 && n_experts < kWideMaxBuckets,
              "exq_dispatch: n_experts=%lld must be in [1, %d)", (long long)n_experts,
              kWideMaxBuckets);
  EXQ_REQUIRE(expert_ends && (n == 0 || (router_indices && sort_order && sorted_expert_ids)),
              "exq_dispatch: null pointer");
  if (n > kRoutePlanOneBlock || n_experts + 1 > MAX_BUCKETS) {
    int grid, per;
    wide_grid(n, &grid, &per);
    hipLaunchKernelGGL(wide_dispatch_kernel, dim3(grid), dim3(RT), 0, as_stream(stream),
                       router_indices, ids_dtype, (int)n, (int)n_experts, per, sort_order,
                       sorted_expert_ids, expert_ends);
    return check_launch("wide_dispatch_kernel");
  }
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(RT), 0, as_stream(stream), router_indices,
                     ids_dtype, (int)n, (int)n_experts, sort_order, sorted_expert_ids,
                     expert_ends);
  return check_launch("dispatch_kernel");
}

extern "C" int exq_build_ends_from_slots(const int32_t* sorted_slot_ids, int64_t em,
                                         const int32_t* flat_router, int64_t n_active,
                                         int64_t n_experts, int32_t* expert_ends,
                                         int64_t* sort_order, exq_stream stream) {
  EXQ_REQUIRE(em >= 0 && em <= INT32_MAX && n_active >= 0 && n_active <= INT32_MAX,
              "exq_build_ends_from_slots: sizes out of range");
  EXQ_REQUIRE(n_experts >= 1 && n_experts <= kWideMaxBuckets,
              "exq_build_ends_from_slots: n_experts=%lld must be in [1, %d]",
              (long long)n_experts, kWideMaxBuckets);
  EXQ_REQUIRE(expert_ends && (em == 0 || (sorted_slot_ids && flat_router && sort_order)),
              "exq_build_ends_from_slots: null pointer");
  if (em > kRoutePlanOneBlock || n_experts > MAX_BUCKETS) {
    int grid, per;
    wide_grid(em, &grid, &per);
    hipLaunchKernelGGL(wide_build_ends_kernel, dim3(grid), dim3(RT), 0, as_stream(stream),
                       sorted_slot_ids, (int)em, flat_router, (int)n_active, (int)n_experts, per,
                       expert_ends, sort_order);
    return check_launch("wide_build_ends_kernel");
  }
  hipLaunchKernelGGL(build_ends_kernel, dim3(1), dim3(RT), 0, as_stream(stream),
                     sorted_slot_ids, (int)em, flat_router, (int)n_active, (int)n_experts,
                     expert_ends, sort_order);
  return check_launch("build_ends_kernel");
}

extern "C" int exq_moe_align_block_size(const void* topk_ids, int ids_dtype, int64_t numel,
                                        int64_t num_experts, int64_t block_size,
                                        int32_t* sorted_token_ids, int64_t sorted_capacity,
                                        int32_t* expert_ids, int64_t expert_ids_capacity,
                                        int32_t* num_tokens_post_pad, int32_t* cumsum,
                                        int pad_sorted_token_ids, exq_stream stream) {
  EXQ_REQUIRE(is_index_dtype(ids_dtype), "exq_moe_align_block_size: ids dtype must be i32/i64");
  EXQ_REQUIRE(numel >= 0 && numel <= INT32_MAX, "exq_moe_align_block_size: numel out of range");
  EXQ_REQUIRE(num_experts >= 1 && num_experts <= kWideMaxBuckets,
              "exq_moe_align_block_size: num_experts=%lld must be in [1, %d]",
              (long long)num_experts, kWideMaxBuckets);
  EXQ_REQUIRE(block_size >= 1 && block_size <= 4096,
              "exq_moe_align_block_size: block_size=%lld out of range", (long long)block_size);
  const int64_t need = numel + num_experts * (block_size - 1);
  EXQ_REQUIRE(sorted_capacity >= need && need <= INT32_MAX,
              "exq_moe_align_block_size: sorted_token_ids capacity %lld < %lld",
              (long long)sorted_capacity, (long long)need);
  EXQ_REQUIRE(expert_ids_capacity >= cdiv(need, block_size),
              "exq_moe_align_block_size: expert_ids capacity %lld < %lld",
              (long long)expert_ids_capacity, (long long)cdiv(need, block_size));
  EXQ_REQUIRE(sorted_token_ids && expert_ids && num_tokens_post_pad && cumsum &&
                  (numel == 0 || topk_ids),
              "exq_moe_align_block_size: null pointer");
  if (numel > kRoutePlanOneBlock || num_experts > MAX_BUCKETS) {
    int grid, per;
    wide_grid(numel, &grid, &per);
    hipLaunchKernelGGL(wide_align_kernel, dim3(grid), dim3(RT), 0, as_stream(stream), topk_ids,
                       ids_dtype, (int)numel, (int)num_experts, (int)block_size, per,
                       sorted_token_ids, (int)sorted_capacity, expert_ids,
                       (int)expert_ids_capacity, num_tokens_post_pad, cumsum,
                       pad_sorted_token_ids ? 1 : 0);
    return check_launch("wide_align_kernel");
  }
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(RT), 0, as_stream(stream), topk_ids, ids_dtype,
                     (int)numel, (int)num_experts, (int)block_size, sorted_token_ids,
                     (int)sorted_capacity, expert_ids, (int)expert_ids_capacity,
                     num_tokens_post_pad, cumsum, pad_sorted_token_ids ? 1 : 0);
  return check_launch("align_kernel");
}

extern "C" int exq_topk_softmax(const void* logits, int logits_dtype, int64_t n_tokens,
                                int64_t n_experts, int64_t top_k, int renormalize,
                                void* topk_ids, int ids_dtype, void* topk_weights,
                                int weights_dtype, exq_stream stream) {
  EXQ_REQUIRE(logits_dtype == EXQ_DTYPE_F32 || is_act_dtype(logits_dtype),
              "exq_topk_softmax: logits dtype must be f32, f16 or bf16");
  EXQ_REQUIRE(is_index_dtype(ids_dtype), "exq_topk_softmax: ids dtype must be i32 or i64");
  EXQ_REQUIRE(weights_dtype == EXQ_DTYPE_F32 || is_act_dtype(weights_dtype),
              "exq_topk_softmax: weights dtype must be f32, f16 or bf16");
  EXQ_REQUIRE(n_tokens >= 0 && n_tokens <= INT32_MAX / 4,
              "exq_topk_softmax: n_tokens=%lld out of range", (long long)n_tokens);
  EXQ_REQUIRE(n_experts >= 1 && n_experts <= 1024,
              "exq_topk_softmax: n_experts=%lld must be in [1, 1024]", (long long)n_experts);
  EXQ_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= 64,
              "exq_topk_softmax: top_k=%lld must be in [1, min(n_experts, 64)]",
              (long long)top_k);
  if (n_tokens == 0) return EXQ_SUCCESS;
  EXQ_REQUIRE(logits && topk_ids && topk_weights, "exq_topk_softmax: null pointer");
  const dim3 g((unsigned)((n_tokens + 3) / 4));
  const hipStream_t s = as_stream(stream);
  if (n_experts <= 256)
    hipLaunchKernelGGL(topk_softmax_kernel<4>, g, dim3(256), 0, s, logits, logits_dtype,
                       (int)n_tokens, (int)n_experts, (int)top_k, renormalize ? 1 : 0, topk_ids,
                       ids_dtype, topk_weights, weights_dtype);
  else
    hipLaunchKernelGGL(topk_softmax_kernel<16>, g, dim3(256), 0, s, logits, logits_dtype,
                       (int)n_tokens, (int)n_experts, (int)top_k, renormalize ? 1 : 0, topk_ids,
                       ids_dtype, topk_weights, weights_dtype);
  return check_launch("topk_softmax_kernel");
}
