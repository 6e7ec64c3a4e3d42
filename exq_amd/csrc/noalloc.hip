// noalloc.hip -- the INT4 MoE layer entry point for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops and
// harnesses that forbid hipMalloc): the fused layer's workspace is a
// file-scope device array instead of a caller buffer.
//
// Each GPU the library runs on holds its own copy of the array (its address
// is looked up once per device with hipGetSymbolAddress and kept), from
// module load until the process ends.  Every call on one GPU shares that
// GPU's array: calls that overlap on one GPU (two streams, two threads) race
// on it.  The array keeps the last call's contents; the only part that must
// start at zero, the decode kernels' combine counters, is cleared by each
// call's first kernel (as for any caller workspace).  The first call on a
// device must be made outside graph capture; later calls may be captured.
#include "exq_internal.h"

#include <mutex>

// EXQ_NOALLOC_SCRATCH_BYTES of scratch for the no-alloc entry point.
static __device__ __align__(256) unsigned char scratch[EXQ_NOALLOC_SCRATCH_BYTES];

namespace exq {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (looked up once per device,
// with that device current).  The first lookup on a device may load the code
// object that holds the array, which places the array in device memory, so it
// is refused while `s` is being captured into a graph: the caller makes one
// call outside capture first (a call with n_tokens = 0 is enough).
int scratch_address(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(EXQ_ERROR_HIP, "exq_moe_int4_fused_forward_noalloc: no usable current device");
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t qe = hipStreamIsCapturing(s, &cs);
    if (qe != hipSuccess || cs != hipStreamCaptureStatusNone) {
      (void)hipGetLastError();  // a failed query must not be reported by a later launch check
      return set_error(EXQ_ERROR_UNSUPPORTED,
                       "exq_moe_int4_fused_forward_noalloc: the first call on device %d is "
                       "under graph capture (or its capture state is unknown: %s); make one "
                       "call outside capture first (n_tokens = 0 is enough)",
                       dev, hipGetErrorString(qe));
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(EXQ_ERROR_HIP,
                       "exq_moe_int4_fused_forward_noalloc: hipGetSymbolAddress failed: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return EXQ_SUCCESS;
}

}  // namespace
}  // namespace exq

using namespace exq;

extern "C" int exq_moe_int4_fused_forward_noalloc(
    const exq_moe_problem* problem, const void* hidden, const void* topk_ids,
    const void* topk_weights, const uint8_t* w13_packed, const uint16_t* w13_scales,
    const uint8_t* w2_packed, const uint16_t* w2_scales, void* out, int64_t* sort_order_out,
    int32_t* expert_ends_out, exq_stream stream) {
  const char* fn = "exq_moe_int4_fused_forward_noalloc";
  EXQ_REQUIRE(problem != nullptr, "%s: null problem", fn);
  const size_t need = exq_moe_workspace_size(problem);
  if (need > (size_t)EXQ_NOALLOC_SCRATCH_BYTES)
    return set_error(EXQ_ERROR_WORKSPACE_TOO_SMALL,
                     "%s: this problem needs %zu bytes of scratch; the no-alloc entry point "
                     "holds %zu (use exq_moe_int4_fused_forward with a workspace)",
                     fn, need, (size_t)EXQ_NOALLOC_SCRATCH_BYTES);
  // the scratch address is resolved even for an empty batch, so that a call with
  // n_tokens = 0 prepares a device for later calls under graph capture
  void* ws = nullptr;
  const int st = scratch_address(as_stream(stream), &ws);
  if (st) return st;
  if (problem->n_tokens == 0) return EXQ_SUCCESS;
  return exq_moe_int4_fused_forward(problem, hidden, topk_ids, topk_weights, w13_packed,
                                    w13_scales, w2_packed, w2_scales, out, sort_order_out,
                                    expert_ends_out, ws, (size_t)EXQ_NOALLOC_SCRATCH_BYTES,
                                    stream);
}
