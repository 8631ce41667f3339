// Allocation-free chained MLP: miaie_mlp_i8 with H in a file-scope device
// array instead of a caller-provided workspace.
//
// For callers that cannot allocate device memory on the call path (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
// The array is part of the library's code object, so every GPU the library
// runs on holds one copy of it from the context's set-up until the process
// ends.  In host code `scratch` names a host-side stand-in, not a device
// address: miaie_init resolves the address on each device once
// (scratch_setup, hipGetSymbolAddress) and kernels only ever see that
// address.  Nothing here calls hipMalloc, hipFree or hipMemset*.
//
// Calls from different streams (contexts) on one GPU are ordered through one
// event per device, created by the same set-up: under a host mutex each call
// makes its stream wait for the event, queues its two GEMMs and records the
// event after them, so the next call's first GEMM starts only after this
// call's second GEMM has read H.  A call recorded into a graph takes no part
// in that chain (its replays are not ordered against other calls).
#include <mutex>

#include "miaie_internal.hpp"

namespace {

constexpr size_t kScratchBytes = MIAIE_MLP_NOALLOC_MAX_H;

// H of miaie_mlp_i8_noalloc: M*F int8 bytes, written completely by the first
// GEMM before the second reads it, so it never needs clearing.
__device__ __align__(256) int8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];       // device address of `scratch`, per device
hipEvent_t g_scratch_ev[kMaxDevices];   // the last queued use of that array, per device

}  // namespace

namespace miaie {

int scratch_setup(miaie_ctx* ctx) {
  const int dev = ctx->device;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ctx, MIAIE_EUNSUPPORTED, "miaie_init: device %d beyond the %d this build tracks", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(ctx, MIAIE_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
    hipEvent_t ev = nullptr;
    const hipError_t e2 = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e2 != hipSuccess) return hip_fail(ctx, e2, "hipEventCreateWithFlags(scratch order)");
    g_scratch_ptr[dev] = p;
    g_scratch_ev[dev] = ev;
  }
  ctx->scratch = g_scratch_ptr[dev];
  return MIAIE_OK;
}

}  // namespace miaie

using namespace miaie;

extern "C" int miaie_mlp_i8_noalloc(miaie_ctx* ctx, const int8_t* X, const int8_t* W1, const int8_t* W2, int8_t* Y,
                                    int M, int K, int F, int Nout, int s1, int s2) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (M >= 1 && F >= 1 && (size_t)M * (size_t)F > kScratchBytes)
    return fail(ctx, MIAIE_EINVAL,
                "%s: H needs M*F = %zu bytes; the allocation-free MLP holds at most %zu "
                "(MIAIE_MLP_NOALLOC_MAX_H); use miaie_mlp_i8 with a caller-provided H",
                __func__, (size_t)M * (size_t)F, kScratchBytes);
  if (ctx->scratch == nullptr) return fail(ctx, MIAIE_EHIP, "%s: scratch address not resolved", __func__);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const hipEvent_t ev = g_scratch_ev[ctx->device];
  if (!ctx->recording) {
    const hipError_t e = hipStreamWaitEvent(ctx->stream, ev, 0);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamWaitEvent(scratch order)");
  }
  rc = mlp_i8_checked(ctx, __func__, X, W1, W2, static_cast<int8_t*>(ctx->scratch), Y, M, K, F, Nout, s1, s2);
  if (!ctx->recording) {
    // also after a failure: whatever part of the call was queued is ordered
    const hipError_t e = hipEventRecord(ev, ctx->stream);
    if (e != hipSuccess && rc == MIAIE_OK) return hip_fail(ctx, e, "hipEventRecord(scratch order)");
  }
  return rc;
}
