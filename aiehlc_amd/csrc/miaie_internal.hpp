// Internal declarations shared by the miaie HIP translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <tuple>
#include <utility>

#include "../../include/miaie.h"
#include "dbg_checks.hpp"

struct miaie_ctx {
  unsigned long long id = 0;  // unique per context in the process (a graph records its context's id)
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  hipEvent_t done = nullptr;  // recorded by miaie_wait
  int cus = 256;              // compute units of the device (grid sizing of persistent kernels)
  bool recording = false;     // between miaie_graph_begin and miaie_graph_end
  void* scratch = nullptr;    // device address of this device's file-scope scratch array (noalloc.hip)
  // Device workspace owned by this context, allocated once at init so that
  // no entry point allocates: the conv's split-K partial sums.  Work queued
  // on the context's one stream uses it in stream order.
  void* work = nullptr;
  size_t work_bytes = 0;
  char err[512] = {0};
};

constexpr size_t MIAIE_CTX_WORK_BYTES = (size_t)16 << 20;

namespace miaie {

// Record an error message on the context (printf-style) and return `code`.
int fail(miaie_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

// Map a HIP error to MIAIE_EHIP with a message naming the call.
int hip_fail(miaie_ctx* ctx, hipError_t e, const char* what);

// Check a launch's result (MIAIE_EHIP naming the kernel when it failed).
int check_launch(miaie_ctx* ctx, hipError_t e, const char* kernel);

template <class F>
struct kernel_sig;
template <class... P>
struct kernel_sig<void (*)(P...)> {
  using args = std::tuple<P...>;
};

// Launch kernel K through the module API, with its handle looked up once per
// device (device < 0: the current one, read on every call), and return the
// launch's own status.  hipLaunchKernel finds the kernel from its host address
// on every call and reports a failed launch only through hipGetLastError, the
// thread's last error from any runtime call (a caller's earlier failure would
// be taken for the launch's): on the host, 2.47-2.95 us per launch with that
// check against 2.22-2.81 us here, box to box, measured with an empty kernel
// of the row-block conv's arguments and grid.  The arguments are first converted to the kernel's parameter
// types, since the runtime copies each by the size of its parameter.  The
// caller has the device current (hipGetFuncBySymbol resolves on it).
constexpr int kLaunchCacheDevices = 64;
template <auto K, class... A>
hipError_t launch(int device, dim3 grid, dim3 block, size_t lds_bytes, hipStream_t st, A&&... a) {
  using Args = typename kernel_sig<decltype(K)>::args;
  static_assert(std::tuple_size<Args>::value == sizeof...(A) && sizeof...(A) > 0, "kernel argument count");
  static std::atomic<hipFunction_t> cache[kLaunchCacheDevices];
  if (device < 0) {
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
  }
  const bool cached = device < kLaunchCacheDevices;
  hipFunction_t f = cached ? cache[device].load(std::memory_order_acquire) : nullptr;
  if (!f) {
    hipError_t e = hipGetFuncBySymbol(&f, reinterpret_cast<const void*>(K));
    if (e != hipSuccess) return e;
    if (cached) cache[device].store(f, std::memory_order_release);
  }
  Args vals(std::forward<A>(a)...);
  void* ptrs[sizeof...(A)];
  std::apply([&](auto&... v) {
    int i = 0;
    ((ptrs[i++] = static_cast<void*>(&v)), ...);
  }, vals);
  return hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)lds_bytes, st, ptrs,
                               nullptr);
}

// A kernel as a type, for launchers that pick one of several kernels at run
// time and launch it through launch<K>: go(kernel_t<some_kernel<...>>{}).
template <auto K>
struct kernel_t {
  static constexpr auto value = K;
};

// Every entry point starts with this: non-null context, its device current.
int enter(miaie_ctx* ctx);

// Entry points that wait for the device or allocate start with this: they
// cannot be recorded into a graph.
int refuse_while_recording(miaie_ctx* ctx, const char* what);

__host__ __device__ inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// The device-check buffer table of the debug build (no-ops returning
// MIAIE_OK in the product build; miaie_runtime.hip): add or replace the
// extent of the buffer at p, drop it, and read (and clear) the fault records
// after the context's stream has drained (MIAIE_EFAULT with a message naming
// the first fault).
int dbg_add(miaie_ctx* ctx, const void* p, size_t bytes);
int dbg_remove(miaie_ctx* ctx, const void* p);
int dbg_take_faults(miaie_ctx* ctx);

// Resolve the device address of the allocation-free entry points' scratch
// array on ctx->device (current) into ctx->scratch (noalloc.hip).
int scratch_setup(miaie_ctx* ctx);

// Validated chained MLP over a caller-chosen H (capi.hip).
int mlp_i8_checked(miaie_ctx* ctx, const char* fn, const int8_t* X, const int8_t* W1, const int8_t* W2, int8_t* H,
                   int8_t* Y, int M, int K, int F, int Nout, int s1, int s2);

// ---- kernel launchers implemented in the kernel translation units ----
// keep_y: Y is read by the next kernel (ordinary stores instead of
// non-temporal ones where the kernel has that form).
int launch_gemm_i8(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C, int M,
                   int N, int K, int lda, int ldb, int ldy, int ldc, int b_nt, int shift, int relu,
                   bool keep_y = false);
// Kernel plan for dense operands (dense_ok: the pipelined kernel's operand
// conditions hold).
int plan_gemm_i8(miaie_ctx* ctx, int M, int N, int K, int dense_ok, miaie_gemm_plan* plan);
int launch_gemm_bf16(miaie_ctx* ctx, const uint16_t* A, const uint16_t* B, float* C, int M, int N,
                     int K);
// MIAIE_CONV_* kernel for a shape on `cus` compute units (conv2d_i8.hip);
// the shape must be valid.
int conv2d_kernel_for(int N, int H, int Wd, int Cin, int Cout, int R, int S, int stride, int pad, bool aligned16,
                      bool shifts_aligned4, int cus);
int launch_conv2d_i8(miaie_ctx* ctx, const int8_t* X, const int8_t* W, const uint8_t* shifts,
                     int8_t* Y, int N, int H, int Wd, int Cin, int Cout, int R, int S, int stride,
                     int pad);

}  // namespace miaie

// Vector types used by the MFMA builtins.
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define MIAIE_CHECK_NOT_NULL(ctx, p)                                              \
  do {                                                                          \
    if ((p) == nullptr) return miaie::fail((ctx), MIAIE_EINVAL, "%s: " #p " is NULL", __func__); \
  } while (0)
