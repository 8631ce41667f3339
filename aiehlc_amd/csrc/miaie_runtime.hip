// miaie runtime: context, device memory, copies, waits, synthetic fills.
//
// These entry points stand in for the aie-rt host calls the reference
// harnesses make (example/perf/aieml_perf.cc:256-328,
// example/matrixmultiply/aieml_mm.cc:108-249): configuration and partition
// set-up become a context bound to one HIP device and stream; MemAllocate
// and MoveData become hipMalloc and stream-ordered copies; Run becomes an
// asynchronous kernel launch; CoreWaitForDone becomes an event wait with a
// deadline.
#include <time.h>

#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "miaie_internal.hpp"

namespace {
thread_local char g_init_err[512] = {0};
}

namespace miaie {

int fail(miaie_ctx* ctx, int code, const char* fmt, ...) {
  char* buf = ctx ? ctx->err : g_init_err;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, 512, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(miaie_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, e == hipErrorOutOfMemory ? MIAIE_ENOMEM : MIAIE_EHIP, "%s: %s (%s)", what,
              hipGetErrorString(e), hipGetErrorName(e));
}

int enter(miaie_ctx* ctx) {
  if (!ctx) return fail(nullptr, MIAIE_EINVAL, "context is NULL");
  // (reading the current device is cheaper than setting it: 0.08 us per
  // call on the host, measured)
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess && cur == ctx->device) return MIAIE_OK;
  e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
  return MIAIE_OK;
}

int check_launch(miaie_ctx* ctx, hipError_t e, const char* kernel) {
  if (e != hipSuccess) return hip_fail(ctx, e, kernel);
  return MIAIE_OK;
}

int refuse_while_recording(miaie_ctx* ctx, const char* what) {
  if (ctx->recording)
    return fail(ctx, MIAIE_EINVAL, "%s: not allowed while a graph is being recorded (miaie_graph_begin)", what);
  return MIAIE_OK;
}

// ---------------------------------------------------------------- device bounds checks
// The buffer table of the debug build (dbg_checks.hpp): one process-wide map
// of [lo, hi) ranges, uploaded into every translation unit's copy of the
// device table on the context's device after each change.  The product build
// keeps nothing: the hooks below return MIAIE_OK.
#if MIAIE_DEVICE_CHECKS
namespace dbg {
namespace {
std::mutex& table_mu() {
  static std::mutex m;
  return m;
}
std::vector<Unit>& units() {
  static std::vector<Unit> u;
  return u;
}
std::map<uint64_t, uint64_t>& table() {
  static std::map<uint64_t, uint64_t> t;
  return t;
}
// with table_mu held
int upload_locked(miaie_ctx* ctx) {
  static Ranges r;
  r.n = 0;
  for (const auto& [lo, hi] : table()) {
    r.lo[r.n] = lo;
    r.hi[r.n] = hi;
    ++r.n;
  }
  // kernels in flight read the table: replace it only when the device is idle
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(ctx, e, "hipDeviceSynchronize (device check table)");
  for (const Unit& u : units()) {
    e = (hipError_t)u.upload(r, ctx->device);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMemcpyToSymbol (device check table)");
  }
  return MIAIE_OK;
}
}  // namespace

void register_unit(const Unit& u) {
  std::lock_guard<std::mutex> lock(table_mu());
  units().push_back(u);
}
}  // namespace dbg

int dbg_add(miaie_ctx* ctx, const void* p, size_t bytes) {
  std::lock_guard<std::mutex> lock(dbg::table_mu());
  auto& t = dbg::table();
  const uint64_t lo = (uint64_t)(uintptr_t)p, hi = lo + bytes;
  t.erase(lo);  // a new extent for a known base replaces the old one
  auto next = t.lower_bound(lo);
  if (next != t.end() && next->first < hi)
    return fail(ctx, MIAIE_EINVAL, "device check table: [%p, +%zu) overlaps the buffer at 0x%llx", p, bytes,
                (unsigned long long)next->first);
  if (next != t.begin() && std::prev(next)->second > lo)
    return fail(ctx, MIAIE_EINVAL, "device check table: [%p, +%zu) overlaps the buffer at 0x%llx", p, bytes,
                (unsigned long long)std::prev(next)->first);
  if (t.size() >= (size_t)dbg::kMaxRanges)
    return fail(ctx, MIAIE_ENOMEM, "device check table: more than %d buffers", dbg::kMaxRanges);
  t[lo] = hi;
  return dbg::upload_locked(ctx);
}

int dbg_remove(miaie_ctx* ctx, const void* p) {
  std::lock_guard<std::mutex> lock(dbg::table_mu());
  if (dbg::table().erase((uint64_t)(uintptr_t)p) == 0) return MIAIE_OK;
  return dbg::upload_locked(ctx);
}

int dbg_take_faults(miaie_ctx* ctx) {
  std::lock_guard<std::mutex> lock(dbg::table_mu());
  unsigned long long total = 0;
  dbg::Fault first{};
  const char* where = "";
  for (const dbg::Unit& u : dbg::units()) {
    dbg::Fault f{};
    hipError_t e = (hipError_t)u.take(&f, ctx->device);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMemcpyFromSymbol (device check record)");
    if (f.count && !total) {
      first = f;
      where = u.name;
    }
    total += f.count;
  }
  if (!total) return MIAIE_OK;
  static const char* const kind[] = {"load", "store", "global->LDS copy"};
  const char* file = nullptr;
  for (const char* f : dbg::kFiles)
    if (dbg::file_id(f) == first.file) file = f;
  const char* base = std::strrchr(where, '/');
  return fail(ctx, MIAIE_EFAULT,
              "device bounds check: %llu access(es) outside every known buffer; first: %s of %llu bytes at 0x%llx "
              "(%s, line %d; kernel from %s)",
              total, kind[first.write >= 0 && first.write <= 2 ? first.write : 0], first.bytes, first.addr,
              file ? file : "?", first.line, base ? base + 1 : where);
}
#else
int dbg_add(miaie_ctx*, const void*, size_t) { return MIAIE_OK; }
int dbg_remove(miaie_ctx*, const void*) { return MIAIE_OK; }
int dbg_take_faults(miaie_ctx*) { return MIAIE_OK; }
#endif

}  // namespace miaie

using namespace miaie;

// ---------------------------------------------------------------- kernels
namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__host__ __device__ inline uint64_t sm64_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Streaming copy: 16-byte vectors for the aligned body, bytes for the rest.
__global__ __launch_bounds__(256) void copy_kernel(v4i* __restrict__ dst,
                                                   const v4i* __restrict__ src, size_t nvec,
                                                   uint8_t* __restrict__ dst_tail,
                                                   const uint8_t* __restrict__ src_tail,
                                                   size_t ntail) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < nvec; i += stride) MIAIE_ST(dst + i, MIAIE_LD_NT(src + i));
  size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (t < ntail) MIAIE_ST(dst_tail + t, MIAIE_LD(src_tail + t));
}

// 16 seeded int8 values per thread.
__global__ __launch_bounds__(256) void fill_i8_kernel(int8_t* __restrict__ dst, size_t n,
                                                      uint64_t state0) {
  size_t base = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) * 16;
  if (base >= n) return;
  if (base + 16 <= n) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint64_t r = sm64_mix(state0 + (base + 4 * q + b + 1) * kGamma);
        v |= (uint32_t)(r >> 56) << (8 * b);
      }
      w[q] = v;
    }
    MIAIE_ST(reinterpret_cast<uint4*>(dst + base), make_uint4(w[0], w[1], w[2], w[3]));
  } else {
    for (size_t i = base; i < n; ++i) MIAIE_ST(dst + i, (int8_t)(uint8_t)(sm64_mix(state0 + (i + 1) * kGamma) >> 56));
  }
}

}  // namespace

// ---------------------------------------------------------------- context
extern "C" int miaie_init_on_stream(miaie_ctx** out, int device, void* stream) {
  if (!out) return fail(nullptr, MIAIE_EINVAL, "miaie_init: ctx out-pointer is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceCount");
  if (device < 0 || device >= count)
    return fail(nullptr, MIAIE_EINVAL, "miaie_init: device %d out of range [0, %d)", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, MIAIE_EUNSUPPORTED, "miaie is built for gfx950 only; device %d is %s", device,
                prop.gcnArchName);
  miaie_ctx* ctx = new (std::nothrow) miaie_ctx();
  if (!ctx) return fail(nullptr, MIAIE_ENOMEM, "miaie_init: host allocation failed");
  static std::atomic<unsigned long long> next_id{1};
  ctx->id = next_id.fetch_add(1);
  ctx->device = device;
  ctx->cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
  if (stream) {
    ctx->stream = static_cast<hipStream_t>(stream);
  } else {
    ctx->stream = nullptr;
  }
  e = hipEventCreateWithFlags(&ctx->done, hipEventDisableTiming);
  if (e != hipSuccess) {
    int rc = hip_fail(nullptr, e, "hipEventCreate");
    delete ctx;
    return rc;
  }
  if (int rc = scratch_setup(ctx)) {
    fail(nullptr, rc, "%s", ctx->err);
    (void)hipEventDestroy(ctx->done);
    delete ctx;
    return rc;
  }
  e = hipMalloc(&ctx->work, MIAIE_CTX_WORK_BYTES);
  if (e != hipSuccess) {
    int rc = hip_fail(nullptr, e, "hipMalloc (context workspace)");
    (void)hipEventDestroy(ctx->done);
    delete ctx;
    return rc;
  }
  ctx->work_bytes = MIAIE_CTX_WORK_BYTES;
  // (debug build) the workspace and the scratch array are buffers the
  // kernels may touch
  int rc = dbg_add(ctx, ctx->work, ctx->work_bytes);
  if (rc == MIAIE_OK) rc = dbg_add(ctx, ctx->scratch, MIAIE_MLP_NOALLOC_MAX_H);
  if (rc != MIAIE_OK) {
    fail(nullptr, rc, "%s", ctx->err);
    (void)dbg_remove(ctx, ctx->work);
    (void)hipFree(ctx->work);
    (void)hipEventDestroy(ctx->done);
    delete ctx;
    return rc;
  }
  *out = ctx;
  return MIAIE_OK;
}

extern "C" int miaie_init(miaie_ctx** out, int device) {
  int rc = miaie_init_on_stream(out, device, nullptr);
  if (rc != MIAIE_OK) return rc;
  miaie_ctx* ctx = *out;
  hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    rc = hip_fail(nullptr, e, "hipStreamCreate");
    (void)hipFree(ctx->work);
    (void)hipEventDestroy(ctx->done);
    delete ctx;
    *out = nullptr;
    return rc;
  }
  ctx->own_stream = true;
  return MIAIE_OK;
}

extern "C" int miaie_finish(miaie_ctx* ctx) {
  if (!ctx) return MIAIE_OK;
  int rc = MIAIE_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->recording) {  // abandon an unfinished recording
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(ctx->stream, &g);
    if (g) (void)hipGraphDestroy(g);
    ctx->recording = false;
  }
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) rc = MIAIE_EHIP;
  if (ctx->work) {
    (void)dbg_remove(ctx, ctx->work);
    (void)hipFree(ctx->work);
  }
  if (ctx->done) (void)hipEventDestroy(ctx->done);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return rc;
}

extern "C" const char* miaie_last_error_string(const miaie_ctx* ctx) {
  return ctx ? ctx->err : g_init_err;
}

extern "C" int miaie_get_stream(miaie_ctx* ctx, void** stream) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, stream);
  *stream = ctx->stream;
  return MIAIE_OK;
}

// ---------------------------------------------------------------- memory
extern "C" int miaie_alloc(miaie_ctx* ctx, size_t bytes, void** dev_ptr) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_alloc"))) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, dev_ptr);
  *dev_ptr = nullptr;
  if (bytes == 0) return fail(ctx, MIAIE_EINVAL, "miaie_alloc: zero bytes");
  hipError_t e = hipMalloc(dev_ptr, bytes);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc");
  if ((rc = dbg_add(ctx, *dev_ptr, bytes))) {
    (void)hipFree(*dev_ptr);
    *dev_ptr = nullptr;
    return rc;
  }
  return MIAIE_OK;
}

extern "C" int miaie_free(miaie_ctx* ctx, void* dev_ptr) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_free"))) return rc;
  if (!dev_ptr) return MIAIE_OK;
  if ((rc = dbg_remove(ctx, dev_ptr))) return rc;
  hipError_t e = hipFree(dev_ptr);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
  return MIAIE_OK;
}

extern "C" int miaie_copy_h2d(miaie_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_copy_h2d"))) return rc;
  if (bytes == 0) return MIAIE_OK;
  MIAIE_CHECK_NOT_NULL(ctx, dst);
  MIAIE_CHECK_NOT_NULL(ctx, src);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMemcpyAsync(H2D)");
  e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return MIAIE_OK;
}

extern "C" int miaie_copy_d2h(miaie_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_copy_d2h"))) return rc;
  if (bytes == 0) return MIAIE_OK;
  MIAIE_CHECK_NOT_NULL(ctx, dst);
  MIAIE_CHECK_NOT_NULL(ctx, src);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMemcpyAsync(D2H)");
  e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return MIAIE_OK;
}

extern "C" int miaie_copy_d2d(miaie_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (bytes == 0) return MIAIE_OK;
  MIAIE_CHECK_NOT_NULL(ctx, dst);
  MIAIE_CHECK_NOT_NULL(ctx, src);
  const bool vec_ok = aligned(dst, 16) && aligned(src, 16);
  const size_t nvec = vec_ok ? bytes / 16 : 0;
  const size_t done = nvec * 16;
  const size_t ntail = bytes - done;
  if (ntail > (size_t)1 << 30) return fail(ctx, MIAIE_EINVAL, "miaie_copy_d2d: unaligned copies are limited to 1 GiB");
  size_t threads_needed = nvec > ntail ? nvec : ntail;
  size_t blocks = (threads_needed + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < (ntail + 255) / 256) blocks = (ntail + 255) / 256;
  if (blocks == 0) blocks = 1;
  const hipError_t e = launch<copy_kernel>(ctx->device, dim3((unsigned)blocks), dim3(256), 0, ctx->stream,
                                           static_cast<v4i*>(dst), static_cast<const v4i*>(src), nvec,
                                           static_cast<uint8_t*>(dst) + done, static_cast<const uint8_t*>(src) + done,
                                           ntail);
  return check_launch(ctx, e, "copy_kernel");
}

// ---------------------------------------------------------------- waits
extern "C" int miaie_wait(miaie_ctx* ctx, int timeout_ms) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_wait"))) return rc;
  hipError_t e = hipEventRecord(ctx->done, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
  if (timeout_ms < 0) {
    e = hipEventSynchronize(ctx->done);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventSynchronize");
    return dbg_take_faults(ctx);
  }
  timespec t0;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (;;) {
    e = hipEventQuery(ctx->done);
    if (e == hipSuccess) return dbg_take_faults(ctx);
    if (e != hipErrorNotReady) return hip_fail(ctx, e, "hipEventQuery");
    timespec t1;
    clock_gettime(CLOCK_MONOTONIC, &t1);
    double ms = (t1.tv_sec - t0.tv_sec) * 1e3 + (t1.tv_nsec - t0.tv_nsec) * 1e-6;
    if (ms >= timeout_ms)
      return fail(ctx, MIAIE_ETIMEDOUT, "miaie_wait: stream not drained after %d ms", timeout_ms);
    // poll without sleeping for the first 0.2 ms (a short kernel finishes
    // within a few microseconds and a 20 us nap would dominate), then nap
    if (ms >= 0.2) {
      timespec nap = {0, 20000};  // 20 us
      nanosleep(&nap, nullptr);
    }
  }
}

// ---------------------------------------------------------------- device bounds checks
extern "C" int miaie_debug_device_checks(void) { return MIAIE_DEVICE_CHECKS ? 1 : 0; }

extern "C" int miaie_debug_register(miaie_ctx* ctx, const void* dev_ptr, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_debug_register"))) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, dev_ptr);
  if (bytes == 0) return fail(ctx, MIAIE_EINVAL, "miaie_debug_register: zero bytes");
  return dbg_add(ctx, dev_ptr, bytes);
}

extern "C" int miaie_debug_unregister(miaie_ctx* ctx, const void* dev_ptr) {
  int rc = enter(ctx);
  if (rc) return rc;
  if ((rc = refuse_while_recording(ctx, "miaie_debug_unregister"))) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, dev_ptr);
  return dbg_remove(ctx, dev_ptr);
}

// ---------------------------------------------------------------- synthetic data
extern "C" int miaie_fill_i8(miaie_ctx* ctx, int8_t* dst, size_t n, uint64_t tensor_id) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (n == 0) return MIAIE_OK;
  MIAIE_CHECK_NOT_NULL(ctx, dst);
  if (!aligned(dst, 16)) return fail(ctx, MIAIE_EINVAL, "miaie_fill_i8: dst must be 16-byte aligned");
  const uint64_t state0 = sm64_mix(0x5EED0000ull + tensor_id + kGamma);
  const size_t threads = (n + 15) / 16;
  const size_t blocks = (threads + 255) / 256;
  if (blocks > 0x7FFFFFFF) return fail(ctx, MIAIE_EINVAL, "miaie_fill_i8: n too large");
  return check_launch(ctx, launch<fill_i8_kernel>(ctx->device, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, dst, n, state0),
                      "fill_i8_kernel");
}

extern "C" const char* miaie_version(void) { return "miaie 0.1 (gfx950)"; }

// ---------------------------------------------------------------- GEMM plan
extern "C" int miaie_plan_gemm_i8(miaie_ctx* ctx, int M, int N, int K, miaie_gemm_plan* plan) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, plan);
  if (M < 1 || N < 1 || K < 1) return fail(ctx, MIAIE_EINVAL, "miaie_plan_gemm_i8: M=%d N=%d K=%d", M, N, K);
  // the operand conditions of miaie_gemm_i8_rq on dense NN operands (lda = K,
  // ldb = ldy = N): 16-byte rows, strides below 2^25, and K < 2^16 for the
  // requantizing epilogue's shortcut
  return plan_gemm_i8(ctx, M, N, K, (K % 16 == 0) && (N % 16 == 0) && K < (1 << 16) && N < (1 << 25), plan);
}

extern "C" int miaie_plan_set_cus(miaie_ctx* ctx, int cus, int* previous) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (cus < 1) return fail(ctx, MIAIE_EINVAL, "miaie_plan_set_cus: cus=%d", cus);
  if (previous) *previous = ctx->cus;
  ctx->cus = cus;
  return MIAIE_OK;
}

// ---------------------------------------------------------------- recorded chains
struct miaie_graph {
  unsigned long long ctx_id = 0;  // the recording context: its workspace may be baked into the graph
  int device = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  size_t nodes = 0;
};

extern "C" int miaie_graph_begin(miaie_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (ctx->recording) return fail(ctx, MIAIE_EINVAL, "miaie_graph_begin: already recording");
  if (!ctx->stream)
    return fail(ctx, MIAIE_EUNSUPPORTED, "miaie_graph_begin: the null stream cannot be recorded; use miaie_init");
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamBeginCapture");
  ctx->recording = true;
  return MIAIE_OK;
}

extern "C" int miaie_graph_end(miaie_ctx* ctx, miaie_graph** out) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (!ctx->recording) return fail(ctx, MIAIE_EINVAL, "miaie_graph_end: not recording (miaie_graph_begin)");
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &g);
  ctx->recording = false;
  if (e != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return hip_fail(ctx, e, "hipStreamEndCapture");
  }
  if (!out) {
    (void)hipGraphDestroy(g);
    return fail(ctx, MIAIE_EINVAL, "miaie_graph_end: graph is NULL (the recording is discarded)");
  }
  *out = nullptr;
  miaie_graph* mg = new (std::nothrow) miaie_graph;
  if (!mg) {
    (void)hipGraphDestroy(g);
    return fail(ctx, MIAIE_ENOMEM, "miaie_graph_end: host allocation failed");
  }
  mg->ctx_id = ctx->id;
  mg->device = ctx->device;
  mg->graph = g;
  (void)hipGraphGetNodes(g, nullptr, &mg->nodes);
  if (mg->nodes == 0) {
    (void)hipGraphDestroy(g);
    delete mg;
    return fail(ctx, MIAIE_EINVAL, "miaie_graph_end: nothing was recorded");
  }
  e = hipGraphInstantiate(&mg->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    delete mg;
    return hip_fail(ctx, e, "hipGraphInstantiate");
  }
  *out = mg;
  return MIAIE_OK;
}

extern "C" int miaie_graph_launch(miaie_ctx* ctx, miaie_graph* graph) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, graph);
  if (ctx->recording) return fail(ctx, MIAIE_EINVAL, "miaie_graph_launch: cannot replay into a recording");
  if (graph->ctx_id != ctx->id)
    return fail(ctx, MIAIE_EINVAL,
                "miaie_graph_launch: the graph was recorded on another context (it may use that context's "
                "workspace); replay it on the context that recorded it");
  hipError_t e = hipGraphLaunch(graph->exec, ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphLaunch");
  return MIAIE_OK;
}

extern "C" int miaie_graph_destroy(miaie_graph* graph) {
  if (!graph) return MIAIE_OK;
  (void)hipSetDevice(graph->device);
  int rc = MIAIE_OK;
  if (graph->exec && hipGraphExecDestroy(graph->exec) != hipSuccess) rc = MIAIE_EHIP;
  if (graph->graph && hipGraphDestroy(graph->graph) != hipSuccess) rc = MIAIE_EHIP;
  delete graph;
  return rc;
}
