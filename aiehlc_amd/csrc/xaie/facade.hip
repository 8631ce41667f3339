// libmiaie_xaie.so: the aie-rt-shaped host facade (include/miaie_xaie.h)
// over the miaie runtime, plus the tile-array kernels XAie_Run launches.
//
// The array's tile data memories live in one HBM slab; a run of N tiles that
// share a kernel is one launch of N workgroups, workgroup b working inside
// tile b's memory.  Each kernel restates one of the reference examples'
// `__global__` functions (cited at the kernel).
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cstddef>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "../../../include/miaie.h"
#include "../../../include/miaie_xaie.h"

namespace {

constexpr u32 kCoreMemAie1 = 32u << 10;   // AIE1 core tile data memory
constexpr u32 kCoreMem = 64u << 10;       // AIE-ML / AIE2PS core tile data memory
constexpr u32 kMemTileMem = 512u << 10;   // memory tile
constexpr u32 kMaxRunTiles = 320;         // tiles in one launch (kernel argument block; a 38x8 array of cores fits)
constexpr u32 kDefaultWaitUs = 500;

enum Builtin : u32 { B_NONE = 0, B_MM_NT = 1, B_K1 = 2, B_K2 = 3, B_MM3_U64 = 4, B_DOT_U8 = 5 };

// ---------------------------------------------------------------- tile kernels
template <int CAP>
struct TileListT {
  u32 n;
  u32 off[CAP];
};
using TileList = TileListT<kMaxRunTiles>;

// A single-tile launch of a built-in carries the tile's queued host -> tile
// copies and a request to mirror its output window into pinned host memory,
// so that the flow "move in, run, wait, move out" is one launch: the copies
// run in the kernel's prologue (reading the pinned staging buffer over PCIe),
// the output window is copied to the host shadow in its epilogue, and `seq`
// is published in a host flag once both are there.
// Copies whose bytes fit kFuseInline travel inside the kernel arguments
// (which the runtime places in device memory) instead of being read from
// the pinned staging buffer over PCIe; the whole argument block (tile list,
// these, the scalars) stays under 4 KiB.
constexpr int kFuseCopies = 4;
constexpr u32 kFuseInline = 2048;
constexpr u32 kNotInline = ~0u;
template <u32 INL>
struct FuseArgsT {
  u32 ncopy;
  u32 dst[kFuseCopies];              // tile-relative byte offsets
  u32 size[kFuseCopies];
  u32 inl_off[kFuseCopies];          // offset of the bytes in inl, or kNotInline
  const uint8_t* src[kFuseCopies];   // pinned staging (copies not inline)
  uint8_t* shadow;                   // pinned host mirror of the output window, or null
  u32 shadow_addr, shadow_size;
  uint32_t* flag;                    // host word that receives seq, or null
  uint32_t seq;
  alignas(16) uint8_t inl[INL];
};
// The host builds the full form; a launch sends the smallest that holds its
// inline bytes.  The argument block is copied to the device on every launch:
// a 0.9 KB block measured about 1 us per launch faster than a 3.5 KB one.
using FuseArgs = FuseArgsT<kFuseInline>;
template <u32 INL>
FuseArgsT<INL> shrink(const FuseArgs& f) {
  FuseArgsT<INL> g;
  g.ncopy = f.ncopy;
  for (int c = 0; c < kFuseCopies; ++c) {
    g.dst[c] = f.dst[c];
    g.size[c] = f.size[c];
    g.inl_off[c] = f.inl_off[c];
    g.src[c] = f.src[c];
  }
  g.shadow = f.shadow;
  g.shadow_addr = f.shadow_addr;
  g.shadow_size = f.shadow_size;
  g.flag = f.flag;
  g.seq = f.seq;
  memcpy(g.inl, f.inl, INL);
  return g;
}

__device__ void block_copy(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, u32 n) {
  if ((((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
    for (u32 i = threadIdx.x; i < n / 16; i += blockDim.x)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    for (u32 i = n / 16 * 16 + threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
  } else {
    for (u32 i = threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
  }
}

// `inl` points at f.inl where the kernel argument segment holds it (read in
// place: indexing the by-value argument itself would copy it to scratch).
template <typename F>
__device__ void fuse_in(uint8_t* base, const F& f, const uint8_t* inl) {
#pragma unroll
  for (int c = 0; c < kFuseCopies; ++c)
    if ((u32)c < f.ncopy)
      block_copy(base + f.dst[c], f.inl_off[c] != kNotInline ? inl + f.inl_off[c] : f.src[c], f.size[c]);
  __syncthreads();
}

// The tile kernels take one argument block each, so the argument segment
// starts with it and its inline bytes sit at a fixed offset.
template <int CAP, u32 INL>
struct MmArgs {
  uint8_t* mem;
  TileListT<CAP> tl;
  u32 in_addr, out_addr;
  int n;
  u32 passes;
  FuseArgsT<INL> fz;
};
template <int CAP, u32 INL>
struct AddArgs {
  uint8_t* mem;
  TileListT<CAP> tl;
  u32 in_addr, out_addr;
  int addend;
  u32 passes;
  FuseArgsT<INL> fz;
};
template <typename Args>
__device__ __forceinline__ const uint8_t* kernarg_inline() {
#if __HIP_DEVICE_COMPILE__  // the builtin exists in the device pass only
  return reinterpret_cast<const uint8_t*>(__builtin_amdgcn_kernarg_segment_ptr()) + offsetof(Args, fz) +
         offsetof(decltype(Args::fz), inl);
#else
  return nullptr;
#endif
}

template <typename F>
__device__ void fuse_out(uint8_t* base, const F& f) {
  __syncthreads();
  if (f.shadow) block_copy(f.shadow, base + f.shadow_addr, f.shadow_size);
  if (f.flag) {
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(f.flag, f.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// `mm` (aieml_mm.cc:41-93) and `perf` (aieml_perf.cc:61-83): the input
// window holds A[n][n] then B as [n][k] (n*n words each); out[i][j] =
// sum_k A[i][k] * B[j][k] in 32-bit wrap-around arithmetic.  n <= 16, so one
// workgroup of 256 lanes covers a tile's whole output.
// The window is read from tile memory into LDS once, all words in flight
// together, so the k-loop does not wait on a global load per step.
template <int CAP, u32 INL>
__global__ __launch_bounds__(256) void tile_mm_nt(MmArgs<CAP, INL> args) {
  const u32 in_addr = args.in_addr, out_addr = args.out_addr, passes = args.passes;
  const int n = args.n;
  const auto& fz = args.fz;
  __shared__ uint32_t win[2 * 16 * 16];
  uint8_t* base = args.mem + args.tl.off[blockIdx.x];
  fuse_in(base, fz, kernarg_inline<MmArgs<CAP, INL>>());
  const uint32_t* in = reinterpret_cast<const uint32_t*>(base + in_addr);
  const int t = threadIdx.x;
  for (int w = t; w < 2 * n * n; w += blockDim.x) win[w] = in[w];
  __syncthreads();
  const uint32_t* a = win;
  const uint32_t* bt = win + n * n;
  uint32_t* out = reinterpret_cast<uint32_t*>(base + out_addr);
  if (t < n * n) {
    const int i = t / n, j = t - i * n;
    for (u32 p = 0; p < passes; ++p) {
      uint32_t acc = 0;
      for (int k = 0; k < n; ++k) acc += a[i * n + k] * bt[j * n + k];
      out[t] = acc;
    }
  }
  fuse_out(base, fz);
}

// `k1` / `k2` (multi_tile.cpp:39-47, seq_full_col.cpp:39-47): 20 words of
// out = in[0] + addend.
template <int CAP, u32 INL>
__global__ __launch_bounds__(64) void tile_add20(AddArgs<CAP, INL> args) {
  const u32 in_addr = args.in_addr, out_addr = args.out_addr, passes = args.passes;
  const int addend = args.addend;
  const auto& fz = args.fz;
  uint8_t* base = args.mem + args.tl.off[blockIdx.x];
  fuse_in(base, fz, kernarg_inline<AddArgs<CAP, INL>>());
  const int32_t* in = reinterpret_cast<const int32_t*>(base + in_addr);
  int32_t* out = reinterpret_cast<int32_t*>(base + out_addr);
  if (threadIdx.x < 20)
    for (u32 p = 0; p < passes; ++p) out[threadIdx.x] = (int32_t)((uint32_t)in[0] + (uint32_t)addend);
  fuse_out(base, fz);
}

// `mm` of vek385_verification.cpp:56-69: out = in . in over 3x3 uint64, the
// sum kept in the kernel's `int` (so wrapped to 32 bits and sign-extended),
// and out[9] = number of passes completed.
__global__ __launch_bounds__(64) void tile_mm3_u64(uint8_t* __restrict__ mem, TileList tl, u32 in_addr, u32 out_addr,
                                                   u32 passes) {
  uint8_t* base = mem + tl.off[blockIdx.x];
  const uint64_t* in = reinterpret_cast<const uint64_t*>(base + in_addr);
  uint64_t* out = reinterpret_cast<uint64_t*>(base + out_addr);
  const int t = threadIdx.x;
  for (u32 p = 0; p < passes; ++p) {
    if (t < 9) {
      const int i = t / 3, j = t % 3;
      uint32_t sum = 0;
      for (int k = 0; k < 3; ++k) sum += (uint32_t)(in[i * 3 + k] * in[k * 3 + j]);
      out[t] = (uint64_t)(int64_t)(int32_t)sum;
    }
    __syncthreads();
    if (t == 0) out[9] = (uint64_t)p + 1;
    __syncthreads();
  }
}

// Host <-> tile copy through the pinned staging buffer, which this kernel
// reads or writes over PCIe directly: small moves skip the DMA engine, whose
// per-copy start-up latency is most of their cost.  16-byte words when both
// ends are 16-byte aligned, bytes otherwise.  With `flag` (host memory), one
// workgroup copies everything and then publishes `seq` there, after a
// system-scope fence, so the host can read the bytes as soon as they have
// landed instead of waiting for the kernel's completion signal.
__global__ __launch_bounds__(256) void stage_copy(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                  size_t n, uint32_t* flag, uint32_t seq) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if ((((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
    const size_t nv = n / 16;
    for (size_t i = t0; i < nv; i += stride)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    for (size_t i = nv * 16 + t0; i < n; i += stride) dst[i] = src[i];
  } else {
    for (size_t i = t0; i < n; i += stride) dst[i] = src[i];
  }
  if (flag) {
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

}  // namespace

// ---------------------------------------------------------------- built-in descriptors
extern "C" {
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_mm = {
    MIAIE_XAIE_KERNEL_MAGIC, "mm", 2, {0x1000, 0x6000}, {512, 512}, 0, nullptr, nullptr, B_MM_NT};
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_mm8 = {
    MIAIE_XAIE_KERNEL_MAGIC, "mm", 2, {0x1000, 0x6000}, {128, 128}, 0, nullptr, nullptr, B_MM_NT};
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_perf = {
    MIAIE_XAIE_KERNEL_MAGIC, "perf", 2, {0x1000, 0x6000}, {512, 512}, 0, nullptr, nullptr, B_MM_NT};
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_k1 = {
    MIAIE_XAIE_KERNEL_MAGIC, "k1", 2, {0, 0}, {0, 0}, 0, nullptr, nullptr, B_K1};
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_k2 = {
    MIAIE_XAIE_KERNEL_MAGIC, "k2", 2, {0, 0}, {0, 0}, 0, nullptr, nullptr, B_K2};
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_mm3_u64 = {
    MIAIE_XAIE_KERNEL_MAGIC, "mm3_u64", 2, {0, 0}, {0, 0}, MIAIE_XAIE_KERNEL_FOREVER, nullptr, nullptr, B_MM3_U64};
MIAIE_XAIE_API const XAie_MiaieKernel miaie_xaie_perf_u8 = {
    MIAIE_XAIE_KERNEL_MAGIC, "perf_u8", 2, {0x1000, 0x6000}, {512, 512}, 0, nullptr, nullptr, B_DOT_U8};
}

namespace {

// Bytes each built-in reads or writes from the start of each window, for the
// load-time bounds check (a launch never touches memory outside its tile).
u32 builtin_extent(const XAie_MiaieKernel* k, u32 param, u32 arg) {
  switch (k->Builtin) {
    case B_MM_NT: return param == 0 ? 2 * arg * arg * 4 : arg * arg * 4;
    case B_K1:
    case B_K2: return param == 0 ? 4 : 20 * 4;
    case B_MM3_U64: return param == 0 ? 9 * 8 : 10 * 8;
    case B_DOT_U8: return param == 0 ? 4 : 5 * 4;
    default: return 0;
  }
}

thread_local std::string g_last_error;

// Every entry point runs inside a function-try-block: a host allocation that
// fails in the bookkeeping (std::bad_alloc) becomes XAIE_ERR (or NULL), not an
// exception crossing the C ABI.
AieRC out_of_memory(const char* fn) noexcept {
  try {
    g_last_error = std::string(fn) + ": out of host memory";
  } catch (...) {
  }
  return XAIE_ERR;
}
std::vector<miaie_xaie_dev*> g_devices;  // initialised instances, for XAie_MiaieRunOnDdr

enum TileKind { T_NONE, T_SHIM, T_MEM, T_CORE };

struct Core {
  const XAie_MiaieKernel* k = nullptr;
  u32 arg = 16;            // n of the mm kernels
  bool reset = true;
  bool enabled = false;
  bool pending = false;    // enabled, launch not issued yet
  bool ran = false;
  uint64_t seq = 0;        // launch batch of the last run
  bool fused = false;      // the last run was a fused single-tile launch ...
  uint32_t fused_seq = 0;  // ... that publishes this number in the host done flag
};

struct PendCopy {          // a staged host -> tile copy not yet issued
  int tile;
  uint64_t addr;
  const uint8_t* src;      // slice of the pinned staging buffer
  size_t size;
};

struct Shadow {            // pinned host mirror of a tile's output window
  bool valid = false;
  uint64_t addr = 0;
  u32 size = 0;
  uint32_t seq = 0;        // fused launch that writes it
};

struct Route {
  u16 src, dst;  // tile index (col * rows + row)
};

}  // namespace

struct XAie_MemInst {
  miaie_xaie_dev* dev;
  uint8_t* host;
  size_t size;
  size_t mapped;  // bytes mmapped (0: malloc)
};

struct XAie_RoutingInstance {
  XAie_DevInst* dev;
  std::vector<Route> routes;
};

struct miaie_xaie_dev {
  miaie_ctx* ctx = nullptr;
  hipStream_t stream = nullptr;
  int device = 0;
  uint8_t* mem = nullptr;  // tile-memory slab
  size_t mem_bytes = 0;
  u32 cols = 0, rows = 0;
  std::vector<TileKind> kind;
  std::vector<u32> off, bytes;
  std::vector<Core> cores;
  std::vector<XAie_MemInst*> ddr;
  std::vector<XAie_RoutingInstance*> routing;
  std::deque<std::pair<uint64_t, hipEvent_t>> inflight;  // launch batches not yet seen complete
  std::vector<hipEvent_t> spare;
  uint64_t issued = 0, completed = 0;
  uint8_t* stage = nullptr;        // pinned, coherent host staging for host <-> tile copies
  uint32_t* stage_flag = nullptr;  // after it: tile -> host copies publish their sequence number here
  uint32_t stage_seq = 0;
  uint32_t* done_flag = nullptr;   // fused launches publish their sequence number here
  uint32_t fuse_seq = 0;
  uint8_t* shadow_mem = nullptr;   // after the flags: kShadowSlot bytes per tile
  std::vector<PendCopy> pend;      // host -> tile copies waiting for the next launch
  std::vector<Shadow> shadow;      // per tile
  size_t stage_used = 0;           // bytes of it taken since the stream last drained
  hipEvent_t stage_ev = nullptr;   // recorded after the latest staged host -> tile copy
  XAie_BackendType backend = XAIE_IO_BACKEND_BAREMETAL;
  std::string err;
};

namespace {

const XAie_Backend kBackends[] = {
    {XAIE_IO_BACKEND_BAREMETAL, "miaie-hip (baremetal calls)"},
    {XAIE_IO_BACKEND_LINUX, "miaie-hip (linux calls)"},
    {XAIE_IO_BACKEND_MIAIE_HIP, "miaie-hip"},
};

AieRC fail(miaie_xaie_dev* d, AieRC rc, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
AieRC fail(miaie_xaie_dev* d, AieRC rc, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  if (d) d->err = buf;
  return rc;
}

AieRC hip_fail(miaie_xaie_dev* d, hipError_t e, const char* what) {
  return fail(d, XAIE_ERR, "%s: %s", what, hipGetErrorString(e));
}

AieRC miaie_fail(miaie_xaie_dev* d, int rc, const char* what) {
  return fail(d, rc == MIAIE_EINVAL ? XAIE_INVALID_ARGS : XAIE_ERR, "%s: %s (status %d)", what,
              miaie_last_error_string(d ? d->ctx : nullptr), rc);
}

miaie_xaie_dev* dev_of(XAie_DevInst* inst) {
  if (!inst || !inst->IsReady || !inst->Priv) {
    fail(nullptr, XAIE_INVALID_DEVICE, "device instance is NULL or not initialised (XAie_CfgInitialize)");
    return nullptr;
  }
  hipError_t e = hipSetDevice(inst->Priv->device);
  if (e != hipSuccess) {
    hip_fail(inst->Priv, e, "hipSetDevice");
    return nullptr;
  }
  return inst->Priv;
}

// Tile index of a location, or -1 outside the partition.
int tile_index(const miaie_xaie_dev* d, XAie_LocType loc) {
  if (loc.Col >= d->cols || loc.Row >= d->rows) return -1;
  return (int)(loc.Col * d->rows + loc.Row);
}

AieRC core_of(miaie_xaie_dev* d, XAie_LocType loc, const char* what, int* idx) {
  const int t = tile_index(d, loc);
  if (t < 0) return fail(d, XAIE_INVALID_TILE, "%s: tile (%u, %u) is outside the %ux%u partition", what, loc.Col,
                         loc.Row, d->cols, d->rows);
  if (d->kind[t] != T_CORE)
    return fail(d, XAIE_INVALID_TILE, "%s: tile (%u, %u) has no core (shim or memory tile)", what, loc.Col, loc.Row);
  *idx = t;
  return XAIE_OK;
}

// Move completed launch batches off the in-flight list.
void retire(miaie_xaie_dev* d) {
  while (!d->inflight.empty()) {
    auto& f = d->inflight.front();
    if (hipEventQuery(f.second) != hipSuccess) break;
    d->completed = f.first;
    d->spare.push_back(f.second);
    d->inflight.pop_front();
  }
}

AieRC record_batch(miaie_xaie_dev* d, uint64_t* seq) {
  hipEvent_t ev;
  if (!d->spare.empty()) {
    ev = d->spare.back();
    d->spare.pop_back();
  } else {
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(d, e, "hipEventCreateWithFlags");
  }
  hipError_t e = hipEventRecord(ev, d->stream);
  if (e != hipSuccess) {
    d->spare.push_back(ev);
    return hip_fail(d, e, "hipEventRecord");
  }
  *seq = ++d->issued;
  d->inflight.emplace_back(*seq, ev);
  // bound the list: a harness that never waits still reuses events
  if (d->inflight.size() > 256) {
    (void)hipEventSynchronize(d->inflight.front().second);
    retire(d);
  }
  return XAIE_OK;
}

// Window addresses of a kernel (the reference compiler's placement rule).
// n of an mm-type kernel: its input window holds A and B, 2 n^2 words, so a
// size_hint of 2 n^2 (n <= 16) fixes n; otherwise the examples' 16.
u32 window_n(const XAie_MiaieKernel* k) {
  if (k->Builtin == B_MM_NT)
    for (u32 n = 1; n <= 16; ++n)
      if (k->SizeHint[0] == 2 * n * n) return n;
  return 16;
}

void window_layout(const XAie_MiaieKernel* k, u32* ping, u32* pong) {
  u32 addr = 0x1000;
  for (u32 i = 0; i < k->NumParams; ++i) {
    const u32 words = 4 * (k->SizeHint[i] ? k->SizeHint[i] : 512);
    if (k->MemAddress[i]) addr = k->MemAddress[i];
    if (ping) ping[i] = addr;
    const u32 p = addr + words * 4;
    if (pong) pong[i] = p;
    addr = p + words * 4;
  }
}

AieRC valid_kernel(miaie_xaie_dev* d, const void* p, const XAie_MiaieKernel** out) {
  const XAie_MiaieKernel* k = static_cast<const XAie_MiaieKernel*>(p);
  if (!k) return fail(d, XAIE_INVALID_ELF, "kernel is NULL");
  if (k->Magic != MIAIE_XAIE_KERNEL_MAGIC)
    return fail(d, XAIE_INVALID_ELF, "not an XAie_MiaieKernel descriptor (magic 0x%08x)", k->Magic);
  if (k->NumParams > MIAIE_XAIE_MAX_PARAMS)
    return fail(d, XAIE_INVALID_ELF, "kernel %s: %u parameters, at most %d", k->Name ? k->Name : "?", k->NumParams,
                MIAIE_XAIE_MAX_PARAMS);
  if (k->Builtin == B_NONE && !k->Launch)
    return fail(d, XAIE_INVALID_ELF, "kernel %s: no launch function", k->Name ? k->Name : "?");
  if (k->Builtin > B_DOT_U8) return fail(d, XAIE_INVALID_ELF, "kernel %s: unknown built-in", k->Name ? k->Name : "?");
  if (k->Builtin != B_NONE && k->NumParams != 2)
    return fail(d, XAIE_INVALID_ELF, "built-in kernel %s must have 2 parameters", k->Name ? k->Name : "?");
  *out = k;
  return XAIE_OK;
}

// Every window of `k` (with mm size `arg`) fits a core tile's data memory.
AieRC check_windows(miaie_xaie_dev* d, const XAie_MiaieKernel* k, u32 arg, u32 tile_bytes) {
  u32 ping[MIAIE_XAIE_MAX_PARAMS], pong[MIAIE_XAIE_MAX_PARAMS];
  window_layout(k, ping, pong);
  for (u32 i = 0; i < k->NumParams; ++i) {
    const u32 need = k->Builtin ? builtin_extent(k, i, arg) : 4 * 4 * (k->SizeHint[i] ? k->SizeHint[i] : 512);
    if ((uint64_t)ping[i] + need > tile_bytes)
      return fail(d, XAIE_INVALID_DATA_MEM_ADDR, "kernel %s: window %u at 0x%x (+%u B) exceeds the %u B data memory",
                  k->Name ? k->Name : "?", i, ping[i], need, tile_bytes);
  }
  return XAIE_OK;
}

// Host <-> tile copies up to kStageBytes go through a pinned, coherent
// staging buffer that the GPU reads and writes directly.
//   host -> tile: the source bytes are copied into a slice of the buffer and
//     the copy is queued.  The next single-tile launch of a built-in on that
//     tile carries it in its prologue (one launch for "move in, run"); any
//     other operation first issues the queued copies as copy kernels.  Either
//     way the device copy runs in stream order ahead of later work, as an AIE
//     DMA runs on after XAie_MoveData returns (the perf example waits for it
//     with XAie_RouteDmaWait, aieml_perf.cc:156-163).
//   tile -> host: returns once the bytes are in the destination.  A range
//     inside the output window of the tile's last fused launch is read from
//     that launch's host shadow once its done flag is up; otherwise a copy
//     kernel writes the staging buffer and publishes a flag.
// Larger copies take the synchronous miaie copies.  Staged slices are taken
// consecutively; when the buffer is full, the stream is drained and it starts
// over.
constexpr size_t kStageBytes = 4u << 20;
constexpr size_t kShadowSlot = 4u << 10;  // largest output window mirrored per tile

AieRC ensure_stage(miaie_xaie_dev* d) {
  hipError_t e = hipSetDevice(d->device);
  if (e != hipSuccess) return hip_fail(d, e, "hipSetDevice");
  if (!d->stage) {
    const size_t bytes = kStageBytes + 256 + kShadowSlot * d->cores.size();
    e = hipHostMalloc(reinterpret_cast<void**>(&d->stage), bytes, hipHostMallocCoherent);
    if (e != hipSuccess) {
      d->stage = nullptr;
      return hip_fail(d, e, "pinned staging buffer");
    }
    d->stage_flag = reinterpret_cast<uint32_t*>(d->stage + kStageBytes);
    d->done_flag = d->stage_flag + 1;
    d->shadow_mem = d->stage + kStageBytes + 256;
    __atomic_store_n(d->stage_flag, d->stage_seq = 0, __ATOMIC_RELEASE);
    __atomic_store_n(d->done_flag, d->fuse_seq = 0, __ATOMIC_RELEASE);
    d->stage_used = 0;
  }
  if (!d->stage_ev) {
    e = hipEventCreateWithFlags(&d->stage_ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      d->stage_ev = nullptr;
      return hip_fail(d, e, "hipEventCreate");
    }
  }
  return XAIE_OK;
}

unsigned stage_blocks(size_t size) { return (unsigned)std::min<size_t>((size + 4095) / 4096, 1024); }

// Issue the queued host -> tile copies as copy kernels.
AieRC issue_pending(miaie_xaie_dev* d) {
  if (d->pend.empty()) return XAIE_OK;
  hipError_t e = hipSuccess;
  for (const PendCopy& c : d->pend) {
    stage_copy<<<stage_blocks(c.size), 256, 0, d->stream>>>(d->mem + d->off[c.tile] + c.addr, c.src, c.size, nullptr,
                                                            0);
    e = hipGetLastError();
    if (e != hipSuccess) break;
  }
  d->pend.clear();
  if (e == hipSuccess) e = hipEventRecord(d->stage_ev, d->stream);
  return e == hipSuccess ? XAIE_OK : hip_fail(d, e, "host to tile copy");
}

AieRC stage_take(miaie_xaie_dev* d, size_t size, uint8_t** slice) {
  if (AieRC rc = ensure_stage(d)) return rc;
  const size_t need = (size + 255) & ~static_cast<size_t>(255);
  if (d->stage_used + need > kStageBytes) {
    if (AieRC rc = issue_pending(d)) return rc;
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return hip_fail(d, e, "waiting for staged copies");
    d->stage_used = 0;
  }
  *slice = d->stage + d->stage_used;
  d->stage_used += need;
  return XAIE_OK;
}

// Anything that writes a tile's memory outside a fused launch makes its
// shadow stale.
void invalidate_shadow(miaie_xaie_dev* d, int t) {
  if (t >= 0 && (size_t)t < d->shadow.size()) d->shadow[t].valid = false;
}

AieRC copy_h2d(miaie_xaie_dev* d, int t, uint64_t addr, const void* src, size_t size) {
  if (size == 0) return XAIE_OK;
  invalidate_shadow(d, t);
  if (size <= kStageBytes) {
    if (d->pend.size() >= (size_t)kFuseCopies)
      if (AieRC rc = issue_pending(d)) return rc;
    uint8_t* st = nullptr;
    if (AieRC rc = stage_take(d, size, &st)) return rc;
    std::memcpy(st, src, size);
    d->pend.push_back(PendCopy{t, addr, st, size});
    return XAIE_OK;
  }
  if (AieRC rc = issue_pending(d)) return rc;
  const int rc = miaie_copy_h2d(d->ctx, d->mem + d->off[t] + addr, src, size);
  return rc ? miaie_fail(d, rc, "host to tile copy") : XAIE_OK;
}

// Spin until the host word `flag` reaches `seq` (wrap-safe), for up to
// kFlagSpinUs; false if it did not.
constexpr int kFlagSpinUs = 2000;
bool spin_flag(const uint32_t* flag, uint32_t seq) {
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(kFlagSpinUs);
  for (;;) {
    if ((int32_t)(__atomic_load_n(flag, __ATOMIC_ACQUIRE) - seq) >= 0) return true;
    if (std::chrono::steady_clock::now() >= deadline) return false;
  }
}

// Tile -> host copies up to kFlagCopyBytes run in one workgroup that
// publishes a sequence number in the staging buffer's flag word once the
// bytes are there; the host spins on it and then falls back to waiting for
// the stream (which also reports a failed launch).
constexpr size_t kFlagCopyBytes = 64u << 10;

AieRC copy_d2h(miaie_xaie_dev* d, int t, uint64_t addr, void* dst, size_t size) {
  if (size == 0) return XAIE_OK;
  const Shadow& sh = d->shadow[t];
  if (sh.valid && addr >= sh.addr && addr + size <= sh.addr + sh.size) {
    if (!spin_flag(d->done_flag, sh.seq)) {
      if (AieRC rc = issue_pending(d)) return rc;
      hipError_t e = hipStreamSynchronize(d->stream);
      if (e != hipSuccess) return hip_fail(d, e, "tile to host copy");
    }
    std::memcpy(dst, d->shadow_mem + (size_t)t * kShadowSlot + (addr - sh.addr), size);
    return XAIE_OK;
  }
  if (AieRC rc = issue_pending(d)) return rc;
  if (size <= kStageBytes) {
    uint8_t* st = nullptr;
    if (AieRC rc = stage_take(d, size, &st)) return rc;
    const bool flagged = size <= kFlagCopyBytes;
    const uint32_t seq = ++d->stage_seq;
    stage_copy<<<flagged ? 1u : stage_blocks(size), 256, 0, d->stream>>>(st, d->mem + d->off[t] + addr, size,
                                                                          flagged ? d->stage_flag : nullptr, seq);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && !(flagged && spin_flag(d->stage_flag, seq))) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return hip_fail(d, e, "tile to host copy");
    std::memcpy(dst, st, size);
    // Every copy queued before this one has completed (the queue was issued
    // first, and this copy ran after it), and this one reads no staged bytes,
    // so the whole buffer is free again.
    d->stage_used = 0;
    return XAIE_OK;
  }
  const int rc = miaie_copy_d2h(d->ctx, dst, d->mem + d->off[t] + addr, size);
  return rc ? miaie_fail(d, rc, "tile to host copy") : XAIE_OK;
}

// XAie_RouteDmaWait: a host -> tile transfer is complete, as far as any
// caller can tell, once its bytes are staged.  The source buffer may be
// reused from then on, and every later access to tile memory (a launch, a
// read, another copy) runs after the device copy in stream order, so there
// is nothing left to wait for; a queued copy stays queued for the next
// launch to carry.
AieRC staged_copies_done(miaie_xaie_dev* d) {
  (void)d;
  return XAIE_OK;
}

// Launch `k` on the tiles in `idx` (all bound to k with the same arg).
AieRC launch_group(miaie_xaie_dev* d, const XAie_MiaieKernel* k, u32 arg, const std::vector<int>& idx, u32 passes) {
  u32 ping[MIAIE_XAIE_MAX_PARAMS] = {0};
  window_layout(k, ping, nullptr);
  // A single-tile launch of mm/perf or k1/k2 is fused: it carries the tile's
  // queued host -> tile copies, mirrors its output window into the tile's
  // host shadow and publishes its number in the host done flag.  Any other
  // launch first issues the queued copies.
  FuseArgs fz{};
  u32 inl_used = 0;  // bytes of fz.inl in use
  const bool fusable = idx.size() == 1 && !(k->Flags & MIAIE_XAIE_KERNEL_FOREVER) &&
                       (k->Builtin == B_MM_NT || k->Builtin == B_K1 || k->Builtin == B_K2);
  if (fusable) {
    const int t = idx[0];
    if (AieRC rc = ensure_stage(d)) return rc;
    bool mine = d->pend.size() <= (size_t)kFuseCopies;
    for (const PendCopy& c : d->pend) mine = mine && c.tile == t;
    if (!mine) {
      if (AieRC rc = issue_pending(d)) return rc;
    }
    for (const PendCopy& c : d->pend) {
      fz.dst[fz.ncopy] = (u32)c.addr;
      fz.size[fz.ncopy] = (u32)c.size;
      fz.src[fz.ncopy] = c.src;
      fz.inl_off[fz.ncopy] = kNotInline;
      if (c.size <= kFuseInline - inl_used) {
        std::memcpy(fz.inl + inl_used, c.src, c.size);
        fz.inl_off[fz.ncopy] = inl_used;
        inl_used += (u32)((c.size + 15) & ~static_cast<size_t>(15));
        if (inl_used > kFuseInline) inl_used = kFuseInline;
      }
      ++fz.ncopy;
    }
    d->pend.clear();
    fz.flag = d->done_flag;
    fz.seq = ++d->fuse_seq;
    // the output window as declared (size_hint words), at least what the
    // kernel writes, within the tile's memory
    const u32 declared = 4 * (k->SizeHint[1] ? k->SizeHint[1] : 512);
    const u32 out_bytes = std::min(std::max(declared, builtin_extent(k, 1, arg)), d->bytes[t] - ping[1]);
    if (out_bytes <= kShadowSlot) {
      fz.shadow = d->shadow_mem + (size_t)t * kShadowSlot;
      fz.shadow_addr = ping[1];
      fz.shadow_size = out_bytes;
      Shadow& sh = d->shadow[t];
      sh.valid = true;
      sh.addr = ping[1];
      sh.size = out_bytes;
      sh.seq = fz.seq;
    } else {
      invalidate_shadow(d, t);
    }
    d->cores[t].fused = true;
    d->cores[t].fused_seq = fz.seq;
  } else {
    if (AieRC rc = issue_pending(d)) return rc;
    for (int t : idx) {
      invalidate_shadow(d, t);
      d->cores[t].fused = false;
    }
  }
  for (size_t s = 0; s < idx.size(); s += kMaxRunTiles) {
    TileList tl;
    tl.n = (u32)std::min<size_t>(kMaxRunTiles, idx.size() - s);
    for (u32 i = 0; i < tl.n; ++i) tl.off[i] = d->off[idx[s + i]];
    if (k->Builtin == B_NONE) {
      const int rc = k->Launch(d->stream, d->mem, tl.off, tl.n, ping, k->NumParams, passes, k->User);
      if (rc != 0) return fail(d, XAIE_ERR, "kernel %s: launch function returned %d", k->Name ? k->Name : "?", rc);
      continue;
    }
    switch (k->Builtin) {
      case B_MM_NT:
      case B_K1:
      case B_K2: {
        const bool mm = k->Builtin == B_MM_NT;
        const int karg = mm ? (int)arg : k->Builtin == B_K2 ? 10 : 1;
        auto go = [&](auto tlist, auto f) {
          constexpr int CAP = sizeof(tlist.off) / sizeof(u32);
          constexpr u32 INL = sizeof(f.inl);
          if (mm)
            tile_mm_nt<CAP, INL><<<tl.n, 256, 0, d->stream>>>(
                MmArgs<CAP, INL>{d->mem, tlist, ping[0], ping[1], karg, passes, f});
          else
            tile_add20<CAP, INL><<<tl.n, 64, 0, d->stream>>>(
                AddArgs<CAP, INL>{d->mem, tlist, ping[0], ping[1], karg, passes, f});
        };
        if (fusable) {  // one tile: a one-entry list and the smallest inline area that holds the moves
          const TileListT<1> one{1, {tl.off[0]}};
          if (inl_used <= 512)
            go(one, shrink<512>(fz));
          else
            go(one, fz);
        } else {
          go(tl, shrink<16>(fz));
        }
        break;
      }
      case B_MM3_U64:
        tile_mm3_u64<<<tl.n, 64, 0, d->stream>>>(d->mem, tl, ping[0], ping[1], passes);
        break;
      case B_DOT_U8:  // the whole-GPU MFMA probe of libmiaie, once per tile and pass
        for (u32 i = 0; i < tl.n; ++i)
          for (u32 p = 0; p < passes; ++p) {
            uint8_t* base = d->mem + tl.off[i];
            const int rc = miaie_dot_u8_probe(d->ctx, reinterpret_cast<const uint32_t*>(base + ping[0]),
                                              reinterpret_cast<uint32_t*>(base + ping[1]));
            if (rc) return miaie_fail(d, rc, "perf_u8");
          }
        break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      for (int t : idx) {  // nothing will fill the shadow or raise the flag
        invalidate_shadow(d, t);
        d->cores[t].fused = false;
      }
      return hip_fail(d, e, k->Name ? k->Name : "tile kernel");
    }
  }
  return XAIE_OK;
}

// Launch the given cores, grouped by (kernel, arg), as one batch.
AieRC launch_cores(miaie_xaie_dev* d, const std::vector<int>& tiles, u32 iterations) {
  if (tiles.empty()) return XAIE_OK;
  std::map<std::pair<const XAie_MiaieKernel*, u32>, std::vector<int>> groups;
  for (int t : tiles) groups[{d->cores[t].k, d->cores[t].arg}].push_back(t);
  for (auto& g : groups) {
    const XAie_MiaieKernel* k = g.first.first;
    // a FOREVER kernel runs its bounded stand-in for "until disabled" whatever the iteration count
    const u32 passes = (k->Flags & MIAIE_XAIE_KERNEL_FOREVER) ? MIAIE_XAIE_FOREVER_PASSES : iterations;
    if (AieRC rc = launch_group(d, k, g.first.second, g.second, passes)) return rc;
  }
  // A lone fused launch signals its completion through the host done flag;
  // only other batches record an event (a later event's completion also
  // covers this batch, the numbers being issued in stream order).
  uint64_t seq = 0;
  if (tiles.size() == 1 && d->cores[tiles[0]].fused)
    seq = ++d->issued;
  else if (AieRC rc = record_batch(d, &seq))
    return rc;
  for (int t : tiles) {
    d->cores[t].seq = seq;
    d->cores[t].ran = true;
    d->cores[t].pending = false;
  }
  return XAIE_OK;
}

// Issue the launches of cores enabled since the last flush.
AieRC flush(miaie_xaie_dev* d) {
  std::vector<int> tiles;
  for (size_t t = 0; t < d->cores.size(); ++t)
    if (d->cores[t].pending) tiles.push_back((int)t);
  return launch_cores(d, tiles, 1);
}

bool core_done(miaie_xaie_dev* d, int t) {
  const Core& c = d->cores[t];
  if (!c.ran || c.pending) return false;
  if ((c.k->Flags & MIAIE_XAIE_KERNEL_FOREVER) && c.enabled) return false;
  // a fused launch raises the host done flag itself, ahead of its completion signal
  if (c.fused && (int32_t)(__atomic_load_n(d->done_flag, __ATOMIC_ACQUIRE) - c.fused_seq) >= 0) return true;
  retire(d);
  return c.seq <= d->completed;
}

bool has_route(const XAie_RoutingInstance* ri, int s, int t) {
  for (const Route& r : ri->routes)
    if (r.src == s && r.dst == t) return true;
  return false;
}

XAie_MemInst* find_ddr(miaie_xaie_dev* d, uintptr_t addr, size_t size) {
  for (XAie_MemInst* m : d->ddr) {
    const uintptr_t b = reinterpret_cast<uintptr_t>(m->host);
    if (addr >= b && addr - b <= m->size && size <= m->size - (addr - b)) return m;
  }
  return nullptr;
}

AieRC tile_range(miaie_xaie_dev* d, int t, uint64_t addr, uint64_t size, const char* what) {
  if (d->bytes[t] == 0)
    return fail(d, XAIE_INVALID_TILE, "%s: tile (%u, %u) has no data memory", what, (u32)(t / d->rows),
                (u32)(t % d->rows));
  if (addr > d->bytes[t] || size > d->bytes[t] - addr)
    return fail(d, XAIE_INVALID_DATA_MEM_ADDR, "%s: [0x%llx, +%llu) outside the %u B memory of tile (%u, %u)", what,
                (unsigned long long)addr, (unsigned long long)size, d->bytes[t], (u32)(t / d->rows),
                (u32)(t % d->rows));
  return XAIE_OK;
}

void free_ddr(XAie_MemInst* m) {
  if (m->mapped)
    munmap(m->host, m->mapped);
  else
    free(m->host);
  delete m;
}

void destroy(miaie_xaie_dev* d) {
  for (size_t i = 0; i < g_devices.size(); ++i)
    if (g_devices[i] == d) g_devices.erase(g_devices.begin() + (long)i--);
  if (d->ctx) miaie_wait(d->ctx, -1);
  for (auto& f : d->inflight) (void)hipEventDestroy(f.second);
  for (hipEvent_t e : d->spare) (void)hipEventDestroy(e);
  for (XAie_MemInst* m : d->ddr) free_ddr(m);
  for (XAie_RoutingInstance* r : d->routing) delete r;
  if (d->stage) (void)hipHostFree(d->stage);
  if (d->stage_ev) (void)hipEventDestroy(d->stage_ev);
  if (d->mem) miaie_free(d->ctx, d->mem);
  if (d->ctx) miaie_finish(d->ctx);
  delete d;
}

void reset_state(miaie_xaie_dev* d) {
  for (Core& c : d->cores) c = Core{};
  for (Shadow& sh : d->shadow) sh = Shadow{};
  d->pend.clear();  // the stream has drained and the tile memory is cleared
  d->stage_used = 0;
  for (XAie_RoutingInstance* r : d->routing) r->routes.clear();
}

}  // namespace

// ======================================================================== C ABI
extern "C" {

MIAIE_XAIE_API AieRC XAie_MiaieWindowLayout(const XAie_MiaieKernel* Kernel, u32* Ping, u32* Pong) try {
  const XAie_MiaieKernel* k = nullptr;
  if (AieRC rc = valid_kernel(nullptr, Kernel, &k)) return rc;
  window_layout(k, Ping, Pong);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API const char* XAie_MiaieLastError(const XAie_DevInst* DevInst) try {
  if (DevInst && DevInst->IsReady && DevInst->Priv) return DevInst->Priv->err.c_str();
  return g_last_error.c_str();
} catch (...) { out_of_memory(__func__); return nullptr; }

MIAIE_XAIE_API u32 XAie_MiaieTileMemBytes(const XAie_DevInst* DevInst, XAie_LocType Loc) try {
  if (!DevInst || !DevInst->IsReady || !DevInst->Priv) return 0;
  const int t = tile_index(DevInst->Priv, Loc);
  return t < 0 ? 0 : DevInst->Priv->bytes[t];
} catch (...) { out_of_memory(__func__); return 0; }

MIAIE_XAIE_API AieRC XAie_SetupPartitionConfig(XAie_DevInst* DevInst, u64 PartBaseAddr, u32 StartCol, u32 NumCols) try {
  if (!DevInst) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_SetupPartitionConfig: DevInst is NULL");
  if (DevInst->IsReady) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_SetupPartitionConfig: already initialised");
  if (NumCols == 0 || NumCols > 255 || StartCol > 255)
    return fail(nullptr, XAIE_INVALID_ARGS, "XAie_SetupPartitionConfig: start %u, %u columns", StartCol, NumCols);
  DevInst->StartCol = (u8)StartCol;
  DevInst->PartNumCols = (u8)NumCols;
  DevInst->PartBaseAddr = PartBaseAddr;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CfgInitialize(XAie_DevInst* DevInst, const XAie_Config* Cfg) try {
  if (!DevInst || !Cfg) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_CfgInitialize: NULL argument");
  if (DevInst->IsReady) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_CfgInitialize: instance already initialised");
  if (Cfg->NumCols == 0 || Cfg->NumRows == 0 || Cfg->ShimRowNum >= Cfg->NumRows ||
      Cfg->MemTileRowStart + Cfg->MemTileNumRows > Cfg->NumRows ||
      Cfg->AieTileRowStart + Cfg->AieTileNumRows > Cfg->NumRows || Cfg->AieTileNumRows == 0)
    return fail(nullptr, XAIE_INVALID_ARGS, "XAie_CfgInitialize: inconsistent geometry (%u cols x %u rows)",
                Cfg->NumCols, Cfg->NumRows);
  const u32 cols = DevInst->PartNumCols ? DevInst->PartNumCols : Cfg->NumCols;
  if (DevInst->PartNumCols && DevInst->StartCol + DevInst->PartNumCols > Cfg->NumCols)
    return fail(nullptr, XAIE_INVALID_ARGS, "XAie_CfgInitialize: partition columns [%u, %u) outside %u columns",
                DevInst->StartCol, DevInst->StartCol + DevInst->PartNumCols, Cfg->NumCols);

  miaie_xaie_dev* d = new miaie_xaie_dev;
  d->cols = cols;
  d->rows = Cfg->NumRows;
  const size_t ntiles = (size_t)d->cols * d->rows;
  d->kind.assign(ntiles, T_NONE);
  d->off.assign(ntiles, 0);
  d->bytes.assign(ntiles, 0);
  d->cores.assign(ntiles, Core{});
  d->shadow.assign(ntiles, Shadow{});
  size_t total = 0;
  for (u32 c = 0; c < d->cols; ++c)
    for (u32 r = 0; r < d->rows; ++r) {
      const size_t t = (size_t)c * d->rows + r;
      u32 b = 0;
      if (r == Cfg->ShimRowNum) {
        d->kind[t] = T_SHIM;
      } else if (r >= Cfg->MemTileRowStart && r < (u32)Cfg->MemTileRowStart + Cfg->MemTileNumRows) {
        d->kind[t] = T_MEM;
        b = kMemTileMem;
      } else if (r >= Cfg->AieTileRowStart && r < (u32)Cfg->AieTileRowStart + Cfg->AieTileNumRows) {
        d->kind[t] = T_CORE;
        b = Cfg->AieGen == XAIE_DEV_GEN_AIE ? kCoreMemAie1 : kCoreMem;
      }
      d->off[t] = (u32)total;
      d->bytes[t] = b;
      total += b;
    }
  if (total >= (1ull << 32)) {
    delete d;
    return fail(nullptr, XAIE_INVALID_ARGS, "XAie_CfgInitialize: tile memories exceed 4 GiB");
  }
  const char* dev_env = getenv("MIAIE_XAIE_DEVICE");
  d->device = dev_env ? atoi(dev_env) : 0;
  int rc = miaie_init(&d->ctx, d->device);
  if (rc) {
    AieRC r = fail(nullptr, XAIE_INVALID_DEVICE, "XAie_CfgInitialize: %s", miaie_last_error_string(nullptr));
    delete d;
    return r;
  }
  void* s = nullptr;
  miaie_get_stream(d->ctx, &s);
  d->stream = static_cast<hipStream_t>(s);
  d->mem_bytes = total;
  void* mem = nullptr;
  rc = miaie_alloc(d->ctx, total, &mem);
  if (rc) {
    AieRC r = fail(nullptr, XAIE_ERR, "XAie_CfgInitialize: tile memory (%zu B): %s", total,
                   miaie_last_error_string(d->ctx));
    destroy(d);
    return r;
  }
  d->mem = static_cast<uint8_t*>(mem);
  hipError_t e = hipSetDevice(d->device);
  if (e == hipSuccess) e = hipMemsetAsync(d->mem, 0, total, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) {
    AieRC r = hip_fail(nullptr, e, "XAie_CfgInitialize: clearing tile memory");
    destroy(d);
    return r;
  }

  DevInst->AieGen = Cfg->AieGen;
  DevInst->BaseAddr = Cfg->BaseAddr;
  DevInst->NumCols = Cfg->NumCols;
  DevInst->NumRows = Cfg->NumRows;
  DevInst->ShimRow = Cfg->ShimRowNum;
  DevInst->MemTileRowStart = Cfg->MemTileRowStart;
  DevInst->MemTileNumRows = Cfg->MemTileNumRows;
  DevInst->AieTileRowStart = Cfg->AieTileRowStart;
  DevInst->AieTileNumRows = Cfg->AieTileNumRows;
  DevInst->Backend = &kBackends[0];
  DevInst->Priv = d;
  DevInst->IsReady = 1;
  g_devices.push_back(d);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_SetIOBackend(XAie_DevInst* DevInst, XAie_BackendType Backend) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  for (const XAie_Backend& b : kBackends)
    if (b.Type == Backend) {
      DevInst->Backend = &b;
      d->backend = Backend;
      return XAIE_OK;
    }
  return fail(d, XAIE_INVALID_ARGS, "XAie_SetIOBackend: unknown backend %d", (int)Backend);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_UpdateNpiAddr(XAie_DevInst* DevInst, u64 NpiAddr) try {
  (void)NpiAddr;
  return dev_of(DevInst) ? XAIE_OK : XAIE_INVALID_DEVICE;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_PartitionInitialize(XAie_DevInst* DevInst, void* Opts) try {
  (void)Opts;
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (miaie_wait(d->ctx, -1)) return miaie_fail(d, MIAIE_EHIP, "XAie_PartitionInitialize: drain");
  retire(d);
  hipError_t e = hipMemsetAsync(d->mem, 0, d->mem_bytes, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) return hip_fail(d, e, "XAie_PartitionInitialize: clearing tile memory");
  reset_state(d);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_PmRequestTiles(XAie_DevInst* DevInst, XAie_LocType* Loc, u32 NumTiles) try {
  (void)Loc;
  (void)NumTiles;
  return XAie_PartitionInitialize(DevInst, nullptr);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_PartitionTeardown(XAie_DevInst* DevInst) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  destroy(d);
  DevInst->Priv = nullptr;
  DevInst->IsReady = 0;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_Finish(XAie_DevInst* DevInst) { return XAie_PartitionTeardown(DevInst); }

// ---------------------------------------------------------------- cores
MIAIE_XAIE_API AieRC XAie_CoreReset(XAie_DevInst* DevInst, XAie_LocType Loc) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_CoreReset", &t)) return rc;
  if (AieRC rc = flush(d)) return rc;
  Core& c = d->cores[t];
  c.reset = true;
  c.enabled = false;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CoreUnreset(XAie_DevInst* DevInst, XAie_LocType Loc) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_CoreUnreset", &t)) return rc;
  d->cores[t].reset = false;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_LoadElfMem(XAie_DevInst* DevInst, XAie_LocType Loc, const unsigned char* ElfMem) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_LoadElfMem", &t)) return rc;
  const XAie_MiaieKernel* k = nullptr;
  if (AieRC rc = valid_kernel(d, ElfMem, &k)) return rc;
  if (AieRC rc = check_windows(d, k, window_n(k), d->bytes[t])) return rc;
  if (AieRC rc = flush(d)) return rc;
  Core& c = d->cores[t];
  c.k = k;
  c.arg = window_n(k);
  c.enabled = false;
  c.ran = false;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CoreEnable(XAie_DevInst* DevInst, XAie_LocType Loc) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_CoreEnable", &t)) return rc;
  Core& c = d->cores[t];
  if (!c.k) return fail(d, XAIE_INVALID_ELF, "XAie_CoreEnable: no kernel loaded on tile (%u, %u)", Loc.Col, Loc.Row);
  if (c.reset) return fail(d, XAIE_ERR, "XAie_CoreEnable: tile (%u, %u) is in reset", Loc.Col, Loc.Row);
  c.enabled = true;
  c.pending = true;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CoreDisable(XAie_DevInst* DevInst, XAie_LocType Loc) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_CoreDisable", &t)) return rc;
  if (AieRC rc = flush(d)) return rc;
  d->cores[t].enabled = false;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CoreWaitForDone(XAie_DevInst* DevInst, XAie_LocType Loc, u32 TimeOut) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_CoreWaitForDone", &t)) return rc;
  if (AieRC rc = flush(d)) return rc;
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(TimeOut ? TimeOut : kDefaultWaitUs);
  for (;;) {
    if (core_done(d, t)) return XAIE_OK;
    const Core& c = d->cores[t];
    if (!c.ran || ((c.k->Flags & MIAIE_XAIE_KERNEL_FOREVER) && c.enabled) ||
        std::chrono::steady_clock::now() >= deadline)
      return fail(d, XAIE_CORE_STATUS_TIMEOUT, "XAie_CoreWaitForDone: tile (%u, %u) not done", Loc.Col, Loc.Row);
    std::this_thread::yield();
  }
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CoreReadDoneBit(XAie_DevInst* DevInst, XAie_LocType Loc, u8* DoneBit) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (!DoneBit) return fail(d, XAIE_INVALID_ARGS, "XAie_CoreReadDoneBit: DoneBit is NULL");
  int t;
  if (AieRC rc = core_of(d, Loc, "XAie_CoreReadDoneBit", &t)) return rc;
  if (AieRC rc = flush(d)) return rc;
  *DoneBit = core_done(d, t) ? 1 : 0;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_CoreGetStatus(XAie_DevInst* DevInst, XAie_LocType Loc, u32* CoreStatus) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (!CoreStatus) return fail(d, XAIE_INVALID_ARGS, "XAie_CoreGetStatus: CoreStatus is NULL");
  const int t = tile_index(d, Loc);
  if (t < 0) return fail(d, XAIE_INVALID_TILE, "XAie_CoreGetStatus: tile (%u, %u) outside the partition", Loc.Col, Loc.Row);
  *CoreStatus = 0;
  if (d->kind[t] != T_CORE) return XAIE_OK;
  if (AieRC rc = flush(d)) return rc;
  const Core& c = d->cores[t];
  u32 s = 0;
  if (c.enabled) s |= XAIE_CORE_STATUS_ENABLE_BIT;
  if (c.reset) s |= XAIE_CORE_STATUS_RESET_BIT;
  if (core_done(d, t)) s |= XAIE_CORE_STATUS_DONE_BIT;
  *CoreStatus = s;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

// ---------------------------------------------------------------- data memory
MIAIE_XAIE_API AieRC XAie_DataMemBlockWrite(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, const void* Src, u32 Size) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (!Src && Size) return fail(d, XAIE_INVALID_ARGS, "XAie_DataMemBlockWrite: Src is NULL");
  const int t = tile_index(d, Loc);
  if (t < 0) return fail(d, XAIE_INVALID_TILE, "XAie_DataMemBlockWrite: tile (%u, %u) outside the partition", Loc.Col, Loc.Row);
  if (AieRC rc = tile_range(d, t, Addr, Size, "XAie_DataMemBlockWrite")) return rc;
  if (AieRC rc = flush(d)) return rc;
  return copy_h2d(d, t, Addr, Src, Size);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_DataMemBlockRead(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, void* Dst, u32 Size) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (!Dst && Size) return fail(d, XAIE_INVALID_ARGS, "XAie_DataMemBlockRead: Dst is NULL");
  const int t = tile_index(d, Loc);
  if (t < 0) return fail(d, XAIE_INVALID_TILE, "XAie_DataMemBlockRead: tile (%u, %u) outside the partition", Loc.Col, Loc.Row);
  if (AieRC rc = tile_range(d, t, Addr, Size, "XAie_DataMemBlockRead")) return rc;
  if (AieRC rc = flush(d)) return rc;
  return copy_d2h(d, t, Addr, Dst, Size);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_DataMemWrWord(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, u32 Data) try {
  return XAie_DataMemBlockWrite(DevInst, Loc, Addr, &Data, sizeof Data);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_DataMemRdWord(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, u32* Data) try {
  if (!Data) return fail(DevInst ? DevInst->Priv : nullptr, XAIE_INVALID_ARGS, "XAie_DataMemRdWord: Data is NULL");
  return XAie_DataMemBlockRead(DevInst, Loc, Addr, Data, sizeof *Data);
} catch (...) { return out_of_memory(__func__); }

// ---------------------------------------------------------------- DDR
MIAIE_XAIE_API XAie_MemInst* XAie_MemAllocate(XAie_DevInst* DevInst, u64 Size, XAie_MemCacheProp Cache) try {
  (void)Cache;
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return nullptr;
  if (Size == 0 || Size > (1ull << 31)) {
    fail(d, XAIE_INVALID_ARGS, "XAie_MemAllocate: size %llu outside [1, 2 GiB]", (unsigned long long)Size);
    return nullptr;
  }
  XAie_MemInst* m = new XAie_MemInst{d, nullptr, (size_t)Size, 0};
  const size_t page = (size_t)sysconf(_SC_PAGESIZE);
  const size_t len = (Size + page - 1) / page * page;
  void* p = MAP_FAILED;
#ifdef MAP_32BIT
  // below 4 GiB: a harness may keep the device address in a u32
  p = mmap(nullptr, len, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_32BIT, -1, 0);
#endif
  if (p != MAP_FAILED) {
    m->host = static_cast<uint8_t*>(p);
    m->mapped = len;
  } else {
    m->host = static_cast<uint8_t*>(calloc(1, (size_t)Size));
    if (!m->host) {
      delete m;
      fail(d, XAIE_ERR, "XAie_MemAllocate: out of host memory (%llu B)", (unsigned long long)Size);
      return nullptr;
    }
  }
  d->ddr.push_back(m);
  return m;
} catch (...) { out_of_memory(__func__); return nullptr; }

MIAIE_XAIE_API AieRC XAie_MemFree(XAie_MemInst* MemInst) try {
  if (!MemInst) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_MemFree: NULL");
  miaie_xaie_dev* d = MemInst->dev;
  for (size_t i = 0; i < d->ddr.size(); ++i)
    if (d->ddr[i] == MemInst) {
      d->ddr.erase(d->ddr.begin() + (long)i);
      free_ddr(MemInst);
      return XAIE_OK;
    }
  return fail(d, XAIE_INVALID_ARGS, "XAie_MemFree: unknown buffer");
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API void* XAie_MemGetVAddr(XAie_MemInst* MemInst) { return MemInst ? MemInst->host : nullptr; }

MIAIE_XAIE_API u64 XAie_MemGetDevAddr(XAie_MemInst* MemInst) try {
  return MemInst ? (u64) reinterpret_cast<uintptr_t>(MemInst->host) : 0;
} catch (...) { out_of_memory(__func__); return 0; }

MIAIE_XAIE_API AieRC XAie_MemSyncForDev(XAie_MemInst* MemInst) try {
  return MemInst ? XAIE_OK : fail(nullptr, XAIE_INVALID_ARGS, "XAie_MemSyncForDev: NULL");
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_MemSyncForCPU(XAie_MemInst* MemInst) try {
  return MemInst ? XAIE_OK : fail(nullptr, XAIE_INVALID_ARGS, "XAie_MemSyncForCPU: NULL");
} catch (...) { return out_of_memory(__func__); }

// ---------------------------------------------------------------- routing and moves
MIAIE_XAIE_API XAie_RoutingInstance* XAie_InitRoutingHandler(XAie_DevInst* DevInst) try {
  miaie_xaie_dev* d = dev_of(DevInst);
  if (!d) return nullptr;
  XAie_RoutingInstance* r = new XAie_RoutingInstance{DevInst, {}};
  d->routing.push_back(r);
  return r;
} catch (...) { out_of_memory(__func__); return nullptr; }

MIAIE_XAIE_API AieRC XAie_RoutingInstanceFree(XAie_RoutingInstance* ri) try {
  if (!ri) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_RoutingInstanceFree: NULL");
  miaie_xaie_dev* d = dev_of(ri->dev);
  if (!d) return XAIE_INVALID_DEVICE;
  for (size_t i = 0; i < d->routing.size(); ++i)
    if (d->routing[i] == ri) {
      d->routing.erase(d->routing.begin() + (long)i);
      delete ri;
      return XAIE_OK;
    }
  return fail(d, XAIE_INVALID_ARGS, "XAie_RoutingInstanceFree: unknown routing instance");
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_Route(XAie_RoutingInstance* ri, void* RouteConstraints, XAie_LocType Source,
                                XAie_LocType Destination) try {
  (void)RouteConstraints;
  if (!ri) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_Route: routing instance is NULL");
  miaie_xaie_dev* d = dev_of(ri->dev);
  if (!d) return XAIE_INVALID_DEVICE;
  const int s = tile_index(d, Source), t = tile_index(d, Destination);
  if (s < 0 || t < 0)
    return fail(d, XAIE_INVALID_TILE, "XAie_Route: (%u, %u) -> (%u, %u) outside the partition", Source.Col, Source.Row,
                Destination.Col, Destination.Row);
  if (s == t) return fail(d, XAIE_INVALID_ARGS, "XAie_Route: source and destination are the same tile");
  if (d->kind[s] == T_NONE || d->kind[t] == T_NONE || (d->kind[s] == T_SHIM && d->kind[t] == T_SHIM))
    return fail(d, XAIE_INVALID_TILE, "XAie_Route: (%u, %u) -> (%u, %u) has no data path", Source.Col, Source.Row,
                Destination.Col, Destination.Row);
  if (!has_route(ri, s, t)) ri->routes.push_back(Route{(u16)s, (u16)t});
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_MoveData(XAie_RoutingInstance* ri, XAie_LocType Source, void* SrcAddr, u32 Size,
                                   void* DstAddr, XAie_LocType Destination) try {
  if (!ri) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_MoveData: routing instance is NULL");
  miaie_xaie_dev* d = dev_of(ri->dev);
  if (!d) return XAIE_INVALID_DEVICE;
  const int s = tile_index(d, Source), t = tile_index(d, Destination);
  if (s < 0 || t < 0) return fail(d, XAIE_INVALID_TILE, "XAie_MoveData: tile outside the partition");
  if (!has_route(ri, s, t))
    return fail(d, XAIE_ERR_NO_ROUTE, "XAie_MoveData: no route (%u, %u) -> (%u, %u)", Source.Col, Source.Row,
                Destination.Col, Destination.Row);
  if (AieRC rc = flush(d)) return rc;
  const uintptr_t src = reinterpret_cast<uintptr_t>(SrcAddr), dst = reinterpret_cast<uintptr_t>(DstAddr);
  if (d->kind[s] == T_SHIM) {  // DDR -> tile
    XAie_MemInst* m = find_ddr(d, src, Size);
    if (!m) return fail(d, XAIE_INVALID_ARGS, "XAie_MoveData: source 0x%llx (+%u) is not in an XAie_MemAllocate buffer",
                        (unsigned long long)src, Size);
    if (AieRC rc = tile_range(d, t, dst, Size, "XAie_MoveData")) return rc;
    return copy_h2d(d, t, dst, reinterpret_cast<const void*>(src), Size);
  }
  if (d->kind[t] == T_SHIM) {  // tile -> DDR
    XAie_MemInst* m = find_ddr(d, dst, Size);
    if (!m) return fail(d, XAIE_INVALID_ARGS, "XAie_MoveData: destination 0x%llx (+%u) is not in an XAie_MemAllocate buffer",
                        (unsigned long long)dst, Size);
    if (AieRC rc = tile_range(d, s, src, Size, "XAie_MoveData")) return rc;
    return copy_d2h(d, s, src, reinterpret_cast<void*>(dst), Size);
  }
  // tile -> tile
  if (AieRC rc = tile_range(d, s, src, Size, "XAie_MoveData (source)")) return rc;
  if (AieRC rc = tile_range(d, t, dst, Size, "XAie_MoveData (destination)")) return rc;
  if (Size == 0) return XAIE_OK;
  if (AieRC rc = issue_pending(d)) return rc;
  invalidate_shadow(d, t);
  const int rc = miaie_copy_d2d(d->ctx, d->mem + d->off[t] + dst, d->mem + d->off[s] + src, Size);
  return rc ? miaie_fail(d, rc, "XAie_MoveData: tile to tile copy") : XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_MoveDataExternal2Aie(XAie_RoutingInstance* ri, XAie_LocType Source, XAie_MemInst* MemInst,
                                               u32 Size, u64 DstAddr, XAie_LocType Destination) try {
  if (!MemInst) return fail(ri && ri->dev ? ri->dev->Priv : nullptr, XAIE_INVALID_ARGS, "XAie_MoveDataExternal2Aie: MemInst is NULL");
  if (Size > MemInst->size)
    return fail(MemInst->dev, XAIE_INVALID_ARGS, "XAie_MoveDataExternal2Aie: %u B from a %zu B buffer", Size, MemInst->size);
  if (ri && tile_index(MemInst->dev, Source) >= 0 && MemInst->dev->kind[tile_index(MemInst->dev, Source)] != T_SHIM)
    return fail(MemInst->dev, XAIE_INVALID_TILE, "XAie_MoveDataExternal2Aie: source (%u, %u) is not a shim tile",
                Source.Col, Source.Row);
  return XAie_MoveData(ri, Source, MemInst->host, Size, reinterpret_cast<void*>((uintptr_t)DstAddr), Destination);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_MoveDataAie2External(XAie_RoutingInstance* ri, XAie_LocType Source, u64 SrcAddr, u32 Size,
                                               XAie_MemInst* MemInst, XAie_LocType Destination) try {
  if (!MemInst) return fail(ri && ri->dev ? ri->dev->Priv : nullptr, XAIE_INVALID_ARGS, "XAie_MoveDataAie2External: MemInst is NULL");
  if (Size > MemInst->size)
    return fail(MemInst->dev, XAIE_INVALID_ARGS, "XAie_MoveDataAie2External: %u B into a %zu B buffer", Size, MemInst->size);
  if (ri && tile_index(MemInst->dev, Destination) >= 0 &&
      MemInst->dev->kind[tile_index(MemInst->dev, Destination)] != T_SHIM)
    return fail(MemInst->dev, XAIE_INVALID_TILE, "XAie_MoveDataAie2External: destination (%u, %u) is not a shim tile",
                Destination.Col, Destination.Row);
  return XAie_MoveData(ri, Source, reinterpret_cast<void*>((uintptr_t)SrcAddr), Size, MemInst->host, Destination);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_RouteDmaWait(XAie_RoutingInstance* ri, XAie_LocType Source, XAie_LocType Destination, u8 IsMm2s) try {
  (void)IsMm2s;
  if (!ri) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_RouteDmaWait: routing instance is NULL");
  miaie_xaie_dev* d = dev_of(ri->dev);
  if (!d) return XAIE_INVALID_DEVICE;
  const int s = tile_index(d, Source), t = tile_index(d, Destination);
  if (s < 0 || t < 0 || !has_route(ri, s, t))
    return fail(d, XAIE_ERR_NO_ROUTE, "XAie_RouteDmaWait: no route (%u, %u) -> (%u, %u)", Source.Col, Source.Row,
                Destination.Col, Destination.Row);
  return staged_copies_done(d);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_Run(XAie_RoutingInstance* ri, u32 Iterations) try {
  if (!ri) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_Run: routing instance is NULL");
  miaie_xaie_dev* d = dev_of(ri->dev);
  if (!d) return XAIE_INVALID_DEVICE;
  if (Iterations == 0 || Iterations > (1u << 20))
    return fail(d, XAIE_INVALID_ARGS, "XAie_Run: iterations %u outside [1, 2^20]", Iterations);
  if (AieRC rc = flush(d)) return rc;
  std::vector<char> on(d->cores.size(), 0);
  for (const Route& r : ri->routes) on[r.src] = on[r.dst] = 1;
  std::vector<int> tiles;
  for (size_t t = 0; t < d->cores.size(); ++t) {
    Core& c = d->cores[t];
    if (on[t] && d->kind[t] == T_CORE && c.k && !c.reset) {
      c.enabled = true;
      tiles.push_back((int)t);
    }
  }
  if (tiles.empty()) return fail(d, XAIE_ERR, "XAie_Run: no loaded, out-of-reset core on this instance's routes");
  return launch_cores(d, tiles, Iterations);
} catch (...) { return out_of_memory(__func__); }

}  // extern "C"

// ======================================================================== kernel-instance API
struct XAie_Kernel_Inst {
  XAie_LocType loc;
  const XAie_MiaieKernel* k;
  XAie_RoutingInstance* ri;
  int shim_in = -1, shim_out = -1;
};

namespace {

struct ImplicitDevice {
  XAie_DevInst inst{};
  int refs = 0;
};
ImplicitDevice g_implicit;

// The implicit partition: the AIE-ML geometry every example configures
// (aieml_mm.cc:21-31).
AieRC implicit_open() {
  if (g_implicit.inst.IsReady) return XAIE_OK;
  XAie_SetupConfig(cfg, XAIE_DEV_GEN_AIEML, 0x20000000000ull, 25, 20, 38, 11, 0, 1, 2, 3, 8);
  if (AieRC rc = XAie_CfgInitialize(&g_implicit.inst, &cfg)) return rc;
  return XAie_PartitionInitialize(&g_implicit.inst, nullptr);
}

const XAie_MiaieKernel* builtin_by_name(const char* name) {
  const XAie_MiaieKernel* all[] = {&miaie_xaie_mm,  &miaie_xaie_perf,    &miaie_xaie_k1,
                                   &miaie_xaie_k2,  &miaie_xaie_mm3_u64, &miaie_xaie_perf_u8};
  for (const XAie_MiaieKernel* k : all)
    if (strcmp(k->Name, name) == 0) return k;
  return nullptr;
}

}  // namespace

extern "C" {

MIAIE_XAIE_API XAie_Kernel_Inst* XAie_LoadKernel(const char* Name, int Col, int Row) try {
  if (!Name) {
    fail(nullptr, XAIE_INVALID_ARGS, "XAie_LoadKernel: Name is NULL");
    return nullptr;
  }
  const XAie_MiaieKernel* k = builtin_by_name(Name);
  if (!k) {
    fail(nullptr, XAIE_INVALID_ELF, "XAie_LoadKernel: no built-in kernel named '%s'", Name);
    return nullptr;
  }
  if (Col < 0 || Col > 255 || Row < 0 || Row > 255) {
    fail(nullptr, XAIE_INVALID_TILE, "XAie_LoadKernel: tile (%d, %d)", Col, Row);
    return nullptr;
  }
  if (implicit_open() != XAIE_OK) return nullptr;
  XAie_DevInst* dev = &g_implicit.inst;
  const XAie_LocType loc = XAie_TileLoc((u8)Col, (u8)Row);
  if (XAie_CoreReset(dev, loc) || XAie_CoreUnreset(dev, loc) ||
      XAie_LoadElfMem(dev, loc, reinterpret_cast<const unsigned char*>(k)))
    return nullptr;
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(dev);
  if (!ri) return nullptr;
  g_implicit.refs++;
  return new XAie_Kernel_Inst{loc, k, ri};
} catch (...) { out_of_memory(__func__); return nullptr; }

MIAIE_XAIE_API AieRC XAie_RoutingHostToAie(XAie_Kernel_Inst* K, XAie_LocType Shim) try {
  if (!K) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_RoutingHostToAie: kernel is NULL");
  if (AieRC rc = XAie_Route(K->ri, nullptr, Shim, K->loc)) return rc;
  K->shim_in = tile_index(g_implicit.inst.Priv, Shim);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_RoutingAieToHost(XAie_Kernel_Inst* K, XAie_LocType Shim) try {
  if (!K) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_RoutingAieToHost: kernel is NULL");
  if (AieRC rc = XAie_Route(K->ri, nullptr, K->loc, Shim)) return rc;
  K->shim_out = tile_index(g_implicit.inst.Priv, Shim);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_MoveDataToAie(XAie_Kernel_Inst* K, int Input, const void* Src, size_t Bytes) try {
  if (!K || !Src) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_MoveDataToAie: NULL argument");
  miaie_xaie_dev* d = dev_of(&g_implicit.inst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (K->shim_in < 0) return fail(d, XAIE_ERR_NO_ROUTE, "XAie_MoveDataToAie: no XAie_RoutingHostToAie for this kernel");
  if (Input != 1) return fail(d, XAIE_INVALID_ARGS, "XAie_MoveDataToAie: kernel %s has one input window, got %d", K->k->Name, Input);
  const int t = tile_index(d, K->loc);
  Core& c = d->cores[t];
  if (K->k->Builtin == B_MM_NT) {
    // the window holds A and B of n x n int32: 8 n^2 bytes fix n
    u32 n = 1;
    while (n <= 16 && 8ull * n * n < Bytes) ++n;
    if (n > 16 || 8ull * n * n != Bytes)
      return fail(d, XAIE_INVALID_ARGS, "XAie_MoveDataToAie: %zu B is not an A||B window of n x n int32, n <= 16", Bytes);
    c.arg = n;
  }
  u32 ping[MIAIE_XAIE_MAX_PARAMS];
  window_layout(K->k, ping, nullptr);
  if (AieRC rc = tile_range(d, t, ping[0], Bytes, "XAie_MoveDataToAie")) return rc;
  if (AieRC rc = flush(d)) return rc;
  return copy_h2d(d, t, ping[0], Src, Bytes);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_RunCore(XAie_Kernel_Inst* K) try {
  if (!K) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_RunCore: kernel is NULL");
  miaie_xaie_dev* d = dev_of(&g_implicit.inst);
  if (!d) return XAIE_INVALID_DEVICE;
  const int t = tile_index(d, K->loc);
  if (AieRC rc = flush(d)) return rc;
  d->cores[t].enabled = true;
  return launch_cores(d, std::vector<int>{t}, 1);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_WaitOutData(XAie_Kernel_Inst* K) try {
  if (!K) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_WaitOutData: kernel is NULL");
  miaie_xaie_dev* d = dev_of(&g_implicit.inst);
  if (!d) return XAIE_INVALID_DEVICE;
  const int t = tile_index(d, K->loc);
  if (!d->cores[t].ran) return fail(d, XAIE_ERR, "XAie_WaitOutData: kernel %s was not run", K->k->Name);
  if (K->k->Flags & MIAIE_XAIE_KERNEL_FOREVER) d->cores[t].enabled = false;
  const Core& c = d->cores[t];
  if (c.fused && spin_flag(d->done_flag, c.fused_seq)) return XAIE_OK;  // its output is in the host shadow
  if (miaie_wait(d->ctx, -1)) return miaie_fail(d, MIAIE_EHIP, "XAie_WaitOutData");
  retire(d);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_MoveAieToData(XAie_Kernel_Inst* K, int Output, void* Dst, size_t Bytes) try {
  if (!K || !Dst) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_MoveAieToData: NULL argument");
  miaie_xaie_dev* d = dev_of(&g_implicit.inst);
  if (!d) return XAIE_INVALID_DEVICE;
  if (K->shim_out < 0) return fail(d, XAIE_ERR_NO_ROUTE, "XAie_MoveAieToData: no XAie_RoutingAieToHost for this kernel");
  if (Output != 1) return fail(d, XAIE_INVALID_ARGS, "XAie_MoveAieToData: kernel %s has one output window, got %d", K->k->Name, Output);
  const int t = tile_index(d, K->loc);
  u32 ping[MIAIE_XAIE_MAX_PARAMS];
  window_layout(K->k, ping, nullptr);
  if (AieRC rc = tile_range(d, t, ping[1], Bytes, "XAie_MoveAieToData")) return rc;
  if (AieRC rc = flush(d)) return rc;
  return copy_d2h(d, t, ping[1], Dst, Bytes);
} catch (...) { return out_of_memory(__func__); }

MIAIE_XAIE_API AieRC XAie_KernelFree(XAie_Kernel_Inst* K) try {
  if (!K) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_KernelFree: NULL");
  XAie_RoutingInstanceFree(K->ri);
  delete K;
  if (--g_implicit.refs == 0) return XAie_PartitionTeardown(&g_implicit.inst);
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }

}  // extern "C"

// ======================================================================== launches on DDR addresses
extern "C" MIAIE_XAIE_API AieRC XAie_MiaieRunOnDdr(const XAie_MiaieKernel* Kernel, u32 Cols, u32 Rows, u32 ColStart,
                                                   u32 RowStart, u64 InAddr, u64 OutAddr) try {
  const XAie_MiaieKernel* k = nullptr;
  if (AieRC rc = valid_kernel(nullptr, Kernel, &k)) return rc;
  if (k->NumParams != 2) return fail(nullptr, XAIE_NOT_SUPPORTED, "XAie_MiaieRunOnDdr: kernel %s has %u windows, not 2",
                                     k->Name ? k->Name : "?", k->NumParams);
  if (Cols == 0 || Rows == 0) return fail(nullptr, XAIE_INVALID_ARGS, "XAie_MiaieRunOnDdr: %u x %u tiles", Cols, Rows);
  // the instance whose XAie_MemAllocate buffers hold both addresses
  miaie_xaie_dev* d = nullptr;
  XAie_MemInst *min = nullptr, *mout = nullptr;
  for (miaie_xaie_dev* c : g_devices) {
    XAie_MemInst* a = find_ddr(c, (uintptr_t)InAddr, 1);
    XAie_MemInst* b = find_ddr(c, (uintptr_t)OutAddr, 1);
    if (a && b) {
      d = c, min = a, mout = b;
      break;
    }
  }
  if (!d)
    return fail(nullptr, XAIE_INVALID_ARGS,
                "XAie_MiaieRunOnDdr: 0x%llx / 0x%llx are not both in XAie_MemAllocate buffers of one initialised instance",
                (unsigned long long)InAddr, (unsigned long long)OutAddr);
  if (hipSetDevice(d->device) != hipSuccess) return fail(d, XAIE_ERR, "XAie_MiaieRunOnDdr: hipSetDevice");
  u32 ping[MIAIE_XAIE_MAX_PARAMS];
  window_layout(k, ping, nullptr);
  // bytes moved: the input window (as much of it as the buffer holds) and
  // what the kernel writes (the output window of a user kernel)
  const u32 win_in = 4 * 4 * (k->SizeHint[0] ? k->SizeHint[0] : 512);
  const u32 in_bytes = (u32)std::min<uint64_t>(win_in, min->size - (InAddr - (uintptr_t)min->host));
  const u32 out_bytes = k->Builtin ? builtin_extent(k, 1, 16) : 4 * 4 * (k->SizeHint[1] ? k->SizeHint[1] : 512);
  const uint64_t out_room = mout->size - (OutAddr - (uintptr_t)mout->host);
  if ((uint64_t)out_bytes * Cols * Rows > out_room)
    return fail(d, XAIE_INVALID_ARGS, "XAie_MiaieRunOnDdr: %u tiles x %u B of output exceed the buffer (%llu B)",
                Cols * Rows, out_bytes, (unsigned long long)out_room);
  std::vector<int> tiles;
  for (u32 c = 0; c < Cols; ++c)
    for (u32 r = 0; r < Rows; ++r) {
      const XAie_LocType loc = XAie_TileLoc((u8)(ColStart + c), (u8)(RowStart + r));
      int t;
      if (ColStart + c > 255 || RowStart + r > 255) return fail(d, XAIE_INVALID_TILE, "XAie_MiaieRunOnDdr: tile outside");
      if (AieRC rc = core_of(d, loc, "XAie_MiaieRunOnDdr", &t)) return rc;
      if (AieRC rc = check_windows(d, k, window_n(k), d->bytes[t])) return rc;
      tiles.push_back(t);
    }
  if (AieRC rc = flush(d)) return rc;
  for (int t : tiles) {
    if (AieRC rc = copy_h2d(d, t, ping[0], reinterpret_cast<const void*>((uintptr_t)InAddr), in_bytes)) return rc;
    Core& c = d->cores[t];
    c.k = k;
    c.arg = window_n(k);
    c.reset = false;
    c.enabled = true;
  }
  if (AieRC rc = launch_cores(d, tiles, 1)) return rc;
  for (size_t i = 0; i < tiles.size(); ++i)
    if (AieRC rc = copy_d2h(d, tiles[i], ping[1], reinterpret_cast<void*>((uintptr_t)OutAddr + i * out_bytes), out_bytes))
      return rc;
  return XAIE_OK;
} catch (...) { return out_of_memory(__func__); }
