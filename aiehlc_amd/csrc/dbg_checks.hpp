// Device-side bounds checks of the debug build.
//
// Built with MIAIE_DEVICE_CHECKS=1 (aiehlc_amd/lib_dbg/libmiaie.so, which a
// process selects with MIAIE_LIB_DIR), every global load and store of the
// library's kernels goes through ld / st / st_nt below, and every 16-byte
// global -> LDS copy through dev::gload_lds16.  Each first looks the byte
// range it would touch up in a table of the buffers the runtime knows (a
// copy: in the buffer its kernel found for that operand at its start): every
// live miaie_alloc allocation, plus what the caller declares with
// miaie_debug_register (buffers from elsewhere, or a sub-range of an
// allocation).  An access that no table entry contains is not performed (a
// load yields zeros, a store or copy is dropped) and is counted in a fault
// record whose first entry keeps the address, size, direction and source line
// of the access; miaie_wait then returns MIAIE_EFAULT and names it.
//
// The table and the record are file-scope device variables, one copy per
// translation unit (the library is built without relocatable device code):
// each unit registers an uploader and a reader with the runtime at static
// initialisation, and the runtime updates every unit's table after each
// change and reads every unit's record after each wait.
//
// In the product build (MIAIE_DEVICE_CHECKS unset or 0) ld / st / st_nt are
// the plain accesses, the line argument is unused, and the device code is the
// same as written without them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

#ifndef MIAIE_DEVICE_CHECKS
#define MIAIE_DEVICE_CHECKS 0
#endif

namespace miaie {
namespace dbg {

constexpr int kMaxRanges = 1024;

template <class T>
struct same_t {
  using type = T;
};

// Buffers as [lo, hi) byte ranges, sorted by lo, not overlapping.
struct Ranges {
  uint64_t lo[kMaxRanges];
  uint64_t hi[kMaxRanges];
  int n;
};

// First access outside every range since the record was last read.
struct Fault {
  unsigned long long count;
  unsigned long long addr;
  unsigned long long bytes;
  int write;      // 0 load, 1 store, 2 global -> LDS copy
  int line;       // source line of the access
  uint32_t file;  // file_id of its source file
  uint32_t pad;
};

// Compile-time id of a source file name (FNV-1a), so a device record can name
// the file: the host maps it back through kFiles.
constexpr uint32_t file_id(const char* s) {
  uint32_t h = 2166136261u;
  while (*s) h = (h ^ (uint8_t)*s++) * 16777619u;
  return h;
}
constexpr const char* kFiles[] = {"gemm_i8_kernels.hpp", "gemm_i8.hip",       "gemm_bf16.hip",   "conv2d_i8.hip",
                                  "conv2d_i8_rows.hpp",  "gfx950_ops.hpp",    "ref_kernels.hip", "miaie_runtime.hip",
                                  "dbg_checks.hpp",      "noalloc.hip"};

// One translation unit's table and record, as the runtime drives them.
struct Unit {
  const char* name;
  int (*upload)(const Ranges& r, int device);  // hipError_t of the copy
  int (*take)(Fault* out, int device);         // read the record and clear it
};

#if MIAIE_DEVICE_CHECKS

// Defined by the runtime (miaie_runtime.hip).
void register_unit(const Unit& u);

static __device__ Ranges g_ranges;
static __device__ Fault g_fault;

__device__ __forceinline__ static bool inside(const void* p, size_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  int lo = 0, hi = g_ranges.n - 1, at = -1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (g_ranges.lo[mid] <= a) {
      at = mid;
      lo = mid + 1;
    } else {
      hi = mid - 1;
    }
  }
  return at >= 0 && a + bytes <= g_ranges.hi[at];
}

__device__ __forceinline__ static void report(const void* p, size_t bytes, int write, int line, uint32_t file) {
  const unsigned long long prev =
      __hip_atomic_fetch_add(&g_fault.count, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (prev == 0) {
    g_fault.addr = (unsigned long long)(uintptr_t)p;
    g_fault.bytes = bytes;
    g_fault.write = write;
    g_fault.line = line;
    g_fault.file = file;
  }
}

// The buffer that contains p (the empty span when none does): the pipelined
// kernels look up each operand's buffer once and check their copies against
// it, instead of searching the table for every copy.
struct Span {
  uint64_t lo, hi;
};
__device__ __forceinline__ Span span_of(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  int lo = 0, hi = g_ranges.n - 1, at = -1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (g_ranges.lo[mid] <= a) {
      at = mid;
      lo = mid + 1;
    } else {
      hi = mid - 1;
    }
  }
  if (at >= 0 && a < g_ranges.hi[at]) return Span{g_ranges.lo[at], g_ranges.hi[at]};
  return Span{0, 0};
}
__device__ __forceinline__ bool in_span(const Span& s, const void* p, size_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return a >= s.lo && a + bytes <= s.hi;
}

__device__ __forceinline__ bool check(const void* p, size_t bytes, int write, int line, uint32_t file) {
  if (inside(p, bytes)) return true;
  report(p, bytes, write, line, file);
  return false;
}
template <class T>
__device__ __forceinline__ T ld(const T* p, int line, uint32_t file) {
  if (inside(p, sizeof(T))) return *p;
  report(p, sizeof(T), 0, line, file);
  return T{};
}
template <class T>
__device__ __forceinline__ T ld_nt(const T* p, int line, uint32_t file) {
  if (inside(p, sizeof(T))) return __builtin_nontemporal_load(p);
  report(p, sizeof(T), 0, line, file);
  return T{};
}
template <class T>
__device__ __forceinline__ void st(T* p, typename same_t<T>::type v, int line, uint32_t file) {
  if (inside(p, sizeof(T)))
    *p = v;
  else
    report(p, sizeof(T), 1, line, file);
}
template <class T>
__device__ __forceinline__ void st_nt(T* p, typename same_t<T>::type v, int line, uint32_t file) {
  if (inside(p, sizeof(T)))
    __builtin_nontemporal_store(v, p);
  else
    report(p, sizeof(T), 1, line, file);
}
// The same two stores checked against a span found before (span_of).
template <class T>
__device__ __forceinline__ void st_in(const Span& s, T* p, typename same_t<T>::type v, int line, uint32_t file) {
  if (in_span(s, p, sizeof(T)))
    *p = v;
  else
    report(p, sizeof(T), 1, line, file);
}
template <class T>
__device__ __forceinline__ void st_nt_in(const Span& s, T* p, typename same_t<T>::type v, int line, uint32_t file) {
  if (in_span(s, p, sizeof(T)))
    __builtin_nontemporal_store(v, p);
  else
    report(p, sizeof(T), 1, line, file);
}

namespace {
int upload_ranges(const Ranges& r, int device) {
  (void)device;
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_ranges), &r, sizeof(Ranges), 0, hipMemcpyHostToDevice);
}
int take_fault(Fault* out, int device) {
  (void)device;
  hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_fault), sizeof(Fault), 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess || out->count == 0) return (int)e;
  const Fault zero{};
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_fault), &zero, sizeof(Fault), 0, hipMemcpyHostToDevice);
}
struct UnitRegistration {
  UnitRegistration() { register_unit(Unit{__BASE_FILE__, &upload_ranges, &take_fault}); }
};
UnitRegistration g_unit_registration;
}  // namespace

#else

struct Span {};
__device__ __forceinline__ Span span_of(const void*) { return Span{}; }
__device__ __forceinline__ constexpr bool check(const void*, size_t, int, int, uint32_t) { return true; }
template <class T>
__device__ __forceinline__ T ld(const T* p, int, uint32_t) {
  return *p;
}
template <class T>
__device__ __forceinline__ T ld_nt(const T* p, int, uint32_t) {
  return __builtin_nontemporal_load(p);
}
template <class T>
__device__ __forceinline__ void st(T* p, typename same_t<T>::type v, int, uint32_t) {
  *p = v;
}
template <class T>
__device__ __forceinline__ void st_nt(T* p, typename same_t<T>::type v, int, uint32_t) {
  __builtin_nontemporal_store(v, p);
}
template <class T>
__device__ __forceinline__ void st_in(const Span&, T* p, typename same_t<T>::type v, int, uint32_t) {
  *p = v;
}
template <class T>
__device__ __forceinline__ void st_nt_in(const Span&, T* p, typename same_t<T>::type v, int, uint32_t) {
  __builtin_nontemporal_store(v, p);
}

#endif

}  // namespace dbg
}  // namespace miaie

// Checked global accesses (plain ones in the product build).  MIAIE_CHECK
// tests (and reports) an access made some other way, e.g. an atomic; it is
// constant true in the product build.
#define MIAIE_DBG_WHERE \
  __LINE__, (::std::integral_constant<uint32_t, ::miaie::dbg::file_id(__FILE_NAME__)>::value)
#define MIAIE_LD(p) (::miaie::dbg::ld((p), MIAIE_DBG_WHERE))
#define MIAIE_LD_NT(p) (::miaie::dbg::ld_nt((p), MIAIE_DBG_WHERE))
#define MIAIE_ST(p, v) (::miaie::dbg::st((p), (v), MIAIE_DBG_WHERE))
#define MIAIE_ST_NT(p, v) (::miaie::dbg::st_nt((p), (v), MIAIE_DBG_WHERE))
#define MIAIE_ST_IN(s, p, v) (::miaie::dbg::st_in((s), (p), (v), MIAIE_DBG_WHERE))
#define MIAIE_ST_NT_IN(s, p, v) (::miaie::dbg::st_nt_in((s), (p), (v), MIAIE_DBG_WHERE))
#define MIAIE_CHECK(p, bytes, write) (::miaie::dbg::check((p), (bytes), (write), MIAIE_DBG_WHERE))
