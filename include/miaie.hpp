// miaie.hpp — C++ host surface over the miaie C ABI (miaie.h).
//
// Header-only; links against libmiaie.so.  Two layers:
//
//  1. RAII wrappers for the aie-rt-shaped runtime calls the reference
//     harnesses make (example/matrixmultiply/aieml_mm.cc:108-249):
//     Context (XAie_CfgInitialize / XAie_PartitionInitialize / teardown),
//     Buffer<T> (XAie_MemAllocate + XAie_MemGetDevAddr), move_in / move_out
//     (XAie_MoveData* + XAie_MemSync*), Context::wait (XAie_CoreWaitForDone,
//     with a deadline).  Failures throw miaie::Error carrying the status.
//
//  2. The aiehlc `__kernel__` launch surface.  aiehlc rewrites a kernel
//     declared `__kernel__` into a template
//       template <int Col, int Row, int colstart, int rowstart, int M, int N, int K,
//                 typename... Args> void NAME(Args&&...)
//     (src/llvm/aiehlc.cc:583-588) that harnesses call as
//       perf<1, 1, 4, 4, 256, 16, 64>(phy, phy_out);   (example/nokernelload/aie_nokernelload.cc:130)
//     Here the same template shapes launch the gfx950 kernels.  Col, Row,
//     colstart and rowstart place a kernel on AIE tiles; on one GPU the
//     placement is the grid decomposition over the CUs, so they are accepted
//     and not used.  M, N, K fix the problem shape at compile time.  Every
//     launch is asynchronous on the current context's stream.
#ifndef MIAIE_HPP
#define MIAIE_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "miaie.h"

namespace miaie {

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

class Context;

namespace detail {
inline Context*& current() {
  static thread_local Context* c = nullptr;
  return c;
}
}  // namespace detail

// One device and one stream.  The most recently constructed Context on a
// thread is that thread's current context (used by the template launchers).
class Context {
 public:
  explicit Context(int device = 0) {
    if (int rc = miaie_init(&h_, device)) throw Error(rc, miaie_last_error_string(nullptr));
    prev_ = detail::current();
    detail::current() = this;
  }
  ~Context() {
    if (detail::current() == this) detail::current() = prev_;
    miaie_finish(h_);
  }
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;

  miaie_ctx* get() const { return h_; }
  static Context& current() {
    if (!detail::current()) throw Error(MIAIE_EINVAL, "no current miaie::Context on this thread");
    return *detail::current();
  }

  // Throw on a non-zero status from an entry point called on this context.
  void check(int rc) const {
    if (rc != MIAIE_OK) throw Error(rc, miaie_last_error_string(h_));
  }
  // XAie_CoreWaitForDone analogue: returns false on MIAIE_ETIMEDOUT.
  bool wait(int timeout_ms = -1) const {
    const int rc = miaie_wait(h_, timeout_ms);
    if (rc == MIAIE_ETIMEDOUT) return false;
    check(rc);
    return true;
  }
  // The tiling planner: the kernel, tile and grid an int8 GEMM of this shape
  // takes, and the CU count it plans for (returns the previous one).
  miaie_gemm_plan plan_gemm_i8(int M, int N, int K) const {
    miaie_gemm_plan p{};
    check(miaie_plan_gemm_i8(h_, M, N, K, &p));
    return p;
  }
  int plan_set_cus(int cus) const {
    int prev = 0;
    check(miaie_plan_set_cus(h_, cus, &prev));
    return prev;
  }

 private:
  miaie_ctx* h_ = nullptr;
  Context* prev_ = nullptr;
};

// Device buffer of n elements of T (XAie_MemAllocate).
template <typename T>
class Buffer {
 public:
  Buffer(Context& ctx, size_t n) : ctx_(&ctx), n_(n) {
    void* p = nullptr;
    ctx.check(miaie_alloc(ctx.get(), n * sizeof(T) > 0 ? n * sizeof(T) : 1, &p));
    p_ = static_cast<T*>(p);
  }
  ~Buffer() {
    if (p_) miaie_free(ctx_->get(), p_);
  }
  Buffer(Buffer&& o) noexcept : ctx_(o.ctx_), p_(o.p_), n_(o.n_) { o.p_ = nullptr; }
  Buffer(const Buffer&) = delete;
  Buffer& operator=(const Buffer&) = delete;

  T* data() const { return p_; }
  size_t size() const { return n_; }
  size_t bytes() const { return n_ * sizeof(T); }

  // XAie_MoveDataExternal2Aie / XAie_MoveData host -> tile (+ MemSyncForDev)
  void move_in(const T* host, size_t n) { ctx_->check(miaie_copy_h2d(ctx_->get(), p_, host, n * sizeof(T))); }
  void move_in(const std::vector<T>& host) { move_in(host.data(), host.size()); }
  // XAie_MoveDataAie2External / XAie_MoveData tile -> host (+ MemSyncForCPU)
  void move_out(T* host, size_t n) const { ctx_->check(miaie_copy_d2h(ctx_->get(), host, p_, n * sizeof(T))); }
  std::vector<T> move_out() const {
    std::vector<T> h(n_);
    move_out(h.data(), n_);
    return h;
  }

 private:
  Context* ctx_;
  T* p_ = nullptr;
  size_t n_;
};

// ---------------------------------------------------------------- aiehlc launch surface
// `mm` of example/matrixmultiply/aieml_mm.cc:41-93 (window in: A[M][K] || B[N][K],
// out: C[M][N] = A . B^T, int32 wrap-around).  The window kernel is square.
template <int Col, int Row, int colstart, int rowstart, int M, int N, int K>
void mm(const int32_t* in_window, int32_t* out_window, Context& ctx = Context::current()) {
  static_assert(M == N && N == K && M >= 1 && M <= 4096, "mm: square window, n in [1, 4096]");
  ctx.check(miaie_mm_window_i32(ctx.get(), in_window, out_window, M));
}

// `perf` of example/perf/aieml_perf.cc:61-83 (uint32 variant of mm).
template <int Col, int Row, int colstart, int rowstart, int M, int N, int K>
void perf(const uint32_t* in_window, uint32_t* out_window, Context& ctx = Context::current()) {
  static_assert(M == N && N == K && M >= 1 && M <= 4096, "perf: square window, n in [1, 4096]");
  ctx.check(miaie_perf_window_u32(ctx.get(), in_window, out_window, M));
}

// `perf` of example/nokernelload/aie_nokernelload.cc:50-83, launched there as
// perf<1,1,4,4,256,16,64>(phy, phy_out): the uint8 MAC probe (in[0] =
// param_nn; out[0..4]).  M/N/K do not change the probe.
template <int Col, int Row, int colstart, int rowstart, int M, int N, int K>
void dot_probe(const uint32_t* in, uint32_t* out, Context& ctx = Context::current()) {
  ctx.check(miaie_dot_u8_probe(ctx.get(), in, out));
}

// int8 GEMM + requant, dense row-major NN: Y[M][N] = rq_shift(A[M][K] . B[K][N]).
template <int Col, int Row, int colstart, int rowstart, int M, int N, int K>
void gemm_i8(const int8_t* A, const int8_t* B, int8_t* Y, int shift, bool relu = false, int32_t* C_dbg = nullptr,
             Context& ctx = Context::current()) {
  static_assert(M >= 1 && N >= 1 && K >= 1, "gemm_i8: positive shape");
  ctx.check(miaie_gemm_i8_rq(ctx.get(), A, B, Y, M, N, K, shift, relu ? 1 : 0, C_dbg, MIAIE_B_NN));
}

// bf16 x bf16 -> fp32 GEMM, dense row-major NN (bf16 as raw uint16 bits).
template <int Col, int Row, int colstart, int rowstart, int M, int N, int K>
void gemm_bf16(const uint16_t* A, const uint16_t* B, float* C, Context& ctx = Context::current()) {
  static_assert(M >= 1 && N >= 1 && K >= 1, "gemm_bf16: positive shape");
  ctx.check(miaie_gemm_bf16_f32(ctx.get(), A, B, C, M, N, K));
}

}  // namespace miaie

#endif  // MIAIE_HPP
