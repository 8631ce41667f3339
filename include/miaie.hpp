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

// ---------------------------------------------------------------- runtime-shape operators
// The typed entry points with shapes known at run time, on device buffers.
// Asynchronous on the context's stream, like the launch templates above.

// Y = rq_shift(A . B) (NN or NT B, layout MIAIE_B_NN / MIAIE_B_NT); C_dbg
// (nullable) receives the int32 accumulators.
inline void gemm_i8_rq(const Buffer<int8_t>& A, const Buffer<int8_t>& B, Buffer<int8_t>& Y, int M, int N, int K,
                       int shift, bool relu = false, Buffer<int32_t>* C_dbg = nullptr, int b_layout = MIAIE_B_NN,
                       Context& ctx = Context::current()) {
  ctx.check(miaie_gemm_i8_rq(ctx.get(), A.data(), B.data(), Y.data(), M, N, K, shift, relu ? 1 : 0,
                             C_dbg ? C_dbg->data() : nullptr, b_layout));
}

// C = A . B in int32, with row pitches (elements) lda / ldb / ldc.
inline void gemm_i8_i32(const Buffer<int8_t>& A, const Buffer<int8_t>& B, Buffer<int32_t>& C, int M, int N, int K,
                        int lda, int ldb, int ldc, int b_layout = MIAIE_B_NN, Context& ctx = Context::current()) {
  ctx.check(miaie_gemm_i8_i32(ctx.get(), A.data(), B.data(), C.data(), M, N, K, lda, ldb, ldc, b_layout));
}

// C = A . B, bf16 in (raw uint16 bits), fp32 accumulate and out, NN.
inline void gemm_bf16(const Buffer<uint16_t>& A, const Buffer<uint16_t>& B, Buffer<float>& C, int M, int N, int K,
                      Context& ctx = Context::current()) {
  ctx.check(miaie_gemm_bf16_f32(ctx.get(), A.data(), B.data(), C.data(), M, N, K));
}

// Shape of an NHWC x OHWI convolution.
struct ConvShape {
  int N, H, W, Cin, Cout, R = 3, S = 3, stride = 1, pad = 1;
  int Ho() const { return (H + 2 * pad - R) / stride + 1; }
  int Wo() const { return (W + 2 * pad - S) / stride + 1; }
};

// Y[N][Ho][Wo][Cout] = per-channel rq(conv(X, Wt)), shifts[c] in [0, 31].
inline void conv2d_i8(const Buffer<int8_t>& X, const Buffer<int8_t>& Wt, const Buffer<uint8_t>& shifts,
                      Buffer<int8_t>& Y, const ConvShape& c, Context& ctx = Context::current()) {
  ctx.check(miaie_conv2d_i8_nhwc(ctx.get(), X.data(), Wt.data(), shifts.data(), Y.data(), c.N, c.H, c.W, c.Cin,
                                 c.Cout, c.R, c.S, c.stride, c.pad));
}

// H = relu(rq_s1(X . W1)), Y = rq_s2(H . W2); H is caller-provided device
// scratch of M x F.
inline void mlp_i8(const Buffer<int8_t>& X, const Buffer<int8_t>& W1, const Buffer<int8_t>& W2, Buffer<int8_t>& H,
                   Buffer<int8_t>& Y, int M, int K, int F, int Nout, int s1, int s2,
                   Context& ctx = Context::current()) {
  ctx.check(miaie_mlp_i8(ctx.get(), X.data(), W1.data(), W2.data(), H.data(), Y.data(), M, K, F, Nout, s1, s2));
}

}  // namespace miaie

#endif  // MIAIE_HPP
