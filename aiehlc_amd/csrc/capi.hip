// Typed C-ABI entries: argument validation, then dispatch to the kernels.
//
// All validation happens on the host before anything is queued, so an
// invalid call never launches (the reference's kernels cannot report errors
// at all; its harnesses check only init-time AieRC values,
// example/perf/aieml_perf.cc:283-310).
#include "miaie_internal.hpp"

using namespace miaie;

namespace {

int check_shift(miaie_ctx* ctx, const char* fn, const char* name, int s) {
  if (s < 0 || s > 31) return fail(ctx, MIAIE_EINVAL, "%s: %s=%d outside [0, 31]", fn, name, s);
  return MIAIE_OK;
}

int check_dims(miaie_ctx* ctx, const char* fn, int M, int N, int K) {
  if (M < 1 || N < 1 || K < 1) return fail(ctx, MIAIE_EINVAL, "%s: M=%d N=%d K=%d must all be >= 1", fn, M, N, K);
  return MIAIE_OK;
}

}  // namespace

extern "C" int miaie_gemm_i8_i32(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int32_t* C, int M, int N, int K,
                                 int lda, int ldb, int ldc, int b_layout) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, A);
  MIAIE_CHECK_NOT_NULL(ctx, B);
  MIAIE_CHECK_NOT_NULL(ctx, C);
  if ((rc = check_dims(ctx, __func__, M, N, K))) return rc;
  if (b_layout != MIAIE_B_NN && b_layout != MIAIE_B_NT)
    return fail(ctx, MIAIE_EINVAL, "%s: b_layout=%d is neither MIAIE_B_NN nor MIAIE_B_NT", __func__, b_layout);
  const int ldb_min = b_layout == MIAIE_B_NT ? K : N;
  if (lda < K || ldb < ldb_min || ldc < N)
    return fail(ctx, MIAIE_EINVAL, "%s: strides lda=%d ldb=%d ldc=%d below K=%d / %s=%d / N=%d", __func__, lda, ldb,
                ldc, K, b_layout == MIAIE_B_NT ? "K" : "N", ldb_min, N);
  if (!aligned(C, 4)) return fail(ctx, MIAIE_EINVAL, "%s: C must be 4-byte aligned", __func__);
  return launch_gemm_i8(ctx, A, B, nullptr, C, M, N, K, lda, ldb, 0, ldc, b_layout == MIAIE_B_NT, 0, 0);
}

extern "C" int miaie_gemm_i8_rq(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int8_t* Y, int M, int N, int K,
                                int shift, int relu, int32_t* C_dbg, int b_layout) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, A);
  MIAIE_CHECK_NOT_NULL(ctx, B);
  MIAIE_CHECK_NOT_NULL(ctx, Y);
  if ((rc = check_dims(ctx, __func__, M, N, K))) return rc;
  if ((rc = check_shift(ctx, __func__, "shift", shift))) return rc;
  if (relu != 0 && relu != 1) return fail(ctx, MIAIE_EINVAL, "%s: relu=%d must be 0 or 1", __func__, relu);
  if (b_layout != MIAIE_B_NN && b_layout != MIAIE_B_NT)
    return fail(ctx, MIAIE_EINVAL, "%s: b_layout=%d is neither MIAIE_B_NN nor MIAIE_B_NT", __func__, b_layout);
  if (C_dbg && !aligned(C_dbg, 4)) return fail(ctx, MIAIE_EINVAL, "%s: C_dbg must be 4-byte aligned", __func__);
  const int ldb = b_layout == MIAIE_B_NT ? K : N;
  return launch_gemm_i8(ctx, A, B, Y, C_dbg, M, N, K, K, ldb, N, N, b_layout == MIAIE_B_NT, shift, relu);
}

extern "C" int miaie_gemm_bf16_f32(miaie_ctx* ctx, const uint16_t* A, const uint16_t* B, float* C, int M, int N,
                                   int K) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, A);
  MIAIE_CHECK_NOT_NULL(ctx, B);
  MIAIE_CHECK_NOT_NULL(ctx, C);
  if ((rc = check_dims(ctx, __func__, M, N, K))) return rc;
  if (!aligned(A, 2) || !aligned(B, 2) || !aligned(C, 4))
    return fail(ctx, MIAIE_EINVAL, "%s: misaligned buffer", __func__);
  return launch_gemm_bf16(ctx, A, B, C, M, N, K);
}

namespace {

int check_conv_shape(miaie_ctx* ctx, const char* fn, int N, int H, int W_, int Cin, int Cout, int R, int S,
                     int stride, int pad) {
  if (N < 1 || H < 1 || W_ < 1 || Cin < 1 || Cout < 1 || R < 1 || S < 1 || stride < 1 || pad < 0)
    return fail(ctx, MIAIE_EINVAL, "%s: invalid shape N=%d H=%d W=%d Cin=%d Cout=%d R=%d S=%d stride=%d pad=%d",
                fn, N, H, W_, Cin, Cout, R, S, stride, pad);
  if (H + 2 * pad < R || W_ + 2 * pad < S)
    return fail(ctx, MIAIE_EINVAL, "%s: filter %dx%d larger than the padded input %dx%d", fn, R, S, H + 2 * pad,
                W_ + 2 * pad);
  if ((size_t)R * S * Cin > (1u << 30) || (size_t)N * H * W_ * Cin > ((size_t)1 << 40))
    return fail(ctx, MIAIE_EINVAL, "%s: problem too large", fn);
  return MIAIE_OK;
}

}  // namespace

extern "C" int miaie_plan_conv2d_i8(int N, int H, int W_, int Cin, int Cout, int R, int S, int stride, int pad,
                                    int* kernel) {
  if (!kernel) return fail(nullptr, MIAIE_EINVAL, "%s: kernel is NULL", __func__);
  int rc = check_conv_shape(nullptr, __func__, N, H, W_, Cin, Cout, R, S, stride, pad);
  if (rc) return rc;
  *kernel = conv2d_kernel_for(N, H, W_, Cin, Cout, R, S, stride, pad, true, true, 256);
  return MIAIE_OK;
}

extern "C" int miaie_conv2d_i8_nhwc(miaie_ctx* ctx, const int8_t* X, const int8_t* W, const uint8_t* shifts,
                                    int8_t* Y, int N, int H, int W_, int Cin, int Cout, int R, int S, int stride,
                                    int pad) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, X);
  MIAIE_CHECK_NOT_NULL(ctx, W);
  MIAIE_CHECK_NOT_NULL(ctx, shifts);
  MIAIE_CHECK_NOT_NULL(ctx, Y);
  if ((rc = check_conv_shape(ctx, __func__, N, H, W_, Cin, Cout, R, S, stride, pad))) return rc;
  return launch_conv2d_i8(ctx, X, W, shifts, Y, N, H, W_, Cin, Cout, R, S, stride, pad);
}

namespace miaie {

int mlp_i8_checked(miaie_ctx* ctx, const char* fn, const int8_t* X, const int8_t* W1, const int8_t* W2, int8_t* H,
                   int8_t* Y, int M, int K, int F, int Nout, int s1, int s2) {
  int rc;
  if (X == nullptr || W1 == nullptr || W2 == nullptr || H == nullptr || Y == nullptr)
    return fail(ctx, MIAIE_EINVAL, "%s: %s is NULL", fn,
                X == nullptr ? "X" : W1 == nullptr ? "W1" : W2 == nullptr ? "W2" : H == nullptr ? "H" : "Y");
  if (M < 1 || K < 1 || F < 1 || Nout < 1)
    return fail(ctx, MIAIE_EINVAL, "%s: M=%d K=%d F=%d Nout=%d must all be >= 1", fn, M, K, F, Nout);
  if ((rc = check_shift(ctx, fn, "s1", s1))) return rc;
  if ((rc = check_shift(ctx, fn, "s2", s2))) return rc;
  // stage 1: H = relu(rq_s1(X . W1))   (k1 of multi_tile.cpp:39-42)
  // (H is written with ordinary stores: stage 2 reads it right after, and
  // non-temporal ones cost 4-5% of the MLP)
  rc = launch_gemm_i8(ctx, X, W1, H, nullptr, M, F, K, K, F, F, F, 0, s1, 1, true);
  if (rc) return rc;
  // stage 2: Y = rq_s2(H . W2), queued behind stage 1 on the same stream
  // (the tile -> tile hand-off of multi_tile.cpp:125-127 without a host trip)
  return launch_gemm_i8(ctx, H, W2, Y, nullptr, M, Nout, F, F, Nout, Nout, Nout, 0, s2, 0);
}

}  // namespace miaie

extern "C" int miaie_mlp_i8(miaie_ctx* ctx, const int8_t* X, const int8_t* W1, const int8_t* W2, int8_t* H,
                            int8_t* Y, int M, int K, int F, int Nout, int s1, int s2) {
  int rc = enter(ctx);
  if (rc) return rc;
  return mlp_i8_checked(ctx, __func__, X, W1, W2, H, Y, M, K, F, Nout, s1, s2);
}
