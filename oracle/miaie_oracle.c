/*
 * miaie CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's golden computations for the
 * GEMM/conv hot path.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline) — never as the product path.
 *
 * Every function cites the reference file:line it follows (paths relative
 * to the Xilinx/aiehlc tree).  Functions whose semantics exist only in the
 * benchmark definition (int8 NN GEMM, requant, bf16, conv2d, MLP) say so;
 * each of them is pinned by the independent checks in tests/test_oracle_*.py
 * (closed forms, brute force with Python integers, invariants), never by a
 * restatement of the same formula.
 *
 * Integer arithmetic that the reference performs in int32/uint32 with
 * wrap-around is done here in uint32 so that overflow is defined.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* Seeded synthetic inputs: SplitMix64 (Steele, Lea, Flood 2014).       */
/* state += 0x9E3779B97F4A7C15; z = mix(state).                         */
/* Per-tensor stream: state0 = splitmix64 step applied to                */
/* 0x5EED0000 + tensor_id; element i uses the (i+1)-th step from state0. */
/* ------------------------------------------------------------------ */
#define SM64_GAMMA 0x9E3779B97F4A7C15ULL

static inline uint64_t sm64_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

ORACLE_API uint64_t oracle_tensor_seed(uint64_t tensor_id) {
  return sm64_mix(0x5EED0000ULL + tensor_id + SM64_GAMMA);
}

/* i-th (0-based) raw draw of the stream that starts at state0 */
ORACLE_API uint64_t oracle_sm64_at(uint64_t state0, uint64_t i) {
  return sm64_mix(state0 + (i + 1) * SM64_GAMMA);
}

ORACLE_API void oracle_fill_i8(int8_t* dst, size_t n, uint64_t tensor_id) {
  uint64_t s = oracle_tensor_seed(tensor_id);
  for (size_t i = 0; i < n; ++i) {
    s += SM64_GAMMA;
    dst[i] = (int8_t)(uint8_t)(sm64_mix(s) >> 56);
  }
}

/* per-output-channel shift in [8, 12] */
ORACLE_API void oracle_fill_shift(uint8_t* dst, size_t n, uint64_t tensor_id) {
  uint64_t s = oracle_tensor_seed(tensor_id);
  for (size_t i = 0; i < n; ++i) {
    s += SM64_GAMMA;
    dst[i] = (uint8_t)(8 + (sm64_mix(s) >> 32) % 5);
  }
}

/* fp32 -> bf16 bits, round to nearest even (NaN kept quiet). */
ORACLE_API uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

ORACLE_API float oracle_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* N(0,1) * scale by Box-Muller on two 53-bit uniforms (z0 only), rounded to bf16. */
ORACLE_API void oracle_fill_bf16_normal(uint16_t* dst, size_t n, uint64_t tensor_id, double scale) {
  uint64_t s = oracle_tensor_seed(tensor_id);
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; ++i) {
    s += SM64_GAMMA;
    uint64_t r1 = sm64_mix(s);
    s += SM64_GAMMA;
    uint64_t r2 = sm64_mix(s);
    double u1 = ((double)(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    dst[i] = oracle_f32_to_bf16((float)(z * scale));
  }
}

/* ------------------------------------------------------------------ */
/* Reference golden: packed-window NT int32 GEMM.                        */
/* example/matrixmultiply/aieml_mm.cc:194-230: A = vmem[i*N+j] (row     */
/* major), B = vmem[MAT_SIZE + i*N + j] stored as [N][K] ("column       */
/* major"), result zero-initialised, result[i][j] += A[i][k]*B[j][k] in  */
/* i-j-k order.  Same loop at example/perf/aieml_perf.cc:195-231,        */
/* example/nokernelload/aie_nokernelload.cc:137-173 and                 */
/* example/other/aieoob.c:97-133 (n = 8).                                */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_mm_window_i32(const int32_t* win, int32_t* out, int n) {
  const int32_t* A = win;
  const int32_t* B = win + (size_t)n * n;
  for (int i = 0; i < n; ++i)
    for (int j = 0; j < n; ++j) {
      uint32_t acc = 0;
      for (int k = 0; k < n; ++k)
        acc += (uint32_t)A[i * n + k] * (uint32_t)B[j * n + k];
      out[i * n + j] = (int32_t)acc;
    }
}

/* Mismatch count, as reported by aieml_mm.cc:232-245. */
ORACLE_API int oracle_count_mismatch_i32(const int32_t* want, const int32_t* got, size_t n) {
  int bad = 0;
  for (size_t i = 0; i < n; ++i) bad += want[i] != got[i];
  return bad;
}

/* ------------------------------------------------------------------ */
/* int8 x int8 -> int32 GEMM, NT layout (B is N x K, k contiguous), the  */
/* reference golden loop of aieml_mm.cc:217-223 with int8 operands.      */
/* Rows [row0, row1) of C only, so a slab can be checked or timed.       */
/* nthreads > 1 splits rows over OpenMP threads (results identical).     */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_gemm_i8_nt_rows(const int8_t* A, const int8_t* B, int32_t* C,
                                       int M, int N, int K, int lda, int ldb, int ldc,
                                       int row0, int row1, int nthreads) {
  (void)M;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int i = row0; i < row1; ++i) {
    for (int j = 0; j < N; ++j) {
      uint32_t acc = 0; /* int32 accumulate, wrap-around defined */
      const int8_t* a = A + (size_t)i * lda;
      const int8_t* b = B + (size_t)j * ldb;
      for (int k = 0; k < K; ++k) acc += (uint32_t)((int32_t)a[k] * (int32_t)b[k]);
      C[(size_t)i * ldc + j] = (int32_t)acc;
    }
  }
  (void)nthreads;
}

/* B (K x N, row major) -> Bt (N x K).  The NN benchmark layout is turned
 * into the reference's NT layout once, outside any timed region. */
ORACLE_API void oracle_transpose_i8(const int8_t* B, int8_t* Bt, int K, int N, int ldb) {
  for (int k = 0; k < K; ++k)
    for (int n = 0; n < N; ++n) Bt[(size_t)n * K + k] = B[(size_t)k * ldb + n];
}

/* NN int8 GEMM (benchmark layout; no reference counterpart): transpose B,
 * then the reference NT loop. */
ORACLE_API int oracle_gemm_i8_nn_rows(const int8_t* A, const int8_t* B, int32_t* C,
                                      int M, int N, int K, int lda, int ldb, int ldc,
                                      int row0, int row1, int nthreads) {
  int8_t* Bt = (int8_t*)malloc((size_t)N * K + 1);
  if (!Bt) return -1;
  oracle_transpose_i8(B, Bt, K, N, ldb);
  oracle_gemm_i8_nt_rows(A, Bt, C, M, N, K, lda, K, ldc, row0, row1, nthreads);
  free(Bt);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Requantize epilogue (benchmark definition; absent from the reference):*/
/*   y = sat_int8(floor((acc + 2^(s-1)) / 2^s)),  s in [0, 31]           */
/* i.e. an arithmetic right shift with round-half-up, then saturation.   */
/* Computed in int64 so that acc + 2^(s-1) cannot overflow; s = 0 is a   */
/* plain saturation.  relu != 0 clamps negatives to 0 after the shift.   */
/* ------------------------------------------------------------------ */
ORACLE_API int8_t oracle_requant(int32_t acc, int shift, int relu) {
  int64_t v = (int64_t)acc;
  if (shift > 0) v = (v + ((int64_t)1 << (shift - 1))) >> shift;
  if (relu && v < 0) v = 0;
  if (v > 127) v = 127;
  if (v < -128) v = -128;
  return (int8_t)v;
}

ORACLE_API void oracle_requant_buf(const int32_t* acc, int8_t* y, size_t n, int shift, int relu) {
  for (size_t i = 0; i < n; ++i) y[i] = oracle_requant(acc[i], shift, relu);
}

/* GEMM (NN or NT) + requant, rows [row0,row1). C_dbg (nullable) gets the int32 accumulators. */
ORACLE_API int oracle_gemm_i8_rq_rows(const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C_dbg,
                                      int M, int N, int K, int b_nt, int shift, int relu,
                                      int row0, int row1, int nthreads) {
  size_t rows = (size_t)(row1 - row0);
  int32_t* C = (int32_t*)malloc(rows * (size_t)N * sizeof(int32_t) + 4);
  if (!C) return -1;
  const int8_t* Ar = A + (size_t)row0 * K;
  int rc = 0;
  if (b_nt)
    oracle_gemm_i8_nt_rows(Ar, B, C, (int)rows, N, K, K, K, N, 0, (int)rows, nthreads);
  else
    rc = oracle_gemm_i8_nn_rows(Ar, B, C, (int)rows, N, K, K, N, N, 0, (int)rows, nthreads);
  if (rc == 0) {
    oracle_requant_buf(C, Y + (size_t)row0 * N, rows * (size_t)N, shift, relu);
    if (C_dbg) memcpy(C_dbg + (size_t)row0 * N, C, rows * (size_t)N * sizeof(int32_t));
  }
  free(C);
  (void)M;
  return rc;
}

/* ------------------------------------------------------------------ */
/* bf16 x bf16 -> fp32 GEMM, NN, fp32 accumulate in k order (benchmark   */
/* definition).  The fp64 variant is the tighter truth for tolerances.   */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_gemm_bf16_rows(const uint16_t* A, const uint16_t* B, float* C,
                                      int M, int N, int K, int row0, int row1, int nthreads) {
  (void)M;
  float* Bt = (float*)malloc((size_t)N * K * sizeof(float) + 4);
  if (!Bt) return;
  for (int k = 0; k < K; ++k)
    for (int n = 0; n < N; ++n) Bt[(size_t)n * K + k] = oracle_bf16_to_f32(B[(size_t)k * N + n]);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int i = row0; i < row1; ++i) {
    float* arow = (float*)malloc((size_t)K * sizeof(float) + 4);
    for (int k = 0; k < K; ++k) arow[k] = oracle_bf16_to_f32(A[(size_t)i * K + k]);
    for (int j = 0; j < N; ++j) {
      float acc = 0.f;
      const float* b = Bt + (size_t)j * K;
      for (int k = 0; k < K; ++k) acc += arow[k] * b[k];
      C[(size_t)(i - row0) * N + j] = acc;
    }
    free(arow);
  }
  free(Bt);
  (void)nthreads;
}

ORACLE_API void oracle_gemm_bf16_f64_rows(const uint16_t* A, const uint16_t* B, double* C,
                                          int M, int N, int K, int row0, int row1, int nthreads) {
  (void)M;
  double* Bt = (double*)malloc((size_t)N * K * sizeof(double) + 8);
  if (!Bt) return;
  for (int k = 0; k < K; ++k)
    for (int n = 0; n < N; ++n) Bt[(size_t)n * K + k] = oracle_bf16_to_f32(B[(size_t)k * N + n]);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int i = row0; i < row1; ++i) {
    double* arow = (double*)malloc((size_t)K * sizeof(double) + 8);
    for (int k = 0; k < K; ++k) arow[k] = oracle_bf16_to_f32(A[(size_t)i * K + k]);
    for (int j = 0; j < N; ++j) {
      double acc = 0.0;
      const double* b = Bt + (size_t)j * K;
      for (int k = 0; k < K; ++k) acc += arow[k] * b[k];
      C[(size_t)(i - row0) * N + j] = acc;
    }
    free(arow);
  }
  free(Bt);
  (void)nthreads;
}

/* ------------------------------------------------------------------ */
/* int8 conv2d, NHWC activations, OHWI weights, zero padding, per-output */
/* channel requant (benchmark definition; the reference ships only the   */
/* generated control code of a conv graph, thirdparty/adf/              */
/* aie_control.cpp:854-1524, with no kernel source).  Direct 7-deep     */
/* loop nest n,h,w,co,r,s,ci.  Y32 (nullable) gets the accumulators.    */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_conv2d_nhwc_i8(const int8_t* X, const int8_t* W, const uint8_t* shifts,
                                      int8_t* Y, int32_t* Y32, int N, int H, int Wd, int Cin,
                                      int Cout, int R, int S, int stride, int pad, int relu,
                                      int nthreads) {
  const int Ho = (H + 2 * pad - R) / stride + 1;
  const int Wo = (Wd + 2 * pad - S) / stride + 1;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int n = 0; n < N; ++n)
    for (int ho = 0; ho < Ho; ++ho)
      for (int wo = 0; wo < Wo; ++wo)
        for (int co = 0; co < Cout; ++co) {
          uint32_t acc = 0;
          for (int r = 0; r < R; ++r) {
            int hi = ho * stride + r - pad;
            if (hi < 0 || hi >= H) continue;
            for (int s = 0; s < S; ++s) {
              int wi = wo * stride + s - pad;
              if (wi < 0 || wi >= Wd) continue;
              const int8_t* x = X + (((size_t)n * H + hi) * Wd + wi) * Cin;
              const int8_t* w = W + (((size_t)co * R + r) * S + s) * Cin;
              for (int ci = 0; ci < Cin; ++ci) acc += (uint32_t)((int32_t)x[ci] * (int32_t)w[ci]);
            }
          }
          size_t o = (((size_t)n * Ho + ho) * Wo + wo) * Cout + co;
          Y[o] = oracle_requant((int32_t)acc, shifts[co], relu);
          if (Y32) Y32[o] = (int32_t)acc;
        }
  (void)nthreads;
}

/* ------------------------------------------------------------------ */
/* Chained int8 MLP (the example/multi/multi_tile.cpp:39-47,125-127     */
/* k1 -> k2 chain at scale; benchmark definition):                       */
/*   H = relu(rq_s1(X . W1)),  Y = rq_s2(H . W2), all NN, int32 acc.      */
/* Rows [row0,row1) of Y (each row of Y needs only the same row of H).   */
/* ------------------------------------------------------------------ */
ORACLE_API int oracle_mlp_i8_rows(const int8_t* X, const int8_t* W1, const int8_t* W2, int8_t* Y,
                                  int8_t* H_out, int M, int K, int F, int Nout, int s1, int s2,
                                  int row0, int row1, int nthreads) {
  size_t rows = (size_t)(row1 - row0);
  int8_t* H = (int8_t*)malloc(rows * (size_t)F + 1);
  if (!H) return -1;
  int rc = oracle_gemm_i8_rq_rows(X + (size_t)row0 * K, W1, H, NULL, (int)rows, F, K, 0, s1, 1, 0,
                                  (int)rows, nthreads);
  if (rc == 0)
    rc = oracle_gemm_i8_rq_rows(H, W2, Y + (size_t)row0 * Nout, NULL, (int)rows, Nout, F, 0, s2, 0,
                                0, (int)rows, nthreads);
  if (rc == 0 && H_out) memcpy(H_out + (size_t)row0 * F, H, rows * (size_t)F);
  free(H);
  (void)M;
  return rc;
}

/* ------------------------------------------------------------------ */
/* example/nokernelload/aie_nokernelload.cc:50-83: the uint8 dot-product */
/* MAC probe.  Note the operator precedence of :67-68:                   */
/* vec1[i] = (i + (p&1)) ? 1 : 2 and vec2[i] = (0 + (p&1)) ? 1 : 2.      */
/* out = {num, 4567, ret, 3, vec1[0]} (uint32, wrap-around).             */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_dot_u8_probe(const uint32_t* in, uint32_t* out) {
  uint32_t param_nn = in[0];
  uint8_t vec1[128], vec2[128];
  for (uint32_t i = 0; i < 128; ++i) {
    vec1[i] = (i + (param_nn & 1)) ? 1 : 2;
    vec2[i] = (0 + (param_nn & 1)) ? 1 : 2;
  }
  uint32_t dot = 0;
  for (int j = 0; j < 128; ++j) dot += (uint32_t)vec1[j] * (uint32_t)vec2[j];
  /* 3 * param_nn repetitions of the same 128-MAC dot product (mod 2^32) */
  uint64_t reps = 3ull * (uint64_t)param_nn;
  uint32_t ret = (uint32_t)((uint64_t)dot * (reps & 0xFFFFFFFFull));
  out[0] = (uint32_t)reps;
  out[1] = 4567;
  out[2] = ret;
  out[3] = 3;
  out[4] = vec1[0];
}

/* ------------------------------------------------------------------ */
/* example/multi/vek385_verification.cpp:56-69: out = in . in (NN) for a */
/* square n x n matrix of uint64, with the sum held in an `int` and the  */
/* iteration counter at out[n*n].  `iters` passes (the reference loops   */
/* forever; every pass writes the same values).                         */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_mm_square_u64(const uint64_t* in, uint64_t* out, int n, uint64_t iters) {
  for (int i = 0; i < n; ++i)
    for (int j = 0; j < n; ++j) {
      uint32_t sum = 0; /* `int sum` of the reference, kept wrap-around defined */
      for (int k = 0; k < n; ++k) sum += (uint32_t)(in[i * n + k] * in[k * n + j]);
      out[i * n + j] = (uint64_t)(int64_t)(int32_t)sum;
    }
  out[n * n] = iters;
}

/* ------------------------------------------------------------------ */
/* example/multi/multi_tile.cpp:39-47 and seq_full_col.cpp:39-47: each   */
/* stage writes out[i] = in[0] + addend for i < len; stages chain.       */
/* ------------------------------------------------------------------ */
ORACLE_API void oracle_chain_add(const int32_t* in, int32_t* out, int len, const int32_t* addends,
                                 int nstages) {
  int32_t v = in[0];
  for (int s = 0; s < nstages; ++s) v = (int32_t)((uint32_t)v + (uint32_t)addends[s]);
  for (int i = 0; i < len; ++i) out[i] = v;
}

ORACLE_API int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
