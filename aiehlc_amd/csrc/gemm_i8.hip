// int8 x int8 -> int32 GEMM on gfx950 MFMA, with the fused requantize epilogue.
//
// Counterpart of the AIE `mm`/`perf` MAC loops (example/matrixmultiply/
// aieml_mm.cc:68-76, example/perf/aieml_perf.cc:69-82) generalised to int8
// operands and any M, N, K, and of the 64x64 sub-tiling that aiehlc's
// tiling prototype plans (src/mlir/mlirfront/tilinglinalg/tilinglinalg.cpp:101-103).
//
// Two kernels:
//   gemm_i8_tile256  256x256x64 workgroup tile, 4 waves of 128x128, each a
//                    4x4 grid of v_mfma_i32_32x32x32_i8.  LDS double buffer
//                    (the DMA ping-pong of aietypes.td:56-76 / the BD pairs of
//                    aie_control.cpp:854-875) fed by 128-bit global loads; the
//                    row-major (NN) B operand is byte-transposed in registers
//                    with v_perm_b32 on its way to LDS.  XCD-aware tile order.
//                    Requires M, N % 256 == 0, K % 64 == 0 and aligned strides.
//   gemm_i8_tile64   64x64x64 tile, bounds-checked, any shape / stride.
//
// MFMA operand roles are swapped (srcA = B fragment, srcB = A fragment) so
// that each lane's accumulator holds 4 consecutive output columns of one row:
// one dword of int8 output or one 16-byte int32 vector per 4 values.
#include "miaie_internal.hpp"

namespace {

// ------------------------------------------------------------- epilogue
// y = sat_int8(floor((acc + 2^(s-1)) / 2^s)) for s in [1, 31], sat_int8(acc)
// for s == 0; ReLU after the shift.  floor((a + 2^(s-1)) / 2^s) equals
// (a >> s) + bit (s-1) of a, which cannot overflow.
__device__ __forceinline__ int requant1(int acc, int s, int relu) {
  int q = s ? (acc >> s) + ((acc >> (s - 1)) & 1) : acc;
  q = relu ? max(q, 0) : q;
  return min(max(q, -128), 127);
}

__device__ __forceinline__ uint32_t requant4(int a0, int a1, int a2, int a3, int s, int relu) {
  return (uint32_t)(requant1(a0, s, relu) & 0xFF) | ((uint32_t)(requant1(a1, s, relu) & 0xFF) << 8) |
         ((uint32_t)(requant1(a2, s, relu) & 0xFF) << 16) | ((uint32_t)(requant1(a3, s, relu) & 0xFF) << 24);
}

// LDS tile rows are 64 bytes = four 16-byte chunks.  The chunk index is
// XOR-swizzled with bits of the row so that (a) 16 or 8 consecutive rows
// read at one logical chunk (the MFMA fragment pattern), (b) 4 rows x 4
// chunks (the A store pattern) and (c) the rotated transposed-B store
// pattern all fall on distinct banks, for 32- and 64-bank LDS alike.
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 64 + ((chunk ^ swz(row)) << 4); }

// ---------------------------------------------------------- 256x256 tile
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int TILE_BYTES = BM * BK;  // per operand per buffer (16 KiB)

template <bool B_NT, bool WRITE_Y, bool WRITE_C>
__global__ __launch_bounds__(256, 1) void gemm_i8_tile256(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int8_t* __restrict__ Y,
    int32_t* __restrict__ C, int M, int N, int K, int lda, int ldb, int ldy, int ldc, int shift,
    int relu) {
  __shared__ __attribute__((aligned(16))) int8_t lds[4 * TILE_BYTES];  // [buf][A|B] = 64 KiB

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // ---- tile order: each XCD (workgroups are dealt round-robin to the 8
  // XCDs) gets a contiguous run of logical tiles, and logical tiles walk
  // groups of 4 tile-rows column by column, so one XCD's run is a compact
  // block that shares A rows and B columns in its L2.
  const int TM = M / BM, TN = N / BN, T = TM * TN;
  int b = blockIdx.x;
  int logical = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
  constexpr int GROUP_M = 4;
  const int group_size = GROUP_M * TN;
  const int first_m = (logical / group_size) * GROUP_M;
  const int gm = min(TM - first_m, GROUP_M);
  const int tm = first_m + (logical % group_size) % gm;
  const int tn = (logical % group_size) / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  // ---- global -> register staging
  // A: thread loads rows tid/4 + 64*i (i < 4), 16-byte chunk tid%4.
  const int a_row = tid >> 2, a_chunk = tid & 3;
  const int8_t* a_src = A + (size_t)(m0 + a_row) * lda + a_chunk * 16;
  const size_t a_step_rows = (size_t)64 * lda;
  int a_dst[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a_dst[i] = lds_off(a_row + 64 * i, a_chunk);

  // B, NT: same pattern as A.  B, NN: lane g holds columns 4g..4g+3 of
  // 16 k-rows (wave w: rows 16w..16w+15), transposed into four 16-byte
  // k-vectors; lane g stores output q to row 4g + ((q + (g>>2)) & 3) so that
  // one store instruction covers distinct banks.
  const int8_t* b_src;
  size_t b_step;
  int b_dst[4];
  uint32_t sel01 = 0, sel23 = 0;
  if constexpr (B_NT) {
    b_src = B + (size_t)(n0 + a_row) * ldb + a_chunk * 16;
    b_step = (size_t)64 * ldb;
#pragma unroll
    for (int i = 0; i < 4; ++i) b_dst[i] = lds_off(a_row + 64 * i, a_chunk);
  } else {
    b_src = B + (size_t)(wave * 16) * ldb + n0 + 4 * lane;
    b_step = (size_t)ldb;
    const int r = (lane >> 2) & 3;
#pragma unroll
    for (int q = 0; q < 4; ++q) b_dst[q] = lds_off(4 * lane + ((q + r) & 3), wave);
    // stage-1 byte selectors, rotated by r columns: t = [x.b(r), y.b(r), x.b(r+1), y.b(r+1)]
    const uint32_t c0 = r, c1 = (r + 1) & 3, c2 = (r + 2) & 3, c3 = (r + 3) & 3;
    sel01 = c0 | ((4 + c0) << 8) | (c1 << 16) | ((4 + c1) << 24);
    sel23 = c2 | ((4 + c2) << 8) | (c3 << 16) | ((4 + c3) << 24);
  }

  v4i ra[4];
  v4i rbv[4];      // NT staging
  uint32_t rb[16]; // NN staging

  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = *reinterpret_cast<const v4i*>(a_src + i * a_step_rows + k0);
    if constexpr (B_NT) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rbv[i] = *reinterpret_cast<const v4i*>(b_src + i * b_step + k0);
    } else {
#pragma unroll
      for (int kk = 0; kk < 16; ++kk)
        rb[kk] = *reinterpret_cast<const uint32_t*>(b_src + (size_t)(k0 + kk) * b_step);
    }
  };

  auto store_lds = [&](int buf) {
    int8_t* as = lds + buf * 2 * TILE_BYTES;
    int8_t* bs = as + TILE_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(as + a_dst[i]) = ra[i];
    if constexpr (B_NT) {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(bs + b_dst[i]) = rbv[i];
    } else {
      uint32_t o[4][4];  // o[q][d]: column (q + r) & 3, k-rows 4d..4d+3
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t x0 = rb[4 * d], x1 = rb[4 * d + 1], x2 = rb[4 * d + 2], x3 = rb[4 * d + 3];
        const uint32_t t0 = __builtin_amdgcn_perm(x1, x0, sel01);
        const uint32_t t1 = __builtin_amdgcn_perm(x1, x0, sel23);
        const uint32_t t2 = __builtin_amdgcn_perm(x3, x2, sel01);
        const uint32_t t3 = __builtin_amdgcn_perm(x3, x2, sel23);
        o[0][d] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
        o[1][d] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
        o[2][d] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
        o[3][d] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v4i v = {(int)o[q][0], (int)o[q][1], (int)o[q][2], (int)o[q][3]};
        *reinterpret_cast<v4i*>(bs + b_dst[q]) = v;
      }
    }
  };

  // ---- fragment read offsets: rows wm*128 + 32i + lane%32, logical chunk 2ks + lane/32
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  int a_frag[2][4], b_frag[2][4];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a_frag[ks][i] = lds_off(wm * 128 + 32 * i + fr, 2 * ks + fh);
      b_frag[ks][i] = lds_off(wn * 128 + 32 * i + fr, 2 * ks + fh);
    }

  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16i{0};

  const int KT = K / BK;
  load_global(0);
  store_lds(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_global((kt + 1) * BK);
    const int8_t* as = lds + cur * 2 * TILE_BYTES;
    const int8_t* bs = as + TILE_BYTES;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v4i af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const v4i*>(as + a_frag[ks][i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const v4i*>(bs + b_frag[ks][j]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_lds(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue.  acc[i][j][4g + t]: row m = wm*128 + 32i + lane%32,
  // column n = wn*128 + 32j + 8g + 4*(lane/32) + t.
  if constexpr (WRITE_C) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = m0 + wm * 128 + 32 * i + fr;
          const int n = n0 + wn * 128 + 32 * j + 8 * g + 4 * fh;
          v4i v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          *reinterpret_cast<v4i*>(C + (size_t)m * ldc + n) = v;
        }
  }
  if constexpr (WRITE_Y) {
    // Stage the 256x256 int8 tile in LDS (16-byte chunk index XOR row%16),
    // then write it out with fully coalesced 16-byte stores.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = wm * 128 + 32 * i + fr;
          const int n = wn * 128 + 32 * j + 8 * g + 4 * fh;
          const uint32_t packed = requant4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                           acc[i][j][4 * g + 3], shift, relu);
          const int off = m * 256 + ((((n >> 4) ^ (m & 15))) << 4) + (n & 15);
          *reinterpret_cast<uint32_t*>(lds + off) = packed;
        }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int flat = it * 256 + tid;
      const int m = flat >> 4, c = flat & 15;
      const v4i v = *reinterpret_cast<const v4i*>(lds + m * 256 + ((c ^ (m & 15)) << 4));
      *reinterpret_cast<v4i*>(Y + (size_t)(m0 + m) * ldy + n0 + c * 16) = v;
    }
  }
}

// ------------------------------------------------------------ 64x64 tile
// Bounds-checked fallback for shapes and strides the 256 kernel does not take.
template <bool B_NT>
__global__ __launch_bounds__(256) void gemm_i8_tile64(const int8_t* __restrict__ A,
                                                      const int8_t* __restrict__ B,
                                                      int8_t* __restrict__ Y, int32_t* __restrict__ C,
                                                      int M, int N, int K, int lda, int ldb, int ldy,
                                                      int ldc, int shift, int relu) {
  __shared__ __attribute__((aligned(16))) int8_t as[64 * 64];
  __shared__ __attribute__((aligned(16))) int8_t bs[64 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;

  v16i acc = v16i{0};
  for (int k0 = 0; k0 < K; k0 += 64) {
    // A (and NT B): thread -> row tid/4, 16-byte chunk tid%4
    {
      const int row = tid >> 2, ch = tid & 3;
      const int m = m0 + row, k = k0 + ch * 16;
      v4i v = v4i{0};
      if (m < M) {
        const int8_t* p = A + (size_t)m * lda + k;
        if (k + 16 <= K && miaie::aligned(p, 16)) {
          v = *reinterpret_cast<const v4i*>(p);
        } else {
          int8_t tmp[16];
#pragma unroll
          for (int t = 0; t < 16; ++t) tmp[t] = (k + t < K) ? p[t] : 0;
          __builtin_memcpy(&v, tmp, 16);
        }
      }
      *reinterpret_cast<v4i*>(as + lds_off(row, ch)) = v;
    }
    if constexpr (B_NT) {
      const int row = tid >> 2, ch = tid & 3;
      const int n = n0 + row, k = k0 + ch * 16;
      v4i v = v4i{0};
      if (n < N) {
        const int8_t* p = B + (size_t)n * ldb + k;
        if (k + 16 <= K && miaie::aligned(p, 16)) {
          v = *reinterpret_cast<const v4i*>(p);
        } else {
          int8_t tmp[16];
#pragma unroll
          for (int t = 0; t < 16; ++t) tmp[t] = (k + t < K) ? p[t] : 0;
          __builtin_memcpy(&v, tmp, 16);
        }
      }
      *reinterpret_cast<v4i*>(bs + lds_off(row, ch)) = v;
    } else {
      // thread -> column tid%64, k-chunk tid/64: 16 byte loads down the column
      const int col = tid & 63, ch = tid >> 6;
      const int n = n0 + col;
      int8_t tmp[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int k = k0 + ch * 16 + t;
        tmp[t] = (n < N && k < K) ? B[(size_t)k * ldb + n] : 0;
      }
      v4i v;
      __builtin_memcpy(&v, tmp, 16);
      *reinterpret_cast<v4i*>(bs + lds_off(col, ch)) = v;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const v4i af = *reinterpret_cast<const v4i*>(as + lds_off(wm * 32 + fr, 2 * ks + fh));
      const v4i bf = *reinterpret_cast<const v4i*>(bs + lds_off(wn * 32 + fr, 2 * ks + fh));
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af, acc, 0, 0, 0);
    }
    __syncthreads();
  }

  const int m = m0 + wm * 32 + fr;
  if (m >= M) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int n = n0 + wn * 32 + 8 * (e >> 2) + 4 * fh + (e & 3);
    if (n < N) {
      if (C) C[(size_t)m * ldc + n] = acc[e];
      if (Y) Y[(size_t)m * ldy + n] = (int8_t)requant1(acc[e], shift, relu);
    }
  }
}

template <bool B_NT>
void launch_tile256(hipStream_t st, const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C, int M,
                    int N, int K, int lda, int ldb, int ldy, int ldc, int shift, int relu) {
  dim3 grid((M / BM) * (N / BN)), block(256);
  if (Y && C)
    hipLaunchKernelGGL((gemm_i8_tile256<B_NT, true, true>), grid, block, 0, st, A, B, Y, C, M, N, K, lda,
                       ldb, ldy, ldc, shift, relu);
  else if (Y)
    hipLaunchKernelGGL((gemm_i8_tile256<B_NT, true, false>), grid, block, 0, st, A, B, Y, C, M, N, K,
                       lda, ldb, ldy, ldc, shift, relu);
  else
    hipLaunchKernelGGL((gemm_i8_tile256<B_NT, false, true>), grid, block, 0, st, A, B, Y, C, M, N, K,
                       lda, ldb, ldy, ldc, shift, relu);
}

}  // namespace

namespace miaie {

// Chooses the kernel.  Y and/or C may be NULL (not both).
int launch_gemm_i8(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C, int M,
                   int N, int K, int lda, int ldb, int ldy, int ldc, int b_nt, int shift, int relu) {
  const bool big = (M % BM == 0) && (N % BN == 0) && (K % BK == 0) && aligned(A, 16) &&
                   aligned(B, 16) && lda % 16 == 0 && (b_nt ? ldb % 16 == 0 : ldb % 4 == 0) &&
                   (!Y || (aligned(Y, 16) && ldy % 16 == 0)) && (!C || (aligned(C, 16) && ldc % 4 == 0)) &&
                   (size_t)M * lda < ((size_t)1 << 40);
  if (big) {
    if (b_nt)
      launch_tile256<true>(ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu);
    else
      launch_tile256<false>(ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu);
    return check_launch(ctx, "gemm_i8_tile256");
  }
  dim3 grid((N + 63) / 64, (M + 63) / 64), block(256);
  if (grid.y > 65535) return fail(ctx, MIAIE_EINVAL, "gemm_i8: M too large for the 64x64 fallback");
  if (b_nt)
    hipLaunchKernelGGL(gemm_i8_tile64<true>, grid, block, 0, ctx->stream, A, B, Y, C, M, N, K, lda, ldb,
                       ldy, ldc, shift, relu);
  else
    hipLaunchKernelGGL(gemm_i8_tile64<false>, grid, block, 0, ctx->stream, A, B, Y, C, M, N, K, lda, ldb,
                       ldy, ldc, shift, relu);
  return check_launch(ctx, "gemm_i8_tile64");
}

}  // namespace miaie
