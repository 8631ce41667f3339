// bf16 x bf16 -> fp32 GEMM on gfx950 MFMA (v_mfma_f32_32x32x16_bf16).
//
// The benchmark's bf16 -> fp32 path; the reference has no bf16 kernel (its
// only float check is the elementwise square of example/other/
// aieml_apu.cc:149-156 with an absolute tolerance of 1e-2 at :190).
//
// Same geometry as the int8 kernel: a row of an LDS tile is 64 bytes
// (32 bf16 of k), read as 16-byte MFMA fragments with the same XOR swizzle;
// the row-major B operand is 16-bit-transposed in registers on its way to LDS.
//   gemm_bf16_tile256  256x256x32, 4 waves x (4x4 MFMA 32x32x16), LDS double buffer.
//   gemm_bf16_tile64   64x64x32 bounds-checked fallback.
#include "miaie_internal.hpp"

namespace {

__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 64 + ((chunk ^ swz(row)) << 4); }

__device__ __forceinline__ v8bf as_bf(v4i x) { return __builtin_bit_cast(v8bf, x); }

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int TILE_BYTES = BM * BK * 2;  // 16 KiB per operand per buffer

__global__ __launch_bounds__(256, 1) void gemm_bf16_tile256(const uint16_t* __restrict__ A,
                                                            const uint16_t* __restrict__ B,
                                                            float* __restrict__ C, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) int8_t lds[4 * TILE_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  const int TM = M / BM, TN = N / BN, T = TM * TN;
  const int b = blockIdx.x;
  const int logical = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
  constexpr int GROUP_M = 4;
  const int group_size = GROUP_M * TN;
  const int first_m = (logical / group_size) * GROUP_M;
  const int gm = min(TM - first_m, GROUP_M);
  const int tm = first_m + (logical % group_size) % gm;
  const int tn = (logical % group_size) / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  // A: rows tid/4 + 64i, 16-byte chunk tid%4 (8 bf16 of k)
  const int a_row = tid >> 2, a_chunk = tid & 3;
  const uint16_t* a_src = A + (size_t)(m0 + a_row) * K + a_chunk * 8;
  int a_dst[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a_dst[i] = lds_off(a_row + 64 * i, a_chunk);

  // B (K x N): lane g of wave w holds columns n = 2p, 2p+1 with
  // p = g + 64*(w&1), for k-blocks kb = 2*(w>>1) + u (u < 2), 8 rows each.
  // Output q goes to row 2p + ((q + f) & 1), f = ((g>>2) ^ (g>>3)) & 1, which
  // spreads one store instruction over distinct banks.
  const int p = lane + 64 * (wave & 1);
  const int kb0 = 2 * (wave >> 1);
  const uint16_t* b_src = B + (size_t)(kb0 * 8) * N + n0 + 2 * p;
  const int f = ((lane >> 2) ^ (lane >> 3)) & 1;
  const uint32_t sel_q0 = f ? 0x07060302u : 0x05040100u;
  const uint32_t sel_q1 = f ? 0x05040100u : 0x07060302u;
  int b_dst[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int q = 0; q < 2; ++q) b_dst[u][q] = lds_off(2 * p + ((q + f) & 1), kb0 + u);

  v4i ra[4];
  uint32_t rb[16];

  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = *reinterpret_cast<const v4i*>(a_src + (size_t)(64 * i) * K + k0);
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) rb[kk] = *reinterpret_cast<const uint32_t*>(b_src + (size_t)(k0 + kk) * N);
  };

  auto store_lds = [&](int buf) {
    int8_t* as = lds + buf * 2 * TILE_BYTES;
    int8_t* bs = as + TILE_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(as + a_dst[i]) = ra[i];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      v4i o0, o1;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t x0 = rb[8 * u + 2 * d], x1 = rb[8 * u + 2 * d + 1];
        o0[d] = (int)__builtin_amdgcn_perm(x1, x0, sel_q0);
        o1[d] = (int)__builtin_amdgcn_perm(x1, x0, sel_q1);
      }
      *reinterpret_cast<v4i*>(bs + b_dst[u][0]) = o0;
      *reinterpret_cast<v4i*>(bs + b_dst[u][1]) = o1;
    }
  };

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

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16f{0.f};

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
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(bf[j]), as_bf(af[i]), acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_lds(cur ^ 1);
    __syncthreads();
  }

  // acc[i][j][4g + t]: row m = wm*128 + 32i + lane%32, column n = wn*128 + 32j + 8g + 4*(lane/32) + t
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + wm * 128 + 32 * i + fr;
        const int n = n0 + wn * 128 + 32 * j + 8 * g + 4 * fh;
        v4f v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        *reinterpret_cast<v4f*>(C + (size_t)m * N + n) = v;
      }
}

__global__ __launch_bounds__(256) void gemm_bf16_tile64(const uint16_t* __restrict__ A,
                                                        const uint16_t* __restrict__ B,
                                                        float* __restrict__ C, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) int8_t as[64 * 64];
  __shared__ __attribute__((aligned(16))) int8_t bs[64 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  v16f acc = v16f{0.f};
  for (int k0 = 0; k0 < K; k0 += 32) {
    {
      const int row = tid >> 2, ch = tid & 3;
      const int m = m0 + row, k = k0 + ch * 8;
      uint16_t tmp[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) tmp[t] = (m < M && k + t < K) ? A[(size_t)m * K + k + t] : 0;
      v4i v;
      __builtin_memcpy(&v, tmp, 16);
      *reinterpret_cast<v4i*>(as + lds_off(row, ch)) = v;
    }
    {
      const int col = tid & 63, ch = tid >> 6;
      const int n = n0 + col;
      uint16_t tmp[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int k = k0 + ch * 8 + t;
        tmp[t] = (n < N && k < K) ? B[(size_t)k * N + n] : 0;
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
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(bf), as_bf(af), acc, 0, 0, 0);
    }
    __syncthreads();
  }
  const int m = m0 + wm * 32 + fr;
  if (m >= M) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int n = n0 + wn * 32 + 8 * (e >> 2) + 4 * fh + (e & 3);
    if (n < N) C[(size_t)m * N + n] = acc[e];
  }
}

}  // namespace

namespace miaie {

int launch_gemm_bf16(miaie_ctx* ctx, const uint16_t* A, const uint16_t* B, float* C, int M, int N, int K) {
  const bool big = M % BM == 0 && N % BN == 0 && K % BK == 0 && N % 2 == 0 && aligned(A, 16) &&
                   aligned(B, 16) && aligned(C, 16);
  if (big) {
    hipLaunchKernelGGL(gemm_bf16_tile256, dim3((M / BM) * (N / BN)), dim3(256), 0, ctx->stream, A, B, C, M, N, K);
    return check_launch(ctx, "gemm_bf16_tile256");
  }
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  if (grid.y > 65535) return fail(ctx, MIAIE_EINVAL, "gemm_bf16: M too large for the 64x64 fallback");
  hipLaunchKernelGGL(gemm_bf16_tile64, grid, dim3(256), 0, ctx->stream, A, B, C, M, N, K);
  return check_launch(ctx, "gemm_bf16_tile64");
}

}  // namespace miaie
