// int8 x int8 -> int32 GEMM on gfx950 MFMA, with the fused requantize epilogue.
//
// Counterpart of the AIE `mm`/`perf` MAC loops (example/matrixmultiply/
// aieml_mm.cc:68-76, example/perf/aieml_perf.cc:69-82) generalised to int8
// operands and any M, N, K, and of the 64x64 sub-tiling that aiehlc's
// tiling prototype plans (src/mlir/mlirfront/tilinglinalg/tilinglinalg.cpp:101-103).
//
// Kernels:
//   gemm_i8_pipe    BM x BN x 64 workgroup tiles (256x256, 256x128, 128x128),
//                   4 waves of BM/2 x BN/2, v_mfma_i32_32x32x32_i8; a 4-stage
//                   LDS pipeline (the DMA ping-pong of aietypes.td:56-76 / the
//                   BD pairs of aie_control.cpp:854-875, generalised) filled
//                   by global_load_lds_dwordx4; the row-major (NN) B operand
//                   is transposed by ds_read_b64_tr_b8 on its way out of LDS.
//                   XCD-aware tile order.  K % 64 == 0, M >= BM, N >= BN;
//                   a tile that does not divide M (N) has its last tile row
//                   (column) moved back to end at M (N), overlapping the one
//                   before it (dev::tile_origin), which needs N % 16 == 0
//                   when BN does not divide N (16-byte column chunks).
//   gemm_i8_pipe16  256-row tiles with K % 128 == 0: the same pipeline with A
//                   staged two k-tiles at a time (A copies move whole cache
//                   lines), multiplied on v_mfma_i32_16x16x64_i8, which runs
//                   at a higher clock than the 32x32 form under the power
//                   limit; gemm_i8_pipe16_mixed puts 256x256 and 256x128
//                   tiles in one launch.
//   gemm_i8_tile64p 64x64x64 tile for K % 16 == 0 and 16-byte aligned rows:
//                   clamped vector loads, next k-tile prefetched into
//                   registers.
//   gemm_i8_tile64  64x64x64 tile, bounds-checked, any shape / stride.
// The requantize epilogue (round, shift, saturate, optional ReLU) is fused
// into all of them.
//
// MFMA operand roles are swapped (srcA = B fragment, srcB = A fragment) so
// that each lane's accumulator holds 4 consecutive output columns of one row:
// one dword of int8 output or one 16-byte int32 vector per 4 values.
#include <type_traits>

#include "gemm_i8_kernels.hpp"
#include "gfx950_ops.hpp"
#include "miaie_internal.hpp"

namespace {

namespace dev = miaie::dev;
using namespace miaie::gemm;
using miaie::kernel_t;
using miaie::launch;

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
          v = MIAIE_LD(reinterpret_cast<const v4i*>(p));
        } else {
          int8_t tmp[16];
#pragma unroll
          for (int t = 0; t < 16; ++t) tmp[t] = (k + t < K) ? MIAIE_LD(p + t) : 0;
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
          v = MIAIE_LD(reinterpret_cast<const v4i*>(p));
        } else {
          int8_t tmp[16];
#pragma unroll
          for (int t = 0; t < 16; ++t) tmp[t] = (k + t < K) ? MIAIE_LD(p + t) : 0;
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
        tmp[t] = (n < N && k < K) ? MIAIE_LD(B + (size_t)k * ldb + n) : 0;
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
      if (C) MIAIE_ST(C + (size_t)m * ldc + n, acc[e]);
      if (Y) MIAIE_ST(Y + (size_t)m * ldy + n, (int8_t)requant1(acc[e], shift, relu));
    }
  }
}

// The 64x64 kernel for K % 16 == 0 and 16-byte aligned operands (a ragged M,
// N or K): every load is a full vector from a clamped, always valid address,
// zeroed when written to LDS if outside the matrix, and the next k-tile's
// loads are issued before this k-tile's LDS reads and MFMAs, so their
// latency overlaps the MFMAs (a load under a condition, or zeroed in place,
// would be waited for on the spot).
template <bool B_NT>
__global__ __launch_bounds__(256) void gemm_i8_tile64p(const int8_t* __restrict__ A,
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

  // A (and NT B): thread -> row tid/4, 16-byte chunk tid%4.  K % 16 == 0, so
  // a chunk lies wholly inside or wholly past K; one past K loads the last
  // chunk of its row instead and is zeroed like a row outside the matrix.
  const int row = tid >> 2, ch = tid & 3;
  const bool a_in = m0 + row < M;
  const int8_t* const a_p = A + (size_t)min(m0 + row, M - 1) * lda;
  // NT B: row n0 + row; NN B: column n0 + tid%64, k-chunk tid/64 (16 byte loads down the column)
  const int bcol = tid & 63, bch = tid >> 6;
  const bool b_in = B_NT ? n0 + row < N : n0 + bcol < N;
  const int8_t* const b_p = B_NT ? B + (size_t)min(n0 + row, N - 1) * ldb : B + min(n0 + bcol, N - 1);
  const int bk = B_NT ? ch : bch;  // this thread's k-chunk of B

  auto load = [&](int k0, v4i& va, v4i& vb) {
    va = MIAIE_LD(reinterpret_cast<const v4i*>(a_p + min(k0 + 16 * ch, K - 16)));
    if constexpr (B_NT) {
      vb = MIAIE_LD(reinterpret_cast<const v4i*>(b_p + min(k0 + 16 * ch, K - 16)));
    } else {
      const int8_t* const p = b_p + (size_t)min(k0 + 16 * bch, K - 16) * ldb;
      int8_t tmp[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) tmp[t] = MIAIE_LD(p + (size_t)t * ldb);
      __builtin_memcpy(&vb, tmp, 16);
    }
  };

  v16i acc = v16i{0};
  v4i va, vb;
  load(0, va, vb);
  for (int k0 = 0; k0 < K; k0 += 64) {
    *reinterpret_cast<v4i*>(as + lds_off(row, ch)) = a_in && k0 + 16 * ch < K ? va : v4i{0};
    if constexpr (B_NT)
      *reinterpret_cast<v4i*>(bs + lds_off(row, ch)) = b_in && k0 + 16 * bk < K ? vb : v4i{0};
    else
      *reinterpret_cast<v4i*>(bs + lds_off(bcol, bch)) = b_in && k0 + 16 * bk < K ? vb : v4i{0};
    __syncthreads();
    if (k0 + 64 < K) load(k0 + 64, va, vb);
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
      if (C) MIAIE_ST(C + (size_t)m * ldc + n, acc[e]);
      if (Y) MIAIE_ST(Y + (size_t)m * ldy + n, (int8_t)requant1(acc[e], shift, relu));
    }
  }
}

// keep_y: the caller reads Y right after (the MLP's H): ordinary stores that
// leave it in the caches (instantiated for NN B with ReLU, the MLP's form;
// other calls ignore it).
template <int BM, int BN, bool B_NT>
hipError_t launch_pipe(int device, hipStream_t st, const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C, int M,
                       int N, int K, int lda, int ldb, int ldy, int ldc, int shift, int relu, bool keep_y) {
  // 128x128 tiles (small grids, where the power limit does not bind): two
  // waves per SIMD, so one wave's MFMAs run while the other waits at the
  // k-tile's barrier or for its LDS reads
  constexpr int NW = BM == 128 ? 8 : 4;
  dim3 grid(((M + BM - 1) / BM) * ((N + BN - 1) / BN)), block(64 * NW);
  const int yq = !Y ? Y_NONE : shift < 8 ? Y_MED3 : relu ? Y_HI_RELU : Y_HI;
  hipError_t e = hipSuccess;
  auto go = [&](auto k) {
    e = launch<decltype(k)::value>(device, grid, block, 0, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu);
  };
  auto go2 = [&](auto k) {
    e = launch<decltype(k)::value>(device, grid, block, 0, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu,
                                   nullptr);
  };
  // 256-row tiles with K a multiple of 128: A staged two k-tiles at a time,
  // 16x16x64 MFMAs (gemm_i8_pipe16).  128x128 tiles keep gemm_i8_pipe.
  if constexpr (BM == 256) {
    if (K % 128 == 0) {
      if constexpr (!B_NT) {
        if (keep_y && Y && !C && relu) {
          if (yq == Y_HI_RELU)
            go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, false, Y_HI_RELU, false, false, true>>{});
          else
            go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, false, Y_MED3, false, false, true>>{});
          return e;
        }
      }
      if (C) {
        switch (yq) {
          case Y_NONE: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_NONE, true>>{}); break;
          case Y_MED3: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_MED3, true>>{}); break;
          case Y_HI: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_HI, true>>{}); break;
          default: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_HI_RELU, true>>{}); break;
        }
      } else {
        switch (yq) {
          case Y_MED3: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_MED3, false>>{}); break;
          case Y_HI: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_HI, false>>{}); break;
          default: go2(kernel_t<gemm_i8_pipe16<BM, BN, NW, B_NT, Y_HI_RELU, false>>{}); break;
        }
      }
      return e;
    }
  }
  if (C) {
    switch (yq) {
      case Y_NONE: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_NONE, true>>{}); break;
      case Y_MED3: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_MED3, true>>{}); break;
      case Y_HI: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_HI, true>>{}); break;
      default: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_HI_RELU, true>>{}); break;
    }
  } else {
    switch (yq) {
      case Y_MED3: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_MED3, false>>{}); break;
      case Y_HI: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_HI, false>>{}); break;
      default: go(kernel_t<gemm_i8_pipe<BM, BN, NW, B_NT, Y_HI_RELU, false>>{}); break;
    }
  }
  return e;
}

template <bool B_NT>
hipError_t launch_pipe_mixed(int device, hipStream_t st, const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C,
                             int M, int N, int K, int lda, int ldb, int ldy, int ldc, int shift, int relu, int nw,
                             bool keep_y) {
  const dim3 grid(((M + 255) / 256) * (nw + (N - 256 * nw + 127) / 128)), block(256);
  const int yq = !Y ? Y_NONE : shift < 8 ? Y_MED3 : relu ? Y_HI_RELU : Y_HI;
  hipError_t e = hipSuccess;
  auto go = [&](auto k) {
    e = launch<decltype(k)::value>(device, grid, block, 0, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu,
                                   nw);
  };
  if constexpr (!B_NT) {
    if (keep_y && Y && !C && relu) {
      if (yq == Y_HI_RELU)
        go(kernel_t<gemm_i8_pipe16_mixed<false, Y_HI_RELU, false, true>>{});
      else
        go(kernel_t<gemm_i8_pipe16_mixed<false, Y_MED3, false, true>>{});
      return e;
    }
  }
  if (C) {
    switch (yq) {
      case Y_NONE: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_NONE, true>>{}); break;
      case Y_MED3: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_MED3, true>>{}); break;
      case Y_HI: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_HI, true>>{}); break;
      default: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_HI_RELU, true>>{}); break;
    }
  } else {
    switch (yq) {
      case Y_MED3: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_MED3, false>>{}); break;
      case Y_HI: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_HI, false>>{}); break;
      default: go(kernel_t<gemm_i8_pipe16_mixed<B_NT, Y_HI_RELU, false>>{}); break;
    }
  }
  return e;
}

// Tiling planner for the pipelined kernel: picks the workgroup tile
// (BM x BN) among 256x256, 256x128 and 128x128 for an M x N x K product on
// `cus` compute units, or a mix of 256x256 and 256x128 tiles in one launch
// (gemm_i8_pipe16_mixed).  A tile's cost, in units of one 256x256x64 k-tile of
// MFMA work: its K/64 k-tiles plus about 6 units of prologue and epilogue,
// scaled by the tile's relative cost per k-tile (1 for 256x256; 0.55 for
// 256x128; 0.35 for 128x128, whose LDS reads per MFMA are twice those of
// 256x256).  A plan's cost is the finishing time of its tiles dealt in
// launch order to the CU that frees first (the dispatcher's order).
struct TileChoice {
  int bm, bn;
  double unit;
};
constexpr TileChoice kTiles[] = {{256, 256, 1.0}, {256, 128, 0.55}, {128, 128, 0.35}};

struct PipePlan {
  int bm = 0, bn = 0;
  int nw = 0;  // > 0: mixed launch, 256-wide tiles over the first 256 nw columns, 256x128 after
};

// Finishing time of `n1` tasks of length d1 then `n2` of length d2, each
// dealt to the earliest-free of `cus` identical CUs.  CUs that free at the
// same time are kept as one group, so the loop runs once per group and round.
double list_makespan(long n1, double d1, long n2, double d2, int cus) {
  struct Grp {
    double t;
    long n;
  };
  Grp g[8];
  int ng = 1;
  g[0] = {0.0, cus};
  auto deal = [&](long tasks, double d) {
    while (tasks > 0) {
      int k = 0;  // earliest group
      for (int i = 1; i < ng; ++i)
        if (g[i].t < g[k].t) k = i;
      const long take = tasks < g[k].n ? tasks : g[k].n;
      tasks -= take;
      const double t_end = g[k].t + d;
      if (take == g[k].n) {
        g[k].t = t_end;
      } else {
        g[k].n -= take;
        int j = -1;  // merge with a group ending at the same time, else a new one
        for (int i = 0; i < ng; ++i)
          if (g[i].t == t_end) j = i;
        if (j >= 0)
          g[j].n += take;
        else if (ng < 8)
          g[ng++] = {t_end, take};
        else
          return false;
      }
    }
    return true;
  };
  if (!deal(n1, d1) || !deal(n2, d2)) return 1e300;  // (more than 8 distinct finishing times: not planned)
  double t = 0;
  for (int i = 0; i < ng; ++i) t = g[i].t > t ? g[i].t : t;
  return t;
}

PipePlan plan_pipe(int M, int N, int K, int cus) {
  PipePlan best;
  if (K % BK != 0 || cus < 1) return best;
  const double work = K / BK + 6.0;
  // lowest finishing time; among equal ones, the least total CU time (fewer
  // of the costlier narrow tiles, less energy under the power limit)
  double best_cost = 0, best_total = 0;
  auto consider = [&](double cost, double total, PipePlan p) {
    if (best.bm == 0 || cost < best_cost - 1e-9 || (cost < best_cost + 1e-9 && total < best_total - 1e-9)) {
      best_cost = cost;
      best_total = total;
      best = p;
    }
  };
  // A tile that does not divide M or N still takes the shape: the last
  // tile row or column overlaps its neighbour (dev::tile_origin), and is
  // planned as a whole tile.  A moved-back column tile starts on a 16-byte
  // chunk only when N % 16 == 0.
  auto cols_ok = [&](int n, int bn) { return n >= bn && (n % bn == 0 || N % 16 == 0); };
  for (const TileChoice& t : kTiles) {
    if (M < t.bm || !cols_ok(N, t.bn)) continue;
    const long tiles = (long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    consider((double)((tiles + cus - 1) / cus) * t.unit * work, tiles * t.unit * work, PipePlan{t.bm, t.bn, 0});
  }
  // mixed 256x256 + 256x128 (the pair-staged kernel: K % 128 == 0)
  if (M >= 256 && K % 128 == 0) {
    const long tm = (M + 255) / 256;
    for (int nw = 1; cols_ok(N - 256 * nw, 128); ++nw) {
      const long wide = tm * nw, narrow = tm * ((N - 256 * nw + 127) / 128);
      const double dw = kTiles[0].unit * work, dn = kTiles[1].unit * work;
      consider(list_makespan(wide, dw, narrow, dn, cus), wide * dw + narrow * dn, PipePlan{256, 256, nw});
    }
  }
  return best;
}

}  // namespace

namespace miaie {

// The pipelined kernel's operand conditions: 16-byte chunks (16-byte
// aligned operands and strides), per-lane offsets of up to 64 rows in 32
// bits, and the requant shortcut's K < 2^16.
static bool pipe_operands_ok(const int8_t* A, const int8_t* B, const int8_t* Y, const int32_t* C, int K, int lda,
                             int ldb, int ldy, int ldc) {
  return (K % BK == 0) && (!Y || K < (1 << 16)) && aligned(A, 16) && aligned(B, 16) && lda % 16 == 0 &&
         ldb % 16 == 0 && lda < (1 << 25) && ldb < (1 << 25) && (!Y || (aligned(Y, 16) && ldy % 16 == 0)) &&
         (!C || (aligned(C, 16) && ldc % 4 == 0));
}

int plan_gemm_i8(miaie_ctx* ctx, int M, int N, int K, int dense_ok, miaie_gemm_plan* plan) {
  const PipePlan p = dense_ok ? plan_pipe(M, N, K, ctx->cus) : PipePlan{};
  *plan = miaie_gemm_plan{};
  plan->threads = p.bm == 128 ? 512 : 256;
  if (p.bm && p.nw) {
    plan->kernel = MIAIE_KERNEL_PIPE_MIXED;
    plan->tile_m = 256;
    plan->tile_n = 256;
    plan->workgroups = ((M + 255) / 256) * (p.nw + (N - 256 * p.nw + 127) / 128);
  } else if (p.bm) {
    plan->kernel = MIAIE_KERNEL_PIPE;
    plan->tile_m = p.bm;
    plan->tile_n = p.bn;
    plan->workgroups = ((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
  } else {
    plan->kernel = MIAIE_KERNEL_TILE64;
    plan->tile_m = 64;
    plan->tile_n = 64;
    plan->workgroups = ((M + 63) / 64) * ((N + 63) / 64);
  }
  return MIAIE_OK;
}

// Chooses the kernel.  Y and/or C may be NULL (not both).
int launch_gemm_i8(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int8_t* Y, int32_t* C, int M,
                   int N, int K, int lda, int ldb, int ldy, int ldc, int b_nt, int shift, int relu, bool keep_y) {
  miaie_gemm_plan plan;
  const bool dense_ok = pipe_operands_ok(A, B, Y, C, K, lda, ldb, ldy, ldc);
  plan_gemm_i8(ctx, M, N, K, dense_ok, &plan);
  if (plan.kernel == MIAIE_KERNEL_PIPE_MIXED) {
    const int nw = plan_pipe(M, N, K, ctx->cus).nw;
    const int dev = ctx->device;
    const hipError_t e =
        b_nt ? launch_pipe_mixed<true>(dev, ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, nw, keep_y)
             : launch_pipe_mixed<false>(dev, ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, nw,
                                        keep_y);
    return check_launch(ctx, e, "gemm_i8_pipe16_mixed");
  }
  if (plan.kernel == MIAIE_KERNEL_PIPE) {
    hipStream_t st = ctx->stream;
    const int dev = ctx->device, bm = plan.tile_m, bn = plan.tile_n;
    hipError_t e;
    if (bm == 256 && bn == 256)
      e = b_nt ? launch_pipe<256, 256, true>(dev, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, keep_y)
               : launch_pipe<256, 256, false>(dev, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, keep_y);
    else if (bm == 256)
      e = b_nt ? launch_pipe<256, 128, true>(dev, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, keep_y)
               : launch_pipe<256, 128, false>(dev, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, keep_y);
    else
      e = b_nt ? launch_pipe<128, 128, true>(dev, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, keep_y)
               : launch_pipe<128, 128, false>(dev, st, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc, shift, relu, keep_y);
    return check_launch(ctx, e, "gemm_i8_pipe");
  }
  dim3 grid((N + 63) / 64, (M + 63) / 64), block(256);
  if (grid.y > 65535) return fail(ctx, MIAIE_EINVAL, "gemm_i8: M too large for the 64x64 fallback");
  // vector loads need K % 16 == 0 and 16-byte aligned A (and NT B) rows
  const bool vec = K % 16 == 0 && aligned(A, 16) && lda % 16 == 0 && (!b_nt || (aligned(B, 16) && ldb % 16 == 0));
  const int dev = ctx->device;
  if (vec) {
    const hipError_t e =
        b_nt ? launch<gemm_i8_tile64p<true>>(dev, grid, block, 0, ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy,
                                             ldc, shift, relu)
             : launch<gemm_i8_tile64p<false>>(dev, grid, block, 0, ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy,
                                              ldc, shift, relu);
    return check_launch(ctx, e, "gemm_i8_tile64p");
  }
  const hipError_t e =
      b_nt ? launch<gemm_i8_tile64<true>>(dev, grid, block, 0, ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc,
                                          shift, relu)
           : launch<gemm_i8_tile64<false>>(dev, grid, block, 0, ctx->stream, A, B, Y, C, M, N, K, lda, ldb, ldy, ldc,
                                           shift, relu);
  return check_launch(ctx, e, "gemm_i8_tile64");
}

}  // namespace miaie
