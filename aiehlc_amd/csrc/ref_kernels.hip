// gfx950 counterparts of the reference's single-tile AIE kernels.
//
//   mm_window_i32      `mm`   example/matrixmultiply/aieml_mm.cc:41-93 and
//                      `perf` example/perf/aieml_perf.cc:61-83 (packed A||B
//                      window, NT, int32 wrap-around; int32 operands have no
//                      MFMA form, so this is an LDS-tiled VALU kernel)
//   dot_u8_probe       `perf` example/nokernelload/aie_nokernelload.cc:50-83
//                      (uint8 MAC probe, run on int8 MFMA over the whole GPU)
//   mm_square_u64      `mm`   example/multi/vek385_verification.cpp:56-69,
//                      replicated over a batch as the reference replicates it
//                      over every tile (:208-215)
//   chain_add_i32      `k1`/`k2` example/multi/multi_tile.cpp:39-47 and
//                      seq_full_col.cpp:39-47, chained on the device
#include "miaie_internal.hpp"

namespace {

// ---------------------------------------------------------------- mm window
constexpr int WT = 16;

__global__ __launch_bounds__(256) void mm_window_i32(const int32_t* __restrict__ win, int32_t* __restrict__ out,
                                                     int n) {
  __shared__ uint32_t as[WT][WT + 1];
  __shared__ uint32_t bs[WT][WT + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int i = blockIdx.y * WT + ty;  // output row
  const int j = blockIdx.x * WT + tx;  // output column
  const int32_t* A = win;
  const int32_t* Bt = win + (size_t)n * n;  // [N][K]
  uint32_t acc = 0;
  for (int k0 = 0; k0 < n; k0 += WT) {
    const int ar = blockIdx.y * WT + ty, ak = k0 + tx;
    as[ty][tx] = (ar < n && ak < n) ? (uint32_t)MIAIE_LD(A + (size_t)ar * n + ak) : 0u;
    const int br = blockIdx.x * WT + ty;
    bs[ty][tx] = (br < n && ak < n) ? (uint32_t)MIAIE_LD(Bt + (size_t)br * n + ak) : 0u;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < WT; ++k) acc += as[ty][k] * bs[tx][k];
    __syncthreads();
  }
  if (i < n && j < n) MIAIE_ST(out + (size_t)i * n + j, (int32_t)acc);
}

// ---------------------------------------------------------------- dot probe
// The reference repeats one 128-element uint8 dot product 3*param_nn times.
// Here 4 MFMA 32x32x32 (one per 32-element chunk) compute that dot into all
// 1024 accumulator elements at once, i.e. 1024 repetitions = 131072 MACs,
// exactly the reference's MACs for those repetitions.  Whole groups of 1024
// repetitions are dealt over all waves of the grid; the remainder (< 1024)
// is added on the VALU.  Sums are uint32 with wrap-around, like `ret`.
__device__ __forceinline__ uint32_t probe_vec1(uint32_t i, uint32_t p) { return (i + (p & 1u)) ? 1u : 2u; }
__device__ __forceinline__ uint32_t probe_vec2(uint32_t p) { return (0u + (p & 1u)) ? 1u : 2u; }

__global__ void dot_probe_init(const uint32_t* __restrict__ in, uint32_t* __restrict__ out) {
  if (threadIdx.x != 0) return;
  const uint32_t p = MIAIE_LD(in);
  const uint64_t reps = 3ull * p;
  uint32_t dot = 0;
  for (uint32_t j = 0; j < 128; ++j) dot += probe_vec1(j, p) * probe_vec2(p);
  const uint32_t rem = (uint32_t)(reps % 1024u);
  MIAIE_ST(out + 0, (uint32_t)reps);
  MIAIE_ST(out + 1, 4567u);
  MIAIE_ST(out + 2, rem * dot);  // the MFMA kernel adds the whole groups
  MIAIE_ST(out + 3, 3u);
  MIAIE_ST(out + 4, probe_vec1(0, p));
}

__global__ __launch_bounds__(256) void dot_probe_mfma(const uint32_t* __restrict__ in, uint32_t* __restrict__ out) {
  const uint32_t p = MIAIE_LD(in);
  const uint64_t groups = (3ull * p) / 1024u;
  const int lane = threadIdx.x & 63;
  const uint64_t wave_id = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const uint64_t nwaves = (uint64_t)gridDim.x * (blockDim.x >> 6);
  // operand bytes: lane supplies k = 16*(lane/32) + b of each 32-element chunk
  v4i a[4], bv;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) v |= probe_vec1(32 * c + 16 * (lane >> 5) + 4 * q + b, p) << (8 * b);
      w[q] = v;
    }
    a[c] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
  const uint32_t v2 = probe_vec2(p) * 0x01010101u;
  bv = v4i{(int)v2, (int)v2, (int)v2, (int)v2};
  v16i acc = v16i{0};
  for (uint64_t g = wave_id; g < groups; g += nwaves) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c], bv, acc, 0, 0, 0);
  }
  uint32_t s = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += (uint32_t)acc[e];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0 && s && MIAIE_CHECK(out + 2, sizeof(uint32_t), 1)) atomicAdd(out + 2, s);
}

// ---------------------------------------------------------------- 3x3 NN, replicated
__global__ __launch_bounds__(256) void mm_square_u64(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                     int n, uint64_t iters) {
  const int b = blockIdx.x;
  const uint64_t* a = in + (size_t)b * n * n;
  uint64_t* o = out + (size_t)b * (n * n + 1);
  for (uint64_t it = 0; it < iters; ++it) {
    for (int e = threadIdx.x; e < n * n; e += blockDim.x) {
      const int i = e / n, j = e - i * n;
      uint32_t sum = 0;  // the reference's `int sum`
      for (int k = 0; k < n; ++k) sum += (uint32_t)(MIAIE_LD(a + i * n + k) * MIAIE_LD(a + k * n + j));
      MIAIE_ST(o + e, (uint64_t)(int64_t)(int32_t)sum);
    }
    __syncthreads();
    if (threadIdx.x == 0) MIAIE_ST(o + n * n, it + 1);
  }
}

// ---------------------------------------------------------------- k1 -> k2 chain
struct ChainArgs {
  int32_t add[64];
};

__global__ __launch_bounds__(256) void chain_add_i32(const int32_t* __restrict__ in, int32_t* __restrict__ out,
                                                     int len, ChainArgs args, int nstages) {
  // every stage writes out[i] = in[0] + addend for all i, and the next stage
  // reads element 0 of that output
  uint32_t v = (uint32_t)MIAIE_LD(in);
  for (int s = 0; s < nstages; ++s) v += (uint32_t)args.add[s];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < len; i += gridDim.x * blockDim.x) MIAIE_ST(out + i, (int32_t)v);
}

}  // namespace

using namespace miaie;

extern "C" int miaie_mm_window_i32(miaie_ctx* ctx, const int32_t* in, int32_t* out, int n) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, in);
  MIAIE_CHECK_NOT_NULL(ctx, out);
  if (n < 1 || n > 4096) return fail(ctx, MIAIE_EINVAL, "miaie_mm_window_i32: n=%d outside [1, 4096]", n);
  if (!aligned(in, 4) || !aligned(out, 4)) return fail(ctx, MIAIE_EINVAL, "miaie_mm_window_i32: misaligned buffer");
  dim3 grid((n + WT - 1) / WT, (n + WT - 1) / WT);
  return check_launch(ctx, launch<mm_window_i32>(ctx->device, grid, dim3(256), 0, ctx->stream, in, out, n), "mm_window_i32");
}

extern "C" int miaie_perf_window_u32(miaie_ctx* ctx, const uint32_t* in, uint32_t* out, int n) {
  // uint32 and int32 wrap-around products and sums have the same bits
  return miaie_mm_window_i32(ctx, reinterpret_cast<const int32_t*>(in), reinterpret_cast<int32_t*>(out), n);
}

extern "C" int miaie_dot_u8_probe(miaie_ctx* ctx, const uint32_t* in, uint32_t* out) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, in);
  MIAIE_CHECK_NOT_NULL(ctx, out);
  if (!aligned(in, 4) || !aligned(out, 4)) return fail(ctx, MIAIE_EINVAL, "miaie_dot_u8_probe: misaligned buffer");
  rc = check_launch(ctx, launch<dot_probe_init>(ctx->device, dim3(1), dim3(64), 0, ctx->stream, in, out), "dot_probe_init");
  if (rc) return rc;
  // 1024 workgroups x 4 waves: per-wave group counts stay far below the
  // int32 accumulator range (dot <= 512, groups per wave <= 3*2^32/2^22).
  return check_launch(ctx, launch<dot_probe_mfma>(ctx->device, dim3(1024), dim3(256), 0, ctx->stream, in, out),
                      "dot_probe_mfma");
}

extern "C" int miaie_mm_square_u64(miaie_ctx* ctx, const uint64_t* in, uint64_t* out, int n, int batch,
                                   uint64_t iters) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, in);
  MIAIE_CHECK_NOT_NULL(ctx, out);
  if (n < 1 || n > 64) return fail(ctx, MIAIE_EINVAL, "miaie_mm_square_u64: n=%d outside [1, 64]", n);
  if (batch < 1 || batch > (1 << 24)) return fail(ctx, MIAIE_EINVAL, "miaie_mm_square_u64: batch=%d", batch);
  if (iters < 1 || iters > (1ull << 20) || iters * (uint64_t)n * n * n > (1ull << 34))
    return fail(ctx, MIAIE_EINVAL, "miaie_mm_square_u64: iters must be in [1, 2^20] with iters*n^3 <= 2^34");
  if (!aligned(in, 8) || !aligned(out, 8)) return fail(ctx, MIAIE_EINVAL, "miaie_mm_square_u64: misaligned buffer");
  return check_launch(ctx, launch<mm_square_u64>(ctx->device, dim3(batch), dim3(64), 0, ctx->stream, in, out, n, iters),
                      "mm_square_u64");
}

extern "C" int miaie_chain_add_i32(miaie_ctx* ctx, const int32_t* in, int32_t* out, int len, const int32_t* addends,
                                   int nstages) {
  int rc = enter(ctx);
  if (rc) return rc;
  MIAIE_CHECK_NOT_NULL(ctx, in);
  MIAIE_CHECK_NOT_NULL(ctx, out);
  if (len < 1) return fail(ctx, MIAIE_EINVAL, "miaie_chain_add_i32: len=%d", len);
  if (nstages < 0 || nstages > 64) return fail(ctx, MIAIE_EINVAL, "miaie_chain_add_i32: nstages=%d outside [0, 64]", nstages);
  if (nstages > 0 && !addends) return fail(ctx, MIAIE_EINVAL, "miaie_chain_add_i32: addends is NULL");
  ChainArgs args{};
  for (int s = 0; s < nstages; ++s) args.add[s] = addends[s];
  const int blocks = (len + 255) / 256 < 1024 ? (len + 255) / 256 : 1024;
  return check_launch(ctx, launch<chain_add_i32>(ctx->device, dim3(blocks), dim3(256), 0, ctx->stream, in, out, len, args,
                                                 nstages),
                      "chain_add_i32");
}
