// gemm_span — in-kernel clocks of the headline int8 GEMM + requant
// (M = N = K = 4096, A and B row-major, shift 10, Y only).
//
// Runs the library's own kernel template (aiehlc_amd/csrc/gemm_i8_kernels.hpp,
// gemm_i8_pipe16<256, 256, 4, NN, Y_HI, no C>) twice over: the product
// instantiation, and the TIMED one, which records per wave the shader clock
// (s_memtime) at its start, after the prologue's barrier, after the last
// k-tile and at its end, and the 100 MHz wall clock (s_memrealtime) at its
// start and end.  The TIMED output must equal the product output byte for
// byte.  After 0.3 s of back-to-back launches (the GPU leaves its idle
// clocks), it reports from the last of 200 TIMED launches:
//   span_us                first wave's start to last wave's end
//   start_spread_us        last workgroup start after the first
//   end_spread_us          last workgroup end after the first
//   prologue / k-tile / epilogue cycles per workgroup (median and max)
//   clock_ghz              shader cycles per wall-clock ns (median)
//   per_xcd                per XCD (workgroup b runs on XCD b % 8): median
//                          clock and the latest end (us after the first start)
// and the time per back-to-back launch of both instantiations (HIP events).
// Prints one JSON object.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../csrc/gemm_i8_kernels.hpp"

#define CHECK(x)                                                        \
  do {                                                                  \
    hipError_t e_ = (x);                                                \
    if (e_ != hipSuccess) {                                             \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));           \
      exit(1);                                                          \
    }                                                                   \
  } while (0)

namespace {

constexpr int M = 4096, N = 4096, K = 4096, BM = 256, BN = 256, NW = 4, SHIFT = 10;
constexpr int WGS = (M / BM) * (N / BN);

uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  return v[v.size() / 2];
}
double maxv(const std::vector<double>& v) { return *std::max_element(v.begin(), v.end()); }

}  // namespace

int main() {
  using namespace miaie::gemm;
  const size_t ab = (size_t)M * K, bb = (size_t)K * N, yb = (size_t)M * N;
  std::vector<int8_t> ha(ab), hb(bb);
  for (size_t i = 0; i < ab; ++i) ha[i] = (int8_t)(mix(0x100000000ull + i) >> 56);
  for (size_t i = 0; i < bb; ++i) hb[i] = (int8_t)(mix(0x200000000ull + i) >> 56);
  int8_t *A, *B, *Y;
  unsigned long long* P;
  CHECK(hipMalloc(&A, ab));
  CHECK(hipMalloc(&B, bb));
  CHECK(hipMalloc(&Y, yb));
  CHECK(hipMalloc(&P, (size_t)WGS * NW * PROBE_WORDS * sizeof(unsigned long long)));
  CHECK(hipMemcpy(A, ha.data(), ab, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(B, hb.data(), bb, hipMemcpyHostToDevice));
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  auto product = [&]() {
    hipLaunchKernelGGL((gemm_i8_pipe16<BM, BN, NW, false, Y_HI, false, false>), dim3(WGS), dim3(64 * NW), 0, st, A, B,
                       Y, (int32_t*)nullptr, M, N, K, K, N, N, N, SHIFT, 0, (unsigned long long*)nullptr);
  };
  auto timed = [&]() {
    hipLaunchKernelGGL((gemm_i8_pipe16<BM, BN, NW, false, Y_HI, false, true>), dim3(WGS), dim3(64 * NW), 0, st, A, B,
                       Y, (int32_t*)nullptr, M, N, K, K, N, N, N, SHIFT, 0, P);
  };
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  auto per_launch_us = [&](auto fn, int n) {
    for (int i = 0; i < 20; ++i) fn();
    CHECK(hipEventRecord(e0, st));
    for (int i = 0; i < n; ++i) fn();
    CHECK(hipEventRecord(e1, st));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    return ms * 1e3 / n;
  };

  product();
  CHECK(hipGetLastError());
  CHECK(hipStreamSynchronize(st));
  std::vector<int8_t> y0(yb), y1(yb);
  CHECK(hipMemcpy(y0.data(), Y, yb, hipMemcpyDeviceToHost));
  // settle: 0.3 s of back-to-back launches
  const auto s0 = std::chrono::steady_clock::now();
  while (std::chrono::duration<double>(std::chrono::steady_clock::now() - s0).count() < 0.3) {
    for (int i = 0; i < 20; ++i) product();
    CHECK(hipStreamSynchronize(st));
  }
  const double us_product = per_launch_us(product, 200);
  const double us_timed = per_launch_us(timed, 200);  // its last launch leaves the probe words
  CHECK(hipGetLastError());
  CHECK(hipStreamSynchronize(st));
  CHECK(hipMemcpy(y1.data(), Y, yb, hipMemcpyDeviceToHost));
  const bool same = memcmp(y0.data(), y1.data(), yb) == 0;

  std::vector<unsigned long long> h((size_t)WGS * NW * PROBE_WORDS);
  CHECK(hipMemcpy(h.data(), P, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  // per workgroup: wave 0's prologue / main loop / epilogue, and the
  // workgroup's first start and last end over its waves
  std::vector<double> pro, ktile, epi, ghz;
  std::vector<unsigned long long> wstart(WGS, ~0ull), wend(WGS, 0);
  for (int b = 0; b < WGS; ++b) {
    for (int w = 0; w < NW; ++w) {
      const unsigned long long* p = &h[((size_t)b * NW + w) * PROBE_WORDS];
      wstart[b] = std::min(wstart[b], p[4]);
      wend[b] = std::max(wend[b], p[5]);
      if (w == 0) {
        pro.push_back((double)(p[1] - p[0]));
        ktile.push_back((double)(p[2] - p[1]) / (K / 64));
        epi.push_back((double)(p[3] - p[2]));
        ghz.push_back((double)(p[3] - p[0]) / ((double)(p[5] - p[4]) * 10.0));
      }
    }
  }
  const unsigned long long first = *std::min_element(wstart.begin(), wstart.end());
  const unsigned long long last_start = *std::max_element(wstart.begin(), wstart.end());
  const unsigned long long first_end = *std::min_element(wend.begin(), wend.end());
  const unsigned long long last_end = *std::max_element(wend.begin(), wend.end());
  printf("{\"kernel\": \"gemm_i8_pipe16<256, 256, 4, NN, Y_HI>\", \"shape\": [%d, %d, %d], "
         "\"timed_output_equals_product\": %s, \"span_us\": %.2f, \"start_spread_us\": %.2f, \"end_spread_us\": %.2f, "
         "\"prologue_cycles\": [%.0f, %.0f], \"cycles_per_k_tile\": [%.0f, %.0f], \"epilogue_cycles\": [%.0f, %.0f], "
         "\"clock_ghz\": %.3f, \"per_xcd\": [",
         M, N, K, same ? "true" : "false", (last_end - first) / 100.0, (last_start - first) / 100.0,
         (last_end - first_end) / 100.0, median(pro), maxv(pro), median(ktile), maxv(ktile), median(epi), maxv(epi),
         median(ghz));
  for (int x = 0; x < 8; ++x) {
    std::vector<double> g;
    unsigned long long e = 0;
    for (int b = x; b < WGS; b += 8) {
      g.push_back(ghz[b]);
      e = std::max(e, wend[b]);
    }
    printf("%s{\"xcd\": %d, \"clock_ghz\": %.3f, \"last_end_us\": %.2f}", x ? ", " : "", x, median(g),
           (e - first) / 100.0);
  }
  printf("], \"us_per_launch_product\": %.2f, \"us_per_launch_timed\": %.2f, "
         "\"cycles_are\": \"[median, max] over the %d workgroups (wave 0) of the last launch\"}\n",
         us_product, us_timed, WGS);
  CHECK(hipFree(A));
  CHECK(hipFree(B));
  CHECK(hipFree(Y));
  CHECK(hipFree(P));
  return same ? 0 : 2;
}
