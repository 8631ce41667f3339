// conv_span — in-kernel clocks of the row-block int8 conv at the benchmark's
// config 4 (N=8, 56x56, Cin=Cout=64, 3x3, stride 1, pad 1).
//
// Runs the library's own kernel template (aiehlc_amd/csrc/conv2d_i8_rows.hpp)
// twice over: the product instantiation, and the TIMED one, which records
// per wave the shader clock (s_memtime) at its start, after the staging
// barrier, after the MFMA loop and at its end, and the 100 MHz wall clock
// (s_memrealtime) at its start and end.  The TIMED output must equal the
// product output byte for byte.  From the last of 2000 back-to-back TIMED
// launches it reports:
//   span_us            first wave's start to last wave's end (wall clock):
//                      the kernel's own execution time, without the command
//                      processor's work between launches
//   last_start_us      how long after the first wave the last one started
//   staging / mfma / epilogue cycles per wave (median and max)
//   clock_ghz          shader cycles per wall-clock ns, averaged over waves
// and the time per back-to-back launch of both instantiations (HIP events).
// For the product instantiation it also reports the host's time per launch
// alone (host_issue_us) and the device's own time per launch with the queue
// already filled (device_us): 1000 launches queued behind a one-wave kernel
// that waits a fixed wall-clock time longer than the host needs to queue
// them, bracketed by events after the wait and after the last launch.
// Prints one JSON object.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../csrc/conv2d_i8_rows.hpp"

#define CHECK(x)                                                        \
  do {                                                                  \
    hipError_t e_ = (x);                                                \
    if (e_ != hipSuccess) {                                             \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));           \
      exit(1);                                                          \
    }                                                                   \
  } while (0)

namespace {

constexpr int N = 8, H = 56, Wd = 56, CIN = 64, COUT = 64, ROWS = 4, WCO = 32;

uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// One wave that returns once `ticks` of the 100 MHz constant clock have
// passed: a wait of fixed length that ends on its own.
__global__ __launch_bounds__(64) void timed_wait(unsigned long long ticks) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(100);
}

using clk = std::chrono::steady_clock;

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  return v[v.size() / 2];
}

}  // namespace

int main(int argc, char** argv) {
  const int launches = argc > 1 ? atoi(argv[1]) : 2000;
  const size_t xb = (size_t)N * H * Wd * CIN, wb = (size_t)COUT * 9 * CIN, yb = (size_t)N * H * Wd * COUT;
  std::vector<int8_t> hx(xb), hw(wb);
  std::vector<uint8_t> hs(COUT);
  for (size_t i = 0; i < xb; ++i) hx[i] = (int8_t)(mix(0x1000 + i) >> 56);
  for (size_t i = 0; i < wb; ++i) hw[i] = (int8_t)(mix(0x2000000 + i) >> 56);
  for (int i = 0; i < COUT; ++i) hs[i] = (uint8_t)(8 + mix(0x3000000 + i) % 5);
  const int waves = 8 * (H / ROWS) * (COUT / WCO) * N;  // 224 workgroups of 8 waves
  int8_t *X, *W, *Y;
  uint8_t* S;
  unsigned long long* P;
  CHECK(hipMalloc(&X, xb));
  CHECK(hipMalloc(&W, wb));
  CHECK(hipMalloc(&Y, yb));
  CHECK(hipMalloc(&S, COUT));
  CHECK(hipMalloc(&P, (size_t)waves * miaie::conv::PROBE_WORDS * sizeof(unsigned long long)));
  CHECK(hipMemcpy(X, hx.data(), xb, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(W, hw.data(), wb, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(S, hs.data(), COUT, hipMemcpyHostToDevice));
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  auto product = [&]() {
    CHECK((miaie::conv::launch_rows_as<CIN, ROWS, WCO, false>(0, st, X, W, S, Y, N, H, Wd, COUT, 1, H, Wd)));
  };
  auto timed = [&]() {
    CHECK((miaie::conv::launch_rows_as<CIN, ROWS, WCO, true>(0, st, X, W, S, Y, N, H, Wd, COUT, 1, H, Wd, P)));
  };
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  double issue_us = 0;  // host time per launch of the last per_launch_us loop
  auto per_launch_us = [&](auto fn) {
    for (int i = 0; i < 500; ++i) fn();
    CHECK(hipEventRecord(e0, st));
    const auto t0 = clk::now();
    for (int i = 0; i < launches; ++i) fn();
    issue_us = std::chrono::duration<double, std::micro>(clk::now() - t0).count() / launches;
    CHECK(hipEventRecord(e1, st));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    return ms * 1e3 / launches;
  };
  // the device's own time per launch: nq launches queued behind a wait of
  // (host issue + 2) us per launch, at most 40 ms
  bool outlasted = false;
  auto device_us = [&](auto fn, double host_us) {
    const int nq = 1000;
    const double wait_us = nq * (host_us + 2.0) < 40000.0 ? nq * (host_us + 2.0) : 40000.0;
    hipLaunchKernelGGL(timed_wait, dim3(1), dim3(64), 0, st, (unsigned long long)(wait_us * 100.0));
    CHECK(hipEventRecord(e0, st));
    for (int i = 0; i < nq; ++i) fn();
    outlasted = hipEventQuery(e0) == hipErrorNotReady;
    CHECK(hipEventRecord(e1, st));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    return ms * 1e3 / nq;
  };

  product();
  CHECK(hipGetLastError());
  CHECK(hipStreamSynchronize(st));
  std::vector<int8_t> y0(yb), y1(yb);
  CHECK(hipMemcpy(y0.data(), Y, yb, hipMemcpyDeviceToHost));
  const double us_product = per_launch_us(product);
  const double issue_product = issue_us;
  const double dev_product = device_us(product, issue_product);
  const double us_timed = per_launch_us(timed);  // its last launch leaves the probe words
  CHECK(hipGetLastError());
  CHECK(hipStreamSynchronize(st));
  CHECK(hipMemcpy(y1.data(), Y, yb, hipMemcpyDeviceToHost));
  const bool same = memcmp(y0.data(), y1.data(), yb) == 0;

  std::vector<unsigned long long> h((size_t)waves * miaie::conv::PROBE_WORDS);
  CHECK(hipMemcpy(h.data(), P, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  std::vector<double> stg, mf, ep;
  unsigned long long wall0 = ~0ull, wall1 = 0, last0 = 0;
  double ghz = 0;
  for (int w = 0; w < waves; ++w) {
    const unsigned long long* p = &h[(size_t)w * miaie::conv::PROBE_WORDS];
    stg.push_back((double)(p[1] - p[0]));
    mf.push_back((double)(p[2] - p[1]));
    ep.push_back((double)(p[3] - p[2]));
    wall0 = std::min(wall0, p[4]);
    wall1 = std::max(wall1, p[5]);
    last0 = std::max(last0, p[4]);
    ghz += (double)(p[3] - p[0]) / ((double)(p[5] - p[4]) * 10.0) / waves;
  }
  const double span_us = (double)(wall1 - wall0) / 100.0;
  printf("{\"kernel\": \"conv2d_i8_rows<3, 3, 64, 4, 32>\", \"config\": \"N=8 56x56 Cin=Cout=64 3x3 pad 1\", "
         "\"timed_output_equals_product\": %s, \"span_us\": %.3f, \"last_start_us\": %.3f, "
         "\"staging_cycles\": [%.0f, %.0f], \"mfma_cycles\": [%.0f, %.0f], \"epilogue_cycles\": [%.0f, %.0f], "
         "\"clock_ghz\": %.3f, \"us_per_launch_product\": %.3f, \"us_per_launch_timed\": %.3f, \"launches\": %d, "
         "\"host_issue_us\": %.3f, \"device_us\": %.3f, \"blocker_outlasted_issue\": %s, "
         "\"cycles_are\": \"[median, max] over the %d waves of the last launch\"}\n",
         same ? "true" : "false", span_us, (double)(last0 - wall0) / 100.0, median(stg),
         *std::max_element(stg.begin(), stg.end()), median(mf), *std::max_element(mf.begin(), mf.end()),
         median(ep), *std::max_element(ep.begin(), ep.end()), ghz, us_product, us_timed, launches, issue_product,
         dev_product, outlasted ? "true" : "false", waves);
  CHECK(hipFree(X));
  CHECK(hipFree(W));
  CHECK(hipFree(Y));
  CHECK(hipFree(S));
  CHECK(hipFree(P));
  return same ? 0 : 2;
}
