// launch_floor — what a launch costs apart from its kernel's work, for the
// grid shapes and LDS sizes of the library's kernels, with an empty kernel
// issued back to back on one stream.  Three figures per grid:
//   us_per_launch       host loop of launches, then a drain: the rate one
//                       host thread gets (events around the loop)
//   host_issue_us       the host's time in hipLaunchKernel per launch (the
//                       loop alone, before the drain)
//   device_us           the device's own rate: the launches are queued behind
//                       a one-wave kernel that waits a fixed wall-clock time
//                       (longer than the host needs to queue them), and
//                       events after the wait and after the last launch
//                       bracket them; blocker_outlasted_issue says whether the
//                       whole batch was queued before the wait ended
// When host_issue_us exceeds device_us, a host thread issuing one launch
// after another is what limits the back-to-back rate, not the device.
// host_launch_paths: the host's time per launch through each launch API.
//
// Prints one JSON object.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>

// `magic` never matches (the host passes 0), but the compiler cannot know,
// so the LDS array stays allocated at its full size.
template <int LDS_BYTES, int THREADS>
__global__ __launch_bounds__(THREADS) void empty_kernel(int* out, int magic) {
  if constexpr (LDS_BYTES > 0) {
    __shared__ int s[LDS_BYTES / 4];
    if (magic == 0x5eed && threadIdx.x == 0) {
      s[blockIdx.x % (LDS_BYTES / 4)] = magic;
      out[blockIdx.x] = s[(blockIdx.x * 7) % (LDS_BYTES / 4)];
    }
  } else {
    if (magic == 0x5eed && threadIdx.x == 0) out[blockIdx.x] = magic;
  }
}

// One wave that returns once `ticks` of the 100 MHz constant clock have
// passed: a wait of fixed length that ends on its own.
__global__ __launch_bounds__(64) void timed_wait(unsigned long long ticks) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(100);
}

#define CHECK(x)                                                        \
  do {                                                                  \
    hipError_t e_ = (x);                                                \
    if (e_ != hipSuccess) {                                             \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));           \
      exit(1);                                                          \
    }                                                                   \
  } while (0)

using clk = std::chrono::steady_clock;
static double us_since(clk::time_point t) { return std::chrono::duration<double, std::micro>(clk::now() - t).count(); }

template <int LDS_BYTES, int THREADS>
void run(hipStream_t st, int* out, int blocks, int iters, const char* name, bool last) {
  auto launch = [&]() {
    hipLaunchKernelGGL((empty_kernel<LDS_BYTES, THREADS>), dim3(blocks), dim3(THREADS), 0, st, out, 0);
  };
  for (int i = 0; i < 2000; ++i) launch();
  CHECK(hipGetLastError());
  CHECK(hipStreamSynchronize(st));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));

  // host loop, then drain
  CHECK(hipEventRecord(e0, st));
  const auto t0 = clk::now();
  for (int i = 0; i < iters; ++i) launch();
  const double issue_us = us_since(t0) / iters;
  CHECK(hipEventRecord(e1, st));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double loop_us = ms * 1e3 / iters;

  // queued behind a wait of 4 us per launch (2 us more than the host's
  // issue time measured above, at most 40 ms)
  const int nq = 1000;
  const double wait_us = nq * (issue_us + 2.0) < 40000.0 ? nq * (issue_us + 2.0) : 40000.0;
  hipLaunchKernelGGL(timed_wait, dim3(1), dim3(64), 0, st, (unsigned long long)(wait_us * 100.0));
  CHECK(hipEventRecord(e0, st));
  for (int i = 0; i < nq; ++i) launch();
  const bool outlasted = hipEventQuery(e0) == hipErrorNotReady;
  CHECK(hipEventRecord(e1, st));
  CHECK(hipEventSynchronize(e1));
  CHECK(hipGetLastError());
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double device_us = ms * 1e3 / nq;

  printf("  \"%s\": {\"workgroups\": %d, \"threads\": %d, \"lds_bytes\": %d, \"us_per_launch\": %.3f, "
         "\"host_issue_us\": %.3f, \"device_us\": %.3f, \"blocker_outlasted_issue\": %s}%s\n",
         name, blocks, THREADS, LDS_BYTES, loop_us, issue_us, device_us, outlasted ? "true" : "false",
         last ? "" : ",");
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

// An empty kernel with the conv2d_i8_rows argument list (11 arguments).
__global__ __launch_bounds__(512) void empty_conv_args(const int8_t* X, const int8_t* W, const uint8_t* s, int8_t* Y,
                                                       int H, int Wd, int pad, int xg, int ncb, int Cout,
                                                       unsigned long long* probe) {
  if (H == 0x5eed && threadIdx.x == 0) Y[blockIdx.x] = (int8_t)Wd;
}

// Host time per launch of the conv grid's empty kernel through the ways a
// library can launch it: hipLaunchKernelGGL alone, with the hipGetLastError
// check, with hipSetDevice or hipGetDevice in front (what each entry point
// does to make its device current), and hipModuleLaunchKernel with a handle
// looked up once (hipGetFuncBySymbol) or hipExtLaunchKernel.  Each figure
// is the median of 9 loops of `iters` launches, the host's clock around the
// loop (the device runs these launches faster than the host issues them).
void launch_paths(hipStream_t st, int8_t* y, int iters) {
  const dim3 grid(8, 14, 2), blk(512);
  const int8_t* X = nullptr;
  const int8_t* W = nullptr;
  const uint8_t* S = nullptr;
  int H = 56, Wd = 56, pad = 1, xg = 1, ncb = 1, Cout = 64;
  unsigned long long* P = nullptr;
  hipFunction_t f;
  CHECK(hipGetFuncBySymbol(&f, reinterpret_cast<const void*>(&empty_conv_args)));
  void* args[] = {&X, &W, &S, &y, &H, &Wd, &pad, &xg, &ncb, &Cout, &P};
  auto ggl = [&]() { hipLaunchKernelGGL(empty_conv_args, grid, blk, 0, st, X, W, S, y, H, Wd, pad, xg, ncb, Cout, P); };
  auto time = [&](auto fn) {
    double t[9];
    for (int r = 0; r < 9; ++r) {
      CHECK(hipStreamSynchronize(st));
      const auto t0 = clk::now();
      for (int i = 0; i < iters; ++i) fn();
      t[r] = us_since(t0) / iters;
      CHECK(hipStreamSynchronize(st));
    }
    std::sort(t, t + 9);
    return t[4];
  };
  int dev = 0;
  CHECK(hipGetDevice(&dev));
  const double a = time(ggl);
  const double b = time([&]() { ggl(); (void)hipGetLastError(); });
  const double c = time([&]() { (void)hipSetDevice(dev); ggl(); (void)hipGetLastError(); });
  const double d = time([&]() { int cur; (void)hipGetDevice(&cur); if (cur != dev) (void)hipSetDevice(dev); ggl(); (void)hipGetLastError(); });
  const double e = time([&]() { (void)hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, blk.x, 1, 1, 0, st, args, nullptr); });
  const double g = time([&]() { int cur; (void)hipGetDevice(&cur); (void)hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, blk.x, 1, 1, 0, st, args, nullptr); });
  const double h = time([&]() { (void)hipExtLaunchKernel(reinterpret_cast<const void*>(&empty_conv_args), grid, blk, args, 0, st, nullptr, nullptr, 0); });
  CHECK(hipGetLastError());
  printf("  \"host_launch_paths\": {\"kernel\": \"empty, the conv kernel's 11 arguments, conv grid 224 x 512\", \"launches\": %d, "
         "\"us\": {\"hipLaunchKernelGGL\": %.3f, \"+hipGetLastError\": %.3f, \"hipSetDevice+GGL+hipGetLastError\": %.3f, "
         "\"hipGetDevice+GGL+hipGetLastError\": %.3f, \"hipModuleLaunchKernel_cached_handle\": %.3f, "
         "\"hipGetDevice+hipModuleLaunchKernel_cached_handle\": %.3f, \"hipExtLaunchKernel\": %.3f}}\n",
         iters, a, b, c, d, e, g, h);
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 5000;
  int* out = nullptr;
  hipStream_t st;
  CHECK(hipStreamCreate(&st));
  CHECK(hipMalloc(&out, 4096 * sizeof(int)));
  printf("{\n");
  // conv2d_i8_rows<3,3,64,4,32> at N=8, 56x56: 224 workgroups (8 x 14 x 2) of 512 threads, 56576 B of LDS
  run<56576, 512>(st, out, 224, iters, "conv2d_rows_grid", false);
  // gemm_i8_pipe16<256,256> at 4096^3: 256 workgroups of 256 threads, 160 KiB of LDS
  run<163840, 256>(st, out, 256, iters, "gemm_256x256_grid", false);
  run<0, 64>(st, out, 1, iters, "one_wave", false);
  launch_paths(st, reinterpret_cast<int8_t*>(out), iters < 500 ? iters : 500);
  printf("}\n");
  CHECK(hipFree(out));
  CHECK(hipStreamDestroy(st));
  return 0;
}
