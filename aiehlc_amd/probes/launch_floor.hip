// launch_floor — the time per launch of a kernel that does nothing, issued
// back to back on one stream, for the grid shapes and LDS sizes of the
// library's kernels.  A launch of a real kernel cannot take less than this on
// the same GPU: the command processor's dispatch, the workgroup launch (the
// LDS allocation included) and the end-of-kernel completion are all in it.
// The int8 conv of the benchmark (8x56x56x64, 3x3) is a few microseconds of
// work, so its time per launch is read against this floor.
//
// Prints one JSON object: per grid shape, microseconds per back-to-back launch.
#include <hip/hip_runtime.h>

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

#define CHECK(x)                                                        \
  do {                                                                  \
    hipError_t e_ = (x);                                                \
    if (e_ != hipSuccess) {                                             \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));           \
      exit(1);                                                          \
    }                                                                   \
  } while (0)

template <int LDS_BYTES, int THREADS>
void run(int* out, int blocks, int iters, const char* name, bool last) {
  auto launch = [&]() { hipLaunchKernelGGL((empty_kernel<LDS_BYTES, THREADS>), dim3(blocks), dim3(THREADS), 0, 0, out, 0); };
  for (int i = 0; i < 2000; ++i) launch();
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  for (int i = 0; i < iters; ++i) launch();
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  printf("  \"%s\": {\"workgroups\": %d, \"threads\": %d, \"lds_bytes\": %d, \"us_per_launch\": %.3f}%s\n", name, blocks,
         THREADS, LDS_BYTES, ms * 1e3 / iters, last ? "" : ",");
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 5000;
  int* out = nullptr;
  CHECK(hipMalloc(&out, 4096 * sizeof(int)));
  printf("{\n");
  // conv2d_i8_rows<3,3,64,2,64> at N=8, 56x56: 224 workgroups (8 x 28 x 1) of 512 threads, 65024 B of LDS
  run<65024, 512>(out, 224, iters, "conv2d_rows_grid", false);
  // gemm_i8_pipe16<256,256> at 4096^3: 256 workgroups of 256 threads, 160 KiB of LDS
  run<163840, 256>(out, 256, iters, "gemm_256x256_grid", false);
  run<0, 64>(out, 1, iters, "one_wave", true);
  printf("}\n");
  CHECK(hipFree(out));
  return 0;
}
