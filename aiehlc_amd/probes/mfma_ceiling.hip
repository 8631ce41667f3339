// mfma_ceiling — measures what the MFMA units sustain on this GPU when fed
// from registers only (no memory traffic), for the two instructions the GEMM
// kernels use, with constant and with random operands.  MFMA power depends on
// operand bit toggling and the MI355X lowers its shader clock under load, so
// the random-operand rate is the practical ceiling for random int8 / bf16
// GEMM inputs; the spec-sheet peak assumes the 2.4 GHz maximum clock.
//
// Prints one JSON object: per (instruction, operands): TOP/s, shader clock
// (from s_memtime over the wall clock), cycles per MFMA.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ unsigned long long g_clk[2048];

template <bool BF16, bool RANDOM>
__global__ __launch_bounds__(256, 1) void probe(int* out, int iters) {
  v16i ai[8];
  v16f af[8];
  for (int i = 0; i < 8; ++i) {
    ai[i] = v16i{0};
    af[i] = v16f{0.f};
  }
  v4i ra[8], rb[8];
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 4; ++e) {
      unsigned z = ((threadIdx.x * 8 + i) * 4 + e) * 2654435761u + blockIdx.x * 7919u + 1u;
      z ^= z >> 15;
      z *= 0x2c1b3c6du;
      z ^= z >> 12;
      z *= 0x297a2d39u;
      z ^= z >> 15;
      const unsigned w = z * 0x9E3779B9u + 12345u;
      // bf16 operands keep finite values (exponent bits masked)
      ra[i][e] = RANDOM ? (int)(BF16 ? (z & 0xBFFFBFFFu) : z) : 0x01020102;
      rb[i][e] = RANDOM ? (int)(BF16 ? (w & 0xBFFFBFFFu) : w) : 0x02010201;
    }
  const unsigned long long c0 = clock64(), w0 = wall_clock64();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (BF16)
          af[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ra[i]),
                                                         __builtin_bit_cast(v8bf, rb[(i + u) & 7]), af[i], 0, 0, 0);
        else
          ai[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ra[i], rb[(i + u) & 7], ai[i], 0, 0, 0);
      }
  }
  const unsigned long long c1 = clock64(), w1 = wall_clock64();
  int s = 0;
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 16; ++e) s += ai[i][e] + (int)af[i][e];
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if (threadIdx.x == 0 && blockIdx.x < 1024) {
    g_clk[2 * blockIdx.x] = c1 - c0;
    g_clk[2 * blockIdx.x + 1] = w1 - w0;
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

template <bool BF16, bool RANDOM>
void run(int* out, int blocks, int iters, const char* name, bool last) {
  hipLaunchKernelGGL((probe<BF16, RANDOM>), dim3(blocks), dim3(256), 0, 0, out, 200);  // warm up
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL((probe<BF16, RANDOM>), dim3(blocks), dim3(256), 0, 0, out, iters);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  static unsigned long long h[2048];
  CHECK(hipMemcpyFromSymbol(h, HIP_SYMBOL(g_clk), sizeof(h)));
  double cyc = 0, wall = 0;
  const int nb = blocks < 1024 ? blocks : 1024;
  for (int b = 0; b < nb; ++b) {
    cyc += h[2 * b];
    wall += h[2 * b + 1];
  }
  const double mfma_per_wave = 64.0 * iters;
  const double ops = 2.0 * (BF16 ? 16384.0 : 32768.0) * mfma_per_wave * 4 * blocks;
  printf("  \"%s\": {\"tops\": %.1f, \"clock_ghz\": %.3f, \"cycles_per_mfma\": %.1f}%s\n", name,
         ops / (ms * 1e-3) / 1e12, cyc / wall * 0.1, cyc / nb / mfma_per_wave, last ? "" : ",");
}

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 4000;
  int dev = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  int* out = nullptr;
  CHECK(hipMalloc(&out, (size_t)cus * 256 * sizeof(int)));
  printf("{\n");
  run<false, false>(out, cus, iters, "i8_32x32x32_constant", false);
  run<false, true>(out, cus, iters, "i8_32x32x32_random", false);
  run<true, false>(out, cus, iters, "bf16_32x32x16_constant", false);
  run<true, true>(out, cus, iters, "bf16_32x32x16_random", true);
  printf("}\n");
  CHECK(hipFree(out));
  return 0;
}
