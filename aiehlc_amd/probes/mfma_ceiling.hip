// mfma_ceiling — measures what the MFMA units sustain on this GPU when fed
// from registers only (no memory traffic), for the instructions the GEMM
// kernels use (int8 32x32x32 and 16x16x64, bf16 32x32x16), with constant and
// with random operands.  MFMA power depends on
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

// KIND 0: v_mfma_i32_32x32x32_i8; 1: v_mfma_f32_32x32x16_bf16; 2: two
// v_mfma_i32_16x16x64_i8 per slot (the same MACs as one 32x32x32), updated in
// place as the GEMM kernel does.
template <int KIND, bool RANDOM>
__global__ __launch_bounds__(256, 1) void probe(int* out, int iters) {
  constexpr bool BF16 = KIND == 1;
  v16i ai[8];
  v16f af[8];
  v4i a16[8];
  for (int i = 0; i < 8; ++i) {
    ai[i] = v16i{0};
    af[i] = v16f{0.f};
    a16[i] = v4i{0};
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
        if constexpr (KIND == 1) {
          af[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ra[i]),
                                                         __builtin_bit_cast(v8bf, rb[(i + u) & 7]), af[i], 0, 0, 0);
        } else if constexpr (KIND == 0) {
          ai[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ra[i], rb[(i + u) & 7], ai[i], 0, 0, 0);
        } else {
          asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(a16[i]) : "v"(ra[i]), "v"(rb[(i + u) & 7]));
          asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0"
              : "+a"(a16[(i + 4) & 7])
              : "v"(rb[i]), "v"(ra[(i + u) & 7]));
        }
      }
  }
  // (the asm MFMAs' results are read below only after their latency)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  const unsigned long long c1 = clock64(), w1 = wall_clock64();
  int s = 0;
  for (int i = 0; i < 8; ++i) {
    for (int e = 0; e < 16; ++e) s += ai[i][e] + (int)af[i][e];
    for (int e = 0; e < 4; ++e) s += a16[i][e];
  }
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

template <int KIND, bool RANDOM>
void run(int* out, int blocks, int iters, const char* name, bool last) {
  constexpr bool BF16 = KIND == 1;
  hipLaunchKernelGGL((probe<KIND, RANDOM>), dim3(blocks), dim3(256), 0, 0, out, 200);  // warm up
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL((probe<KIND, RANDOM>), dim3(blocks), dim3(256), 0, 0, out, iters);
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
  const double slots_per_wave = 64.0 * iters;  // 32768 int8 or 16384 bf16 MACs each
  const double mfma_per_wave = slots_per_wave * (KIND == 2 ? 2 : 1);
  const double ops = 2.0 * (BF16 ? 16384.0 : 32768.0) * slots_per_wave * 4 * blocks;
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
  run<0, false>(out, cus, iters, "i8_32x32x32_constant", false);
  run<0, true>(out, cus, iters, "i8_32x32x32_random", false);
  run<2, true>(out, cus, iters, "i8_16x16x64_random", false);
  run<1, false>(out, cus, iters, "bf16_32x32x16_constant", false);
  run<1, true>(out, cus, iters, "bf16_32x32x16_random", true);
  printf("}\n");
  CHECK(hipFree(out));
  return 0;
}
