// A host program in the aiehlc dialect with `__kernel__` launches: the
// template call perf<Col, Row, colstart, rowstart, M, N, K>(phy, phy_out)
// of example/nokernelload on DDR addresses, and a GEMM launched on device
// buffers.  aiehlc_amd/hlc.py replaces the kernel definitions with
// forwarding templates.
#include <stdint.h>
#include <stdio.h>

#include <vector>

#include "miaie.hpp"
#include "xaiengine.h"

// uint8 dot-product throughput probe: 3 * in[0] repetitions of a 128-element
// dot, results in 5 words (AIE code; cut out by the rewriter).
__kernel__ void perf(input_window_int32* win __attribute__((annotate("mem_address:0x1000"))),
                     output_window_int32* out __attribute__((annotate("mem_address:0x6000")))) {
  uint32_t* o = (uint32_t*)(0x70000 + 0x6000);
  const uint32_t p = *(uint32_t*)(0x70000 + 0x1000);
  uint8_t v1[128], v2[128];
  uint32_t ret = 0, num = 0;
  for (uint32_t i = 0; i < 128; i++) {
    v1[i] = i + (p & 1) ? 1 : 2;
    v2[i] = 0 + (p & 1) ? 1 : 2;
  }
  for (int k = 0; k < 3; k++)
    for (uint32_t i = 0; i < p; i++, num++)
      for (int j = 0; j < 128; j++) ret += v1[j] * v2[j];
  o[0] = num; o[1] = 4567; o[2] = ret; o[3] = 3; o[4] = v1[0];
}

// int8 GEMM + requant on device buffers (AIE code; cut out by the rewriter).
__kernel__ void gemm_i8(const int8_t* A, const int8_t* B, int8_t* Y, int shift) {
  aie::mmul<4, 8, 8, int8, int8> m;
  m.mac(aie::load_v<32>(A), aie::load_v<64>(B));
  aie::store_v(Y, m.to_vector<int8>(shift));
}

static int probe() {
  XAie_SetupConfig(cfg, XAIE_DEV_GEN_AIEML, 0x20000000000ull, 25, 20, 38, 11, 0, 1, 2, 3, 8);
  XAie_InstDeclare(dev, &cfg);
  if (XAie_CfgInitialize(&dev, &cfg) != XAIE_OK) {
    printf("init failed: %s\n", XAie_MiaieLastError(NULL));
    return 2;
  }
  XAie_PartitionInitialize(&dev, NULL);
  XAie_MemInst* in = XAie_MemAllocate(&dev, 512 * sizeof(u32), XAIE_MEM_CACHEABLE);
  XAie_MemInst* out = XAie_MemAllocate(&dev, 512 * sizeof(u32), XAIE_MEM_CACHEABLE);
  const u64 phy = (u32)XAie_MemGetDevAddr(in), phy_out = (u32)XAie_MemGetDevAddr(out);
  ((uint32_t*)phy)[0] = 1u << 20;
  perf<1, 1, 4, 4, 256, 16, 64>(phy, phy_out);
  const uint32_t* o = (const uint32_t*)phy_out;
  // closed form for in[0] = 2^20: 3*2^20 repetitions of sum_j v1[j]*v2[j] = 2*(2*2 + 127*1*2)... as uint32
  const uint32_t want[5] = {3u << 20, 4567u, 811597824u, 3u, 2u};
  int bad = 0;
  for (int i = 0; i < 5; i++) bad += o[i] != want[i];
  printf("perf: out = {%u, %u, %u, %u, %u}, %d mismatches\n", o[0], o[1], o[2], o[3], o[4], bad);
  XAie_PartitionTeardown(&dev);
  return bad;
}

static int gemm() {
  enum { M = 256, N = 256, K = 512 };
  miaie::Context ctx(0);
  std::vector<int8_t> a(M * K), b(K * N);
  uint32_t x = 12345;
  for (auto& v : a) v = (int8_t)((x = x * 1664525u + 1013904223u) >> 24);
  for (auto& v : b) v = (int8_t)((x = x * 1664525u + 1013904223u) >> 24);
  miaie::Buffer<int8_t> A(ctx, a.size()), B(ctx, b.size()), Y(ctx, M * N);
  A.move_in(a);
  B.move_in(b);
  gemm_i8<1, 1, 0, 0, M, N, K>(A.data(), B.data(), Y.data(), 10);
  ctx.wait();
  const std::vector<int8_t> y = Y.move_out();
  int bad = 0;
  for (int i = 0; i < M; i++)
    for (int j = 0; j < N; j++) {
      int32_t s = 0;
      for (int k = 0; k < K; k++) s += a[i * K + k] * b[k * N + j];
      int32_t q = (s + (1 << 9)) >> 10;
      q = q < -128 ? -128 : q > 127 ? 127 : q;
      bad += q != y[i * N + j];
    }
  printf("gemm_i8: %d x %d x %d, %d mismatches\n", M, N, K, bad);
  return bad;
}

int main() {
  const int bad = probe() + gemm();
  printf(bad ? "kernel_flow: FAILED\n" : "kernel_flow: all results match\n");
  return bad != 0;
}
