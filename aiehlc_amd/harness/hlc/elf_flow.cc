// A host program in the aiehlc dialect: AIE kernels declared `__global__`
// inline, loaded with XAie_LoadElfMem and driven through aie-rt calls.
// aiehlc_amd/hlc.py cuts the kernel definitions out and points
// XAie_LoadElfMem at the gfx950 kernels; the rest compiles as written.
#include <stdint.h>
#include <stdio.h>

#include "xaiengine.h"

#define CORE_IP_MEM 0x1000
#define CORE_OP_MEM 0x6000
#define CHAIN_IP_MEM 0x1000
#define CHAIN_OP_MEM 0x5000
#define N 16

// 16x16 int32 product of a packed window: A row-major, then B as [N][K].
// The body is AIE code (window API); it never reaches the host compiler.
__global__ void mm(input_window_int32* win __attribute__((annotate("mem_address:0x1000"), annotate("size_hint:512"))),
                   output_window_int32* out __attribute__((annotate("mem_address:0x6000"), annotate("size_hint:512")))) {
  int32_t a[N * N], b[N * N];
  for (unsigned w = 0; w < 2 * N * N / 16; w++) {
    aie::vector<int32_t, 16> v = window_readincr_v<16>(win);
    aie::store_unaligned_v<16>(w < N ? a + 16 * w : b + 16 * (w - N), v);
  }
  for (int i = 0; i < N; i++)
    for (int j = 0; j < N; j++) {
      int32_t s = 0;
      for (int k = 0; k < N; k++) s += a[i * N + k] * b[j * N + k];
      window_writeincr(out, s);
    }
}

// "/* __global__ in a string is not a kernel */"
__global__ void k1(int* in, int* out) {
  for (int i = 0; i < 20; ++i) *(out++) = *in + 1;
}

__global__ void k2(int* in, int* out) {
  for (int i = 0; i < 20; ++i) *(out++) = *in + 10;
}

static void wait_done(XAie_DevInst* dev, XAie_LocType loc) {
  while (XAie_CoreWaitForDone(dev, loc, 0) != XAIE_OK) {
  }
}

static int run_mm(XAie_DevInst* dev) {
  const XAie_LocType core = XAie_TileLoc(4, 4), shim = XAie_TileLoc(2, 0);
  XAie_CoreReset(dev, core);
  XAie_CoreUnreset(dev, core);
  XAie_LoadElfMem(dev, core, (unsigned char*)mm);
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(dev);
  XAie_Route(ri, NULL, shim, core);
  XAie_Route(ri, NULL, core, shim);
  XAie_MemInst* in = XAie_MemAllocate(dev, 2 * N * N * sizeof(u32), XAIE_MEM_CACHEABLE);
  XAie_MemInst* out = XAie_MemAllocate(dev, N * N * sizeof(u32), XAIE_MEM_CACHEABLE);
  int32_t* vin = (int32_t*)XAie_MemGetVAddr(in);
  int32_t* vout = (int32_t*)XAie_MemGetVAddr(out);
  for (int i = 0; i < 2 * N * N; i++) vin[i] = i;
  XAie_MemSyncForDev(in);
  XAie_MoveDataExternal2Aie(ri, shim, in, 2 * N * N * sizeof(u32), CORE_IP_MEM, core);
  XAie_Run(ri, 1);
  wait_done(dev, core);
  XAie_MoveDataAie2External(ri, core, CORE_OP_MEM, N * N * sizeof(u32), out, shim);
  XAie_MemSyncForCPU(out);
  int bad = 0;
  for (int i = 0; i < N; i++)
    for (int j = 0; j < N; j++) {
      int32_t s = 0;
      for (int k = 0; k < N; k++) s += vin[i * N + k] * vin[N * N + j * N + k];
      bad += s != vout[i * N + j];
    }
  printf("mm: C[0][0] = %d, C[15][15] = %d, %d mismatches\n", vout[0], vout[N * N - 1], bad);
  return bad;
}

static int run_chain(XAie_DevInst* dev) {
  const XAie_LocType shim = XAie_TileLoc(2, 0), t1 = XAie_TileLoc(1, 3), t2 = XAie_TileLoc(1, 4);
  XAie_CoreReset(dev, t1);
  XAie_CoreUnreset(dev, t1);
  XAie_LoadElfMem(dev, t1, (unsigned char *) k1);
  XAie_CoreReset(dev, t2);
  XAie_CoreUnreset(dev, t2);
  XAie_LoadElfMem(dev, t2, (unsigned char *) k2);
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(dev);
  XAie_Route(ri, NULL, shim, t1);
  XAie_Route(ri, NULL, t1, t2);
  XAie_Route(ri, NULL, t2, shim);
  XAie_MemInst* in = XAie_MemAllocate(dev, 20 * sizeof(u32), XAIE_MEM_CACHEABLE);
  XAie_MemInst* out = XAie_MemAllocate(dev, 20 * sizeof(u32), XAIE_MEM_CACHEABLE);
  int* vin = (int*)XAie_MemGetVAddr(in);
  int* vout = (int*)XAie_MemGetVAddr(out);
  for (int i = 0; i < 20; i++) vin[i] = 15, vout[i] = -1;
  XAie_MoveDataExternal2Aie(ri, shim, in, 20 * sizeof(u32), CHAIN_IP_MEM, t1);
  XAie_Run(ri, 1);
  wait_done(dev, t1);
  XAie_MoveData(ri, t1, (void*)CHAIN_OP_MEM, 20 * sizeof(u32), (void*)CHAIN_IP_MEM, t2);
  XAie_Run(ri, 1);
  wait_done(dev, t2);
  XAie_MoveDataAie2External(ri, t2, CHAIN_OP_MEM, 20 * sizeof(u32), out, shim);
  int bad = 0;
  for (int i = 0; i < 20; i++) bad += vout[i] != 26;
  printf("chain: out[0] = %d, %d mismatches\n", vout[0], bad);
  return bad;
}

int main(void) {
  XAie_SetupConfig(cfg, XAIE_DEV_GEN_AIEML, 0x20000000000ull, 25, 20, 38, 11, 0, 1, 2, 3, 8);
  XAie_InstDeclare(dev, &cfg);
  if (XAie_CfgInitialize(&dev, &cfg) != XAIE_OK) {
    printf("init failed: %s\n", XAie_MiaieLastError(NULL));
    return 2;
  }
  XAie_SetIOBackend(&dev, XAIE_IO_BACKEND_BAREMETAL);
  XAie_PartitionInitialize(&dev, NULL);
  const int bad = run_mm(&dev) + run_chain(&dev);
  XAie_PartitionTeardown(&dev);
  printf(bad ? "elf_flow: FAILED\n" : "elf_flow: all results match\n");
  return bad != 0;
}
