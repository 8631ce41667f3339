/*
 * xaie_flows — the reference examples' host flows, written in C against the
 * aie-rt-shaped facade (include/miaie_xaie.h) and run on the GPU.
 *
 * Each subcommand follows one example's sequence of XAie_* calls and checks
 * the result the way that example does (CPU golden or its constant), then
 * exits 0 on a match:
 *   mm [reps]     example/matrixmultiply/aieml_mm.cc:108-249 (+ main :251-296),
 *                 timed over the span aieml_mm.cc:148-190 times
 *   mm8 [reps]    the same flow for the program's 8x8 build (MAT_SIZE 64),
 *                 the "15us(8*8)" case aieml_mm.cc:257 prints
 *   perf [reps]   example/perf/aieml_perf.cc:105-254, partitioned at column 2
 *   multi_tile    example/multi/multi_tile.cpp:65-181 (expects 26)
 *   seq_full_col  example/multi/seq_full_col.cpp:65-181 (expects 23)
 *   vek385 [cols] example/multi/vek385_verification.cpp:72-230 (expects 3*v^2)
 *   oob           example/other/aieoob.c:76-150 (kernel-instance calls, 8x8)
 *   errors        argument and routing errors the facade must reject
 */
#define _POSIX_C_SOURCE 199309L /* clock_gettime */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "miaie_xaie.h"

/* The AIE-ML array geometry of the examples (aieml_mm.cc:19-31). */
#define HW_GEN XAIE_DEV_GEN_AIEML
#define XAIE_BASE_ADDR 0x20000000000ull
#define XAIE_COL_SHIFT 25
#define XAIE_ROW_SHIFT 20
#define XAIE_NUM_ROWS 11
#define XAIE_NUM_COLS 38
#define XAIE_SHIM_ROW 0
#define XAIE_RES_TILE_ROW_START 1
#define XAIE_RES_TILE_NUM_ROWS 2
#define XAIE_AIE_TILE_ROW_START 3
#define XAIE_AIE_TILE_NUM_ROWS 8

#define CHECK(call)                                                                   \
  do {                                                                                \
    AieRC rc_ = (call);                                                               \
    if (rc_ != XAIE_OK) {                                                             \
      fprintf(stderr, "%s:%d: %s -> %d (%s)\n", __FILE__, __LINE__, #call, (int)rc_, \
              XAie_MiaieLastError(NULL));                                             \
      exit(1);                                                                        \
    }                                                                                 \
  } while (0)

/* Configure, initialise and (optionally) partition the array, as each
 * example's main() does (aieml_perf.cc:265-313). */
static void open_device(XAie_DevInst* dev, int startcol, int ncols) {
  XAie_SetupConfig(cfg, HW_GEN, XAIE_BASE_ADDR, XAIE_COL_SHIFT, XAIE_ROW_SHIFT, XAIE_NUM_COLS, XAIE_NUM_ROWS,
                   XAIE_SHIM_ROW, XAIE_RES_TILE_ROW_START, XAIE_RES_TILE_NUM_ROWS, XAIE_AIE_TILE_ROW_START,
                   XAIE_AIE_TILE_NUM_ROWS);
  memset(dev, 0, sizeof *dev);
  if (ncols) CHECK(XAie_SetupPartitionConfig(dev, XAIE_BASE_ADDR + ((u64)startcol << XAIE_COL_SHIFT), startcol, ncols));
  CHECK(XAie_CfgInitialize(dev, &cfg));
  CHECK(XAie_SetIOBackend(dev, XAIE_IO_BACKEND_BAREMETAL));
  if (dev->Backend->Type == XAIE_IO_BACKEND_BAREMETAL) CHECK(XAie_UpdateNpiAddr(dev, 0xF6D10000));
  CHECK(XAie_PartitionInitialize(dev, NULL));
}

/* The golden loop and mismatch count of aieml_mm.cc:194-245: A row-major
 * from words [0, n*n), B as [n][k] from words [n*n, 2*n*n). */
static int golden_mismatches(const int32_t* in, const int32_t* out, int n) {
  int bad = 0;
  for (int i = 0; i < n; i++)
    for (int j = 0; j < n; j++) {
      uint32_t acc = 0;
      for (int k = 0; k < n; k++) acc += (uint32_t)in[i * n + k] * (uint32_t)in[n * n + j * n + k];
      if ((int32_t)acc != out[i * n + j]) {
        if (bad < 8) printf("Mismatch at index %d: CPU=%d, AIE=%d\n", i * n + j, (int32_t)acc, out[i * n + j]);
        bad++;
      }
    }
  return bad;
}

static double now_us(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return t.tv_sec * 1e6 + t.tv_nsec * 1e-3;
}

static int cmp_double(const void* a, const void* b) {
  const double x = *(const double*)a, y = *(const double*)b;
  return (x > y) - (x < y);
}

/* Wait for one core the way the examples do: poll until XAIE_OK
 * (aieml_mm.cc:172-182), here with an upper bound so a failure ends. */
static void wait_core(XAie_DevInst* dev, XAie_LocType loc) {
  for (long polls = 0; XAie_CoreWaitForDone(dev, loc, 0) != XAIE_OK; polls++)
    if (polls > 200000) {
      fprintf(stderr, "core (%u, %u) never finished: %s\n", loc.Col, loc.Row, XAie_MiaieLastError(dev));
      exit(1);
    }
}

/* aieml_mm.cc / aieml_perf.cc: one n x n NT tile (n = 16, or 8 for the
 * MAT_SIZE 64 build of aieml_mm.cc) through DDR -> tile -> DDR. */
static int flow_window(const XAie_MiaieKernel* kernel, int N, int startcol, int ncols, int shimcol, int first_value,
                       int use_ext_calls, int reps) {
  const int MAT_SIZE = N * N;
  XAie_DevInst dev;
  open_device(&dev, startcol, ncols);
  const XAie_LocType core = XAie_TileLoc(4, 4), shim = XAie_TileLoc((u8)shimcol, 0);
  CHECK(XAie_CoreReset(&dev, core));
  CHECK(XAie_CoreUnreset(&dev, core));
  CHECK(XAie_LoadElfMem(&dev, core, (const unsigned char*)kernel));
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(&dev);
  CHECK(XAie_Route(ri, NULL, shim, core));
  CHECK(XAie_Route(ri, NULL, core, shim));

  const u32 mlen = MAT_SIZE * 2, recv_len = MAT_SIZE;
  XAie_MemInst* in = XAie_MemAllocate(&dev, mlen * sizeof(u32), XAIE_MEM_CACHEABLE);
  XAie_MemInst* out = XAie_MemAllocate(&dev, mlen * sizeof(u32), XAIE_MEM_CACHEABLE);
  if (!in || !out) {
    fprintf(stderr, "XAie_MemAllocate: %s\n", XAie_MiaieLastError(&dev));
    return 1;
  }
  /* the examples keep the device address in 32 bits and write through it */
  const u64 phy = (u32)XAie_MemGetDevAddr(in), phy_out = (u32)XAie_MemGetDevAddr(out);
  for (u32 i = 0; i < mlen; i++) {
    ((int32_t*)(uintptr_t)phy)[i] = (int32_t)i + first_value;
    ((int32_t*)(uintptr_t)phy_out)[i] = 0;
  }
  CHECK(XAie_MemSyncForDev(in));
  CHECK(XAie_MemSyncForDev(out));

  const u32 CORE_IP_MEM = 0x1000, CORE_OP_MEM = 0x6000;
  /* The stopwatch spans what aieml_mm.cc:148-190 times: the move into the
   * tile, the run, the wait, the move back and MemSyncForCPU.  With reps > 1
   * the same sequence repeats and the median is printed as well. */
  double* us = (double*)calloc((size_t)reps, sizeof(double));
  if (!us) return 1;
  for (int r = 0; r < reps; r++) {
    const double t0 = now_us();
    if (use_ext_calls) {
      CHECK(XAie_MoveDataExternal2Aie(ri, shim, in, mlen * sizeof(u32), CORE_IP_MEM, core));
      CHECK(XAie_RouteDmaWait(ri, shim, core, 1));
    } else {
      CHECK(XAie_MoveData(ri, shim, (void*)(uintptr_t)phy, mlen * sizeof(u32), (void*)(uintptr_t)CORE_IP_MEM, core));
    }
    CHECK(XAie_Run(ri, 1));
    wait_core(&dev, core);
    if (use_ext_calls)
      CHECK(XAie_MoveDataAie2External(ri, core, CORE_OP_MEM, mlen * sizeof(u32), out, shim));
    else
      CHECK(XAie_MoveData(ri, core, (void*)(uintptr_t)CORE_OP_MEM, recv_len * sizeof(u32), (void*)(uintptr_t)phy_out,
                          shim));
    CHECK(XAie_MemSyncForCPU(out));
    us[r] = now_us() - t0;
  }
  printf("Output took %.2f us.\n", us[0]);
  if (reps > 1) {
    qsort(us, (size_t)reps, sizeof(double), cmp_double);
    printf("median over %d runs: %.2f us (min %.2f us)\n", reps, us[reps / 2], us[0]);
  }
  free(us);

  const int bad = golden_mismatches((const int32_t*)XAie_MemGetVAddr(in), (const int32_t*)XAie_MemGetVAddr(out), N);
  const int32_t* o = (const int32_t*)XAie_MemGetVAddr(out);
  printf("C[0][0] = %d, C[%d][%d] = %d\n", o[0], N - 1, N - 1, o[MAT_SIZE - 1]);
  if (bad == 0)
    printf("%s: CPU result matches the device output.\n", kernel->Name);
  else
    printf("%s: there were %d mismatches.\n", kernel->Name, bad);
  CHECK(XAie_MemFree(in));
  CHECK(XAie_MemFree(out));
  CHECK(XAie_PartitionTeardown(&dev));
  return bad != 0;
}

/* multi_tile.cpp:65-181: k1 on (1,3), k2 on (1,4), chained through a
 * tile-to-tile move. */
static int flow_multi_tile(void) {
  XAie_DevInst dev;
  open_device(&dev, 0, 0);
  const XAie_LocType in_t = XAie_TileLoc(2, 0), out_t = XAie_TileLoc(2, 0);
  const XAie_LocType k1 = XAie_TileLoc(1, 3), k2 = XAie_TileLoc(1, 4);
  CHECK(XAie_CoreReset(&dev, k1));
  CHECK(XAie_CoreUnreset(&dev, k1));
  CHECK(XAie_LoadElfMem(&dev, k1, (const unsigned char*)&miaie_xaie_k1));
  CHECK(XAie_CoreReset(&dev, k2));
  CHECK(XAie_CoreUnreset(&dev, k2));
  CHECK(XAie_LoadElfMem(&dev, k2, (const unsigned char*)&miaie_xaie_k2));
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(&dev);
  CHECK(XAie_Route(ri, NULL, in_t, k1));
  CHECK(XAie_Route(ri, NULL, k1, k2));
  CHECK(XAie_Route(ri, NULL, k2, out_t));

  const int len = 20;
  XAie_MemInst* in = XAie_MemAllocate(&dev, len * sizeof(u32), XAIE_MEM_CACHEABLE);
  XAie_MemInst* out = XAie_MemAllocate(&dev, len * sizeof(u32), XAIE_MEM_CACHEABLE);
  int* in_ptr = (int*)XAie_MemGetVAddr(in);
  int* out_ptr = (int*)XAie_MemGetVAddr(out);
  for (int i = 0; i < len; i++) {
    in_ptr[i] = 15;
    out_ptr[i] = 9999;
  }
  CHECK(XAie_MemSyncForDev(in));
  CHECK(XAie_MemSyncForCPU(out));
  const u32 CORE_IP_MEM = 0x1000, CORE_OP_MEM = 0x5000;
  CHECK(XAie_MoveDataExternal2Aie(ri, in_t, in, len * sizeof(u32), CORE_IP_MEM, k1));
  CHECK(XAie_Run(ri, 1));
  wait_core(&dev, k1);
  CHECK(XAie_MoveData(ri, k1, (void*)(uintptr_t)CORE_OP_MEM, len * sizeof(u32), (void*)(uintptr_t)CORE_IP_MEM, k2));
  CHECK(XAie_Run(ri, 1));
  wait_core(&dev, k2);
  CHECK(XAie_MoveDataAie2External(ri, k2, CORE_OP_MEM, len * sizeof(u32), out, out_t));

  const int c = 15 + 10 + 1;  /* multi_tile.cpp:150 */
  int bad = 0;
  for (int i = 0; i < len; i++) bad += out_ptr[i] != c;
  printf("out[0] = %d (expected %d), %d mismatches\n", out_ptr[0], c, bad);
  CHECK(XAie_PartitionTeardown(&dev));
  return bad != 0;
}

/* seq_full_col.cpp:65-181: k1 on every core tile of column 1 that reports a
 * status, chained tile to tile, one run per stage. */
static int flow_seq_full_col(void) {
  XAie_DevInst dev;
  open_device(&dev, 0, 0);
  const int col = 1;
  int start_row = -1, end_row = -1;
  for (int row = 0; row < XAIE_NUM_ROWS; ++row) {
    u32 status = 0;
    CHECK(XAie_CoreGetStatus(&dev, XAie_TileLoc(col, row), &status));
    if (status) {
      if (start_row == -1) start_row = row;
      end_row = row;
    }
  }
  printf("core tiles with a status: rows %d..%d\n", start_row, end_row);
  for (int i = start_row; i <= end_row; i++) {
    CHECK(XAie_CoreReset(&dev, XAie_TileLoc(col, i)));
    CHECK(XAie_CoreUnreset(&dev, XAie_TileLoc(col, i)));
    CHECK(XAie_LoadElfMem(&dev, XAie_TileLoc(col, i), (const unsigned char*)&miaie_xaie_k1));
  }
  const XAie_LocType in_t = XAie_TileLoc(2, 0), out_t = XAie_TileLoc(2, 0);
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(&dev);
  CHECK(XAie_Route(ri, NULL, in_t, XAie_TileLoc(col, start_row)));
  for (int i = start_row; i < end_row; i++) CHECK(XAie_Route(ri, NULL, XAie_TileLoc(col, i), XAie_TileLoc(col, i + 1)));
  CHECK(XAie_Route(ri, NULL, XAie_TileLoc(col, end_row), out_t));

  const int len = 20;
  XAie_MemInst* in = XAie_MemAllocate(&dev, len * sizeof(u32), XAIE_MEM_CACHEABLE);
  XAie_MemInst* out = XAie_MemAllocate(&dev, len * sizeof(u32), XAIE_MEM_CACHEABLE);
  int* in_ptr = (int*)XAie_MemGetVAddr(in);
  int* out_ptr = (int*)XAie_MemGetVAddr(out);
  for (int i = 0; i < len; i++) {
    in_ptr[i] = 15;
    out_ptr[i] = 9999;
  }
  const u32 CORE_IP_MEM = 0x1000, CORE_OP_MEM = 0x5000;
  CHECK(XAie_MoveDataExternal2Aie(ri, in_t, in, len * sizeof(u32), CORE_IP_MEM, XAie_TileLoc(1, 3)));
  for (int i = start_row; i <= end_row; i++) {
    CHECK(XAie_Run(ri, 1));
    wait_core(&dev, XAie_TileLoc(col, i));
    if (i != end_row)
      CHECK(XAie_MoveData(ri, XAie_TileLoc(col, i), (void*)(uintptr_t)CORE_OP_MEM, len * sizeof(u32),
                          (void*)(uintptr_t)CORE_IP_MEM, XAie_TileLoc(col, i + 1)));
  }
  CHECK(XAie_MoveDataAie2External(ri, XAie_TileLoc(col, end_row), CORE_OP_MEM, len * sizeof(u32), out, out_t));
  const int c = 23;  /* seq_full_col.cpp:163 */
  int bad = 0;
  for (int i = 0; i < len; i++) bad += out_ptr[i] != c;
  printf("out[0] = %d (expected %d), %d mismatches\n", out_ptr[0], c, bad);
  CHECK(XAie_PartitionTeardown(&dev));
  return bad != 0;
}

/* vek385_verification.cpp:72-230: the 3x3 kernel on rows 3..6 of every
 * column, inputs written straight into tile memory, cores enabled one by
 * one and read back while "running". */
static int flow_vek385(int num_cols) {
  enum { START_ROW = 3, END_ROW = 6 };
  const uint64_t CORE_IP_MEM = 0x1000, CORE_OP_MEM = 0x5000;
  XAie_DevInst dev;
  open_device(&dev, 0, 0);
  for (int col = 0; col < num_cols; col++) {
    for (int r = START_ROW; r <= END_ROW; r++) {
      CHECK(XAie_CoreReset(&dev, XAie_TileLoc(col, r)));
      CHECK(XAie_CoreUnreset(&dev, XAie_TileLoc(col, r)));
      CHECK(XAie_LoadElfMem(&dev, XAie_TileLoc(col, r), (const unsigned char*)&miaie_xaie_mm3_u64));
    }
    for (uint64_t r = START_ROW; r <= END_ROW; r++) {
      uint64_t input[9];
      for (int e = 0; e < 9; e++) input[e] = r;
      CHECK(XAie_DataMemBlockWrite(&dev, XAie_TileLoc(col, (u8)r), CORE_IP_MEM, input, sizeof input));
    }
    for (int r = START_ROW; r <= END_ROW; r++) CHECK(XAie_CoreEnable(&dev, XAie_TileLoc(col, r)));
  }
  int failed_cols = 0, executing = 0;
  const int expected[END_ROW - START_ROW + 1] = {27, 48, 75, 108}; /* vek385_verification.cpp:138 */
  uint64_t last[10] = {0};
  for (int col = 0; col < num_cols; col++) {
    int bad = 0;
    for (int i = 0; i <= END_ROW - START_ROW; i++) {
      u8 done = 1;
      CHECK(XAie_CoreReadDoneBit(&dev, XAie_TileLoc(col, START_ROW + i), &done));
      executing += done == 0;
      CHECK(XAie_DataMemBlockRead(&dev, XAie_TileLoc(col, START_ROW + i), CORE_OP_MEM, last, sizeof last));
      for (int e = 0; e < 9; e++) bad += last[e] != (uint64_t)expected[i];
      if (last[9] == 0) bad++;
    }
    failed_cols += bad != 0;
  }
  for (int r = START_ROW; r <= END_ROW; r++) CHECK(XAie_CoreDisable(&dev, XAie_TileLoc(1 % num_cols, r)));
  u8 done = 0;
  CHECK(XAie_CoreReadDoneBit(&dev, XAie_TileLoc(1 % num_cols, START_ROW), &done));
  printf("%d columns x %d rows: %d columns failed, %d cores executing while enabled, disabled core done=%u\n",
         num_cols, END_ROW - START_ROW + 1, failed_cols, executing, done);
  printf("out[0] = %llu, iterations = %llu\n", (unsigned long long)last[0], (unsigned long long)last[9]);
  CHECK(XAie_PartitionTeardown(&dev));
  return failed_cols != 0 || executing != num_cols * (END_ROW - START_ROW + 1) || done != 1;
}

/* aieoob.c:76-150: the kernel-instance calls on an 8x8 window. */
static int flow_oob(void) {
  enum { DATA_SIZE = 128, MAT_SIZE = 64, N = 8 };
  const size_t bytes = DATA_SIZE * sizeof(uint32_t);
  uint32_t* h_a = (uint32_t*)malloc(bytes);
  uint32_t* h_c = (uint32_t*)malloc(bytes);
  for (int i = 0; i < DATA_SIZE; i++) {
    h_a[i] = (uint32_t)i;
    h_c[i] = 0;
  }
  XAie_Kernel_Inst* k = XAie_LoadKernel("mm", 12, 3);
  if (!k) {
    fprintf(stderr, "XAie_LoadKernel: %s\n", XAie_MiaieLastError(NULL));
    return 1;
  }
  CHECK(XAie_RoutingHostToAie(k, XAie_TileLoc(2, 0)));
  CHECK(XAie_RoutingAieToHost(k, XAie_TileLoc(35, 0)));
  CHECK(XAie_MoveDataToAie(k, 1, h_a, bytes));
  CHECK(XAie_RunCore(k));
  CHECK(XAie_WaitOutData(k));
  CHECK(XAie_MoveAieToData(k, 1, h_c, bytes));
  const int bad = golden_mismatches((const int32_t*)h_a, (const int32_t*)h_c, N);
  printf("C[0][0] = %d, C[7][7] = %d\n", (int)h_c[0], (int)h_c[MAT_SIZE - 1]);
  if (bad == 0)
    printf("oob: CPU result matches the device output.\n");
  else
    printf("oob: there were %d mismatches.\n", bad);
  CHECK(XAie_KernelFree(k));
  free(h_a);
  free(h_c);
  return bad != 0;
}

#define EXPECT_RC(call, want)                                                                          \
  do {                                                                                                 \
    AieRC rc_ = (call);                                                                                \
    if (rc_ != (want)) {                                                                               \
      fprintf(stderr, "%s:%d: %s -> %d, expected %d (%s)\n", __FILE__, __LINE__, #call, (int)rc_, \
              (int)(want), XAie_MiaieLastError(NULL));                                                 \
      return 1;                                                                                        \
    }                                                                                                  \
    printf("rejected as expected: %s -> %s\n", #call, XAie_MiaieLastError(NULL));                      \
  } while (0)

/* What the facade must refuse, each without launching anything. */
static int flow_errors(void) {
  XAie_DevInst dev;
  open_device(&dev, 0, 0);
  const XAie_LocType core = XAie_TileLoc(4, 4), shim = XAie_TileLoc(2, 0), other = XAie_TileLoc(5, 4);
  unsigned char not_a_kernel[64] = {0};
  EXPECT_RC(XAie_LoadElfMem(&dev, core, not_a_kernel), XAIE_INVALID_ELF);
  EXPECT_RC(XAie_LoadElfMem(&dev, XAie_TileLoc(4, 1), (const unsigned char*)&miaie_xaie_mm), XAIE_INVALID_TILE);
  EXPECT_RC(XAie_CoreReset(&dev, XAie_TileLoc(40, 4)), XAIE_INVALID_TILE);
  CHECK(XAie_CoreReset(&dev, core));
  CHECK(XAie_CoreUnreset(&dev, core));
  CHECK(XAie_LoadElfMem(&dev, core, (const unsigned char*)&miaie_xaie_mm));
  XAie_RoutingInstance* ri = XAie_InitRoutingHandler(&dev);
  XAie_MemInst* in = XAie_MemAllocate(&dev, 2048, XAIE_MEM_CACHEABLE);
  /* no route yet */
  EXPECT_RC(XAie_MoveDataExternal2Aie(ri, shim, in, 2048, 0x1000, core), XAIE_ERR_NO_ROUTE);
  CHECK(XAie_Route(ri, NULL, shim, core));
  /* a tile that is not on any route of this instance */
  EXPECT_RC(XAie_MoveData(ri, core, (void*)0x6000, 64, (void*)0x1000, other), XAIE_ERR_NO_ROUTE);
  /* a DDR address no XAie_MemAllocate buffer holds */
  int stack_word = 0;
  EXPECT_RC(XAie_MoveData(ri, shim, &stack_word, 4, (void*)0x1000, core), XAIE_INVALID_ARGS);
  /* more than the buffer holds */
  EXPECT_RC(XAie_MoveDataExternal2Aie(ri, shim, in, 4096, 0x1000, core), XAIE_INVALID_ARGS);
  /* past the end of the 64 KiB data memory */
  EXPECT_RC(XAie_MoveDataExternal2Aie(ri, shim, in, 2048, 0xFC00, core), XAIE_INVALID_DATA_MEM_ADDR);
  uint32_t w = 0;
  EXPECT_RC(XAie_DataMemRdWord(&dev, core, 0x10000, &w), XAIE_INVALID_DATA_MEM_ADDR);
  EXPECT_RC(XAie_DataMemRdWord(&dev, shim, 0, &w), XAIE_INVALID_TILE);
  /* a core that never ran is not done; a run with zero iterations is refused */
  EXPECT_RC(XAie_CoreWaitForDone(&dev, core, 100), XAIE_CORE_STATUS_TIMEOUT);
  EXPECT_RC(XAie_Run(ri, 0), XAIE_INVALID_ARGS);
  CHECK(XAie_MoveDataExternal2Aie(ri, shim, in, 2048, 0x1000, core));
  CHECK(XAie_Run(ri, 3));
  wait_core(&dev, core);
  u32 status = 0;
  CHECK(XAie_CoreGetStatus(&dev, core, &status));
  if (!(status & XAIE_CORE_STATUS_DONE_BIT)) {
    fprintf(stderr, "status 0x%x lacks the done bit after a run\n", status);
    return 1;
  }
  /* reset clears enable; a core in reset cannot be enabled */
  CHECK(XAie_CoreReset(&dev, core));
  EXPECT_RC(XAie_CoreEnable(&dev, core), XAIE_ERR);
  EXPECT_RC(XAie_Run(ri, 1), XAIE_ERR);
  CHECK(XAie_PartitionTeardown(&dev));
  EXPECT_RC(XAie_CoreReset(&dev, core), XAIE_INVALID_DEVICE);
  EXPECT_RC(XAie_CfgInitialize(NULL, NULL), XAIE_INVALID_ARGS);
  if (XAie_LoadKernel("no_such_kernel", 4, 4) != NULL) return 1;
  printf("errors: all rejected as expected.\n");
  return 0;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s mm [reps]|mm8 [reps]|perf [reps]|multi_tile|seq_full_col|vek385 [cols]|oob|errors\n",
            argv[0]);
    return 64;
  }
  const char* cmd = argv[1];
  const int reps = argc > 2 ? atoi(argv[2]) : 1;
  if (!strcmp(cmd, "mm") || !strcmp(cmd, "mm8") || !strcmp(cmd, "perf")) {
    if (reps < 1 || reps > 100000) return 64;
    if (!strcmp(cmd, "mm")) return flow_window(&miaie_xaie_mm, 16, 0, 0, 2, 0, 0, reps);  /* aieml_mm.cc:137-140 */
    if (!strcmp(cmd, "mm8")) return flow_window(&miaie_xaie_mm8, 8, 0, 0, 2, 0, 0, reps); /* aieml_mm.cc:257, 8x8 */
    return flow_window(&miaie_xaie_perf, 16, 2, 34, 33, 1, 1, reps);                      /* aieml_perf.cc:141-144 */
  }
  if (!strcmp(cmd, "multi_tile")) return flow_multi_tile();
  if (!strcmp(cmd, "seq_full_col")) return flow_seq_full_col();
  if (!strcmp(cmd, "vek385")) {
    const int cols = argc > 2 ? atoi(argv[2]) : XAIE_NUM_COLS;
    if (cols < 1 || cols > XAIE_NUM_COLS) return 64;
    return flow_vek385(cols);
  }
  if (!strcmp(cmd, "oob")) return flow_oob();
  if (!strcmp(cmd, "errors")) return flow_errors();
  fprintf(stderr, "unknown subcommand %s\n", cmd);
  return 64;
}
