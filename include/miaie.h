/*
 * miaie.h — C ABI of the MI355X (gfx950) GEMM/conv path.
 *
 * This is the drop-in boundary for the data-parallel path that
 * Xilinx/aiehlc compiles onto the AI Engine array.  Every entry point takes
 * plain device pointers and sizes (no C++ or torch types) and returns an int
 * status: MIAIE_OK (0) on success, a negative MIAIE_E* code otherwise — the
 * same "0 means OK" convention as aie-rt's AieRC/XAIE_OK that the reference
 * harnesses test (example/perf/aieml_perf.cc:283-310).  Nothing throws
 * across this ABI.  Arguments are validated before any launch; on error
 * miaie_last_error_string() describes the first problem.
 *
 * Kernel launches are asynchronous on the context's HIP stream (the
 * XAie_Run analogue); miaie_wait() is the XAie_CoreWaitForDone analogue,
 * with a real deadline.  A context is thread-compatible, not thread-safe:
 * use one context per host thread.  The caller owns every device buffer;
 * no compute entry point allocates device memory.
 *
 * Reference citations are relative to the Xilinx/aiehlc source tree.
 */
#ifndef MIAIE_H
#define MIAIE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIAIE_API __attribute__((visibility("default")))

/* ---- status codes ------------------------------------------------------ */
#define MIAIE_OK 0
#define MIAIE_EINVAL (-1)       /* bad argument: null pointer, shape, stride, alignment */
#define MIAIE_EHIP (-2)         /* a HIP runtime call failed */
#define MIAIE_ETIMEDOUT (-3)    /* miaie_wait deadline passed before the stream drained */
#define MIAIE_ENOMEM (-4)       /* device allocation failed */
#define MIAIE_EUNSUPPORTED (-5) /* valid request this build does not implement */
#define MIAIE_EFAULT (-6)       /* debug build: a kernel access outside every known buffer (miaie_wait) */

/* B operand layout of the int8 GEMM.  NT is the reference golden's layout:
 * B stored as [N][K] ("column major", aieml_mm.cc:210-215).  NN is the
 * benchmark layout: B stored as [K][N] row major. */
#define MIAIE_B_NN 0
#define MIAIE_B_NT 1

typedef struct miaie_ctx miaie_ctx;

/* ---- runtime: the aie-rt host calls the reference harnesses make ------- */

/* Replaces XAie_SetupConfig + XAie_CfgInitialize + XAie_PartitionInitialize
 * (example/perf/aieml_perf.cc:265-313).  Binds `device` and creates a
 * stream owned by the context.  It also allocates the context's 16 MiB
 * device workspace (split-K partial sums of deep convolutions), released by
 * miaie_finish, so that no compute entry point allocates. */
MIAIE_API int miaie_init(miaie_ctx** ctx, int device);

/* As miaie_init, but launches go to the caller's hipStream_t `stream`
 * (borrowed, not destroyed by miaie_finish).  NULL selects the null stream. */
MIAIE_API int miaie_init_on_stream(miaie_ctx** ctx, int device, void* stream);

/* Replaces XAie_PartitionTeardown (aieml_perf.cc:321).  Waits for the
 * stream, then releases the context.  NULL is a no-op. */
MIAIE_API int miaie_finish(miaie_ctx* ctx);

/* Text of the most recent error on this context ("" if none).  A NULL
 * context returns the text of the most recent miaie_init failure. */
MIAIE_API const char* miaie_last_error_string(const miaie_ctx* ctx);

/* The hipStream_t that launches go to. */
MIAIE_API int miaie_get_stream(miaie_ctx* ctx, void** stream);

/* Replaces XAie_MemAllocate + XAie_MemGetDevAddr (aieml_perf.cc:132-135).
 * 256-byte aligned device memory. */
MIAIE_API int miaie_alloc(miaie_ctx* ctx, size_t bytes, void** dev_ptr);
MIAIE_API int miaie_free(miaie_ctx* ctx, void* dev_ptr);

/* Replace XAie_MoveDataExternal2Aie / XAie_MoveData (host -> tile) and
 * XAie_MoveDataAie2External (tile -> host) together with
 * XAie_MemSyncForDev / XAie_MemSyncForCPU (aieml_perf.cc:148-188,
 * aieml_mm.cc:149-151,184-187).  Ordered on the context stream; they return
 * once the copy has completed. */
MIAIE_API int miaie_copy_h2d(miaie_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
MIAIE_API int miaie_copy_d2h(miaie_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);

/* Device-to-device copy by miaie's own streaming kernel (asynchronous).
 * The tile->tile XAie_MoveData of example/multi/multi_tile.cpp:125-127;
 * also the known-size copy used to calibrate HBM byte counters. */
MIAIE_API int miaie_copy_d2d(miaie_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes);

/* Replaces the busy loop over XAie_CoreWaitForDone (aieml_perf.cc:174-184),
 * which has no deadline.  Returns MIAIE_OK once all work queued on the
 * context has finished, MIAIE_ETIMEDOUT if timeout_ms elapses first
 * (timeout_ms < 0 waits without a deadline). */
MIAIE_API int miaie_wait(miaie_ctx* ctx, int timeout_ms);

/* ---- device bounds checks (debug build) --------------------------------- */

/* No counterpart in the reference, whose kernels run unchecked on the AIE
 * tiles.  The debug build of this library (aiehlc_amd/lib_dbg/, built with
 * MIAIE_DEVICE_CHECKS=1) checks every global load, store and global->LDS copy
 * of its kernels against a table of known buffers: every live miaie_alloc
 * allocation, the context's workspace, the allocation-free entry points'
 * scratch array, and whatever the caller declares here.  An access that no
 * buffer contains is not performed (a load reads zeros, a store or copy is
 * dropped) and is counted; miaie_wait then returns MIAIE_EFAULT, and
 * miaie_last_error_string names the first such access (load/store/copy,
 * bytes, address, source file and line).  The product build checks nothing:
 * miaie_debug_device_checks returns 0 there and the two calls below only
 * validate their arguments.  Changing the table waits for the whole device
 * to go idle. */
MIAIE_API int miaie_debug_device_checks(void);
/* Declare [dev_ptr, dev_ptr + bytes) as a buffer kernels may touch (memory
 * not from miaie_alloc), or give a known buffer (same dev_ptr) a new extent,
 * e.g. a smaller one to check that a kernel stays inside it.  A range that
 * overlaps another known buffer is refused with MIAIE_EINVAL. */
MIAIE_API int miaie_debug_register(miaie_ctx* ctx, const void* dev_ptr, size_t bytes);
/* Forget the buffer that starts at dev_ptr (miaie_free does this itself). */
MIAIE_API int miaie_debug_unregister(miaie_ctx* ctx, const void* dev_ptr);

/* ---- GEMM planning ------------------------------------------------------ */

#define MIAIE_KERNEL_TILE64 0     /* bounds-checked 64x64 kernel, any shape and stride */
#define MIAIE_KERNEL_PIPE 1       /* pipelined tile_m x tile_n kernel, 4-stage LDS DMA pipeline; M >= tile_m,
                                     N >= tile_n, and N % 16 == 0 where tile_n does not divide N (the
                                     last tile row/column overlaps the one before it) */
#define MIAIE_KERNEL_PIPE_MIXED 2 /* pipelined kernel, 256x256 tiles over the first columns and 256x128
                                     tiles over the rest, in one launch (tile_m = tile_n = 256) */

/* How miaie_gemm_i8_rq would run an M x N x K product on this context with
 * dense 16-byte-aligned NN operands (the tiling planner: the grid
 * decomposition and tile choice that stand in for the reference's tiling
 * prototype, src/mlir/mlirfront/tilinglinalg/tilinglinalg.cpp:38-146).
 * miaie_gemm_i8_i32 runs the same plan, except that for K >= 2^16, where the
 * requantizing entry takes the 64x64 kernel, it keeps the pipelined one. */
typedef struct {
  int kernel;         /* MIAIE_KERNEL_* */
  int tile_m, tile_n; /* workgroup output tile */
  int workgroups;     /* grid size */
  int threads;        /* per workgroup */
} miaie_gemm_plan;
MIAIE_API int miaie_plan_gemm_i8(miaie_ctx* ctx, int M, int N, int K, miaie_gemm_plan* plan);

/* The number of compute units the planner distributes tiles over on this
 * context (the reference prototype's thread count, numThreads = {8, 16} at
 * src/mlir/mlirfront/tilinglinalg/tilinglinalg.cpp:101).  It starts at the
 * device's CU count; a caller sharing the GPU with other streams can plan for
 * fewer.  cus >= 1; *previous (nullable) receives the old value. */
MIAIE_API int miaie_plan_set_cus(miaie_ctx* ctx, int cus, int* previous);

/* Which kernel miaie_conv2d_i8_nhwc runs for a shape, given 16-byte aligned
 * X, W and Y and 4-byte aligned shifts (what miaie_alloc returns).  The
 * reference's conv exists only as AIE graph configuration
 * (thirdparty/adf/aie_control.cpp:2554-2559), so there is no reference
 * counterpart; the choice is exposed so callers and tests can see it.  Needs
 * no context and no device: it reports the choice for a 256-CU MI355X.  A
 * launch weighs the same estimates on its context's CU count (the device's,
 * or miaie_plan_set_cus), which may pick another kernel where two apply.
 * Invalid shapes return MIAIE_EINVAL, as the entry point does. */
#define MIAIE_CONV_ROWS 0   /* row-block kernel: 3x3, stride 1, Cin 32/64/128, Cout % 32 == 0 (rows in blocks of 64) */
#define MIAIE_CONV_IGEMM 1  /* implicit-GEMM kernel: Cin % 32 == 0, Cout % 64 == 0 */
#define MIAIE_CONV_DIRECT 2 /* any shape, one thread per output element */
#define MIAIE_CONV_TAPS 3   /* LDS-staged implicit GEMM over filter taps: Cin % 128 == 0, Cout % 64 == 0 */
#define MIAIE_CONV_ROWS_DEEP 4 /* row-block kernel over 64-channel chunks of Cin: 3x3, stride 1, Cin % 64 == 0 up to 4096, Cout % 32 == 0 */
MIAIE_API int miaie_plan_conv2d_i8(int N, int H, int W, int Cin, int Cout, int R, int S, int stride, int pad,
                                   int* kernel);

/* ---- recorded kernel chains --------------------------------------------- */

/* The reference chains kernels through the host: run k1, wait, move k1's
 * output to k2's input tile, run k2, wait (example/multi/multi_tile.cpp:
 * 110-140, seq_full_col.cpp:137-152).  Here a chain of entry points is
 * recorded once as a HIP graph and replayed with one call: intermediates
 * stay in device memory and no host step runs between kernels.
 *
 * miaie_graph_begin starts recording the context's stream.  Entry points
 * called until miaie_graph_end are recorded, not run; the arguments
 * (pointers, shapes) are fixed at recording time, while the buffers'
 * contents are read at replay time.  While recording, entry points that
 * wait for the device or allocate (miaie_copy_h2d, miaie_copy_d2h,
 * miaie_wait, miaie_alloc, miaie_free) return MIAIE_EINVAL and record
 * nothing.  A context created on the null stream cannot record
 * (MIAIE_EUNSUPPORTED).  miaie_graph_launch queues one replay on the
 * context's stream (asynchronous, like any launch).  A graph replays only on
 * the context that recorded it (another context gets MIAIE_EINVAL), before
 * that context's miaie_finish: a recorded convolution may use the context's
 * workspace. */
typedef struct miaie_graph miaie_graph;
MIAIE_API int miaie_graph_begin(miaie_ctx* ctx);
MIAIE_API int miaie_graph_end(miaie_ctx* ctx, miaie_graph** graph);
MIAIE_API int miaie_graph_launch(miaie_ctx* ctx, miaie_graph* graph);
/* Waits for nothing: destroy a graph only once its replays have finished. */
MIAIE_API int miaie_graph_destroy(miaie_graph* graph);

/* ---- reference kernels (single AIE tile in the reference) -------------- */

/* `mm` of example/matrixmultiply/aieml_mm.cc:41-93 and `perf` of
 * example/perf/aieml_perf.cc:61-83: one packed input window
 * in[0 .. n*n) = A (n x n, row major) followed by in[n*n .. 2*n*n) = B
 * stored [N][K]; out (n x n, row major) = A . B^T with int32 wrap-around
 * arithmetic, zero-initialised (the CPU golden of aieml_mm.cc:194-230).
 * n in [1, 4096]. */
MIAIE_API int miaie_mm_window_i32(miaie_ctx* ctx, const int32_t* in_window, int32_t* out_window, int n);
/* Same kernel, typed as the uint32 `perf` variant (aieml_perf.cc:69-81). */
MIAIE_API int miaie_perf_window_u32(miaie_ctx* ctx, const uint32_t* in_window, uint32_t* out_window, int n);

/* `perf` of example/nokernelload/aie_nokernelload.cc:50-83: the uint8
 * dot-product MAC probe.  in[0] = param_nn; out[0..4] =
 * {3*param_nn, 4567, 3*param_nn*dot (mod 2^32), 3, vec1[0]} where dot is the
 * 128-element dot of the reference's vectors.  The 3*param_nn*128 MACs are
 * executed on int8 MFMA across the whole GPU, so the call also measures
 * MAC throughput. */
MIAIE_API int miaie_dot_u8_probe(miaie_ctx* ctx, const uint32_t* in, uint32_t* out);

/* `mm` of example/multi/vek385_verification.cpp:56-69, replicated over
 * `batch` independent tiles as the reference replicates it over every AIE
 * tile (:208-215): out_b = in_b . in_b (n x n, NN), uint64 storage, the sum
 * held in a 32-bit int, out_b[n*n] = iters (the reference's pass counter;
 * it loops forever, this runs `iters` passes).  Tile b reads
 * in + b*n*n and writes out + b*(n*n+1).  n in [1, 64]. */
MIAIE_API int miaie_mm_square_u64(miaie_ctx* ctx, const uint64_t* in, uint64_t* out, int n, int batch,
                                  uint64_t iters);

/* k1 -> k2 chains of example/multi/multi_tile.cpp:39-47,125-127 and
 * seq_full_col.cpp:39-47,146-151: stage s writes out_s[i] = in_s[0] +
 * addends[s] for i < len and feeds the next stage, all on the device with no
 * host round trip (one launch).  addends is a host array of nstages. */
MIAIE_API int miaie_chain_add_i32(miaie_ctx* ctx, const int32_t* in, int32_t* out, int len,
                                  const int32_t* addends, int nstages);

/* ---- typed GEMM / conv entries (the benchmark's shapes) ---------------- */

/* int8 x int8 -> int32 GEMM, C = A . B.  A: M x K row major (lda >= K).
 * b_layout MIAIE_B_NN: B is K x N row major (ldb >= N); MIAIE_B_NT: B is
 * N x K row major (ldb >= K).  C: M x N row major (ldc >= N).  Generalises
 * the reference golden loop (aieml_mm.cc:217-223) to int8 operands and any
 * M, N, K >= 1. */
MIAIE_API int miaie_gemm_i8_i32(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int32_t* C, int M,
                                int N, int K, int lda, int ldb, int ldc, int b_layout);

/* int8 GEMM with the fused requantize epilogue:
 *   Y = sat_int8((acc + 2^(shift-1)) >> shift), arithmetic shift,
 *   round half up, then ReLU if relu != 0; shift in [0, 31] (0: saturate only).
 * Dense row-major A (M x K), B (NN: K x N, NT: N x K), Y (M x N).
 * C_dbg, if not NULL, also receives the int32 accumulators (M x N). */
MIAIE_API int miaie_gemm_i8_rq(miaie_ctx* ctx, const int8_t* A, const int8_t* B, int8_t* Y, int M,
                               int N, int K, int shift, int relu, int32_t* C_dbg, int b_layout);

/* bf16 x bf16 -> fp32 GEMM, fp32 accumulate, dense row major NN:
 * A M x K, B K x N, C M x N.  bf16 values are passed as raw uint16 bits. */
MIAIE_API int miaie_gemm_bf16_f32(miaie_ctx* ctx, const uint16_t* A, const uint16_t* B, float* C, int M,
                                  int N, int K);

/* int8 conv2d, NHWC activations X[N][H][W][Cin], OHWI weights
 * W[Cout][R][S][Cin], zero padding, stride, per-output-channel requant
 * Y = sat_int8((acc + 2^(s_c-1)) >> s_c) with s_c = shifts[c] in [0, 31]
 * (a device array the library cannot check: other values give unspecified
 * results), Y[N][Ho][Wo][Cout] with Ho = (H + 2*pad - R)/stride + 1 (Wo
 * alike).  Any shape: 3x3 stride-1 convolutions with Cin 32, 64 or 128 and
 * Cout a multiple of 32 take the row-block kernel, and with another Cin
 * that is a multiple of 64 (up to 4096) the row-block kernel over
 * 64-channel chunks, or the taps kernel where its estimated time is lower;
 * Cin a multiple of 128 with Cout a multiple of 64 the LDS-staged taps
 * kernel; Cin a multiple of 32 with Cout a multiple of 64 the implicit-GEMM
 * kernel (the last two split K over workgroups for small grids, through the
 * context's workspace); everything else a direct kernel
 * (miaie_plan_conv2d_i8 reports which).
 * R*S*Cin above 2^30 or N*H*W*Cin above 2^40 return MIAIE_EINVAL. */
MIAIE_API int miaie_conv2d_i8_nhwc(miaie_ctx* ctx, const int8_t* X, const int8_t* W,
                                   const uint8_t* shifts, int8_t* Y, int N, int H, int W_, int Cin,
                                   int Cout, int R, int S, int stride, int pad);

/* Chained int8 MLP (the multi_tile.cpp k1 -> k2 chain at scale):
 *   H = relu(rq_s1(X . W1)),  Y = rq_s2(H . W2)
 * X: M x K, W1: K x F, W2: F x Nout, H: M x F (caller-provided device
 * scratch), Y: M x Nout, all int8 row major NN.  Both GEMMs are queued
 * back to back on the context stream; H never leaves the device. */
MIAIE_API int miaie_mlp_i8(miaie_ctx* ctx, const int8_t* X, const int8_t* W1, const int8_t* W2,
                           int8_t* H, int8_t* Y, int M, int K, int F, int Nout, int s1, int s2);

/* Allocation-free variant of miaie_mlp_i8.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as miaie_mlp_i8 without H: H lives in a file-scope
 * device array of MIAIE_MLP_NOALLOC_MAX_H bytes that every GPU the library
 * runs on holds from miaie_init until the process ends.  M*F above that
 * returns MIAIE_EINVAL without launching.  The call allocates nothing.  All
 * calls on one GPU share that GPU's array.  Eager calls from different
 * streams or contexts are ordered on the device (each waits for the previous
 * call's use of the array through one event per GPU), so they queue behind
 * each other rather than overlap.  A call recorded into a graph is not part
 * of that order: its replays race with any other use of the array that
 * overlaps them on the same GPU. */
#define MIAIE_MLP_NOALLOC_MAX_H ((size_t)32 << 20)
MIAIE_API int miaie_mlp_i8_noalloc(miaie_ctx* ctx, const int8_t* X, const int8_t* W1, const int8_t* W2, int8_t* Y,
                                   int M, int K, int F, int Nout, int s1, int s2);

/* ---- synthetic inputs --------------------------------------------------- */

/* Fill dst[0..n) with the seeded int8 stream of tensor `tensor_id`
 * (SplitMix64; element i = (int8)(mix(state0 + (i+1)*gamma) >> 56) with
 * state0 = mix(0x5EED0000 + tensor_id + gamma)).  Generated on the device. */
MIAIE_API int miaie_fill_i8(miaie_ctx* ctx, int8_t* dst, size_t n, uint64_t tensor_id);

/* ---- build information -------------------------------------------------- */
MIAIE_API const char* miaie_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MIAIE_H */
