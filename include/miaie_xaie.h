/*
 * miaie_xaie.h — aie-rt-shaped host facade over miaie (libmiaie_xaie.so).
 *
 * The reference's example programs drive the AI Engine array through
 * aie-rt's C API (XAie_*): configure a partition, reset and load cores,
 * route the shim DMA to the tiles, allocate DDR, move data into the tiles'
 * data memories, run, poll for done, move the result back, compare with a
 * CPU golden.  aie-rt itself is not vendored with the reference; every
 * signature below is inferred from the reference's call sites, cited per
 * function.  A harness written against those calls compiles against this
 * header (in place of xaiengine.h) and links -lmiaie_xaie -lmiaie.
 *
 * How the array maps onto one MI355X:
 *   - Each tile of the configured partition has a data memory (64 KiB for a
 *     core tile, 512 KiB for a memory tile, none for a shim tile), all held in
 *     one HBM slab allocated by XAie_CfgInitialize.  Tile addresses
 *     (CORE_IP_MEM 0x1000, CORE_OP_MEM 0x5000/0x6000 in the examples) are
 *     byte offsets into that tile's memory.
 *   - "DDR" (XAie_MemInst) is host memory.  On x86-64 it is mapped below
 *     4 GiB, so a harness that keeps XAie_MemGetDevAddr() in a u32
 *     (aieml_mm.cc:133) still holds a usable address; the address is the
 *     host virtual address, so writing through it (aieml_mm.cc:137-140) is
 *     writing the buffer.
 *   - Moves between DDR and a tile are host<->device copies; tile-to-tile
 *     moves are device copies inside the slab.  Every move is complete when
 *     the call returns, after all kernels queued before it.
 *   - An "ELF" is an XAie_MiaieKernel descriptor.  XAie_Run launches one grid
 *     per distinct kernel over every routed, loaded, out-of-reset tile, one
 *     workgroup per tile: the replicated-per-tile pattern of
 *     vek385_verification.cpp:208-215 becomes one data-parallel launch.
 *   - Routes are recorded and checked: a move between two tiles needs an
 *     XAie_Route between them first, as on the array.
 *
 * Status: AieRC, XAIE_OK == 0 on success.  XAie_MiaieLastError() gives the
 * text of the last failure on a device instance.  Nothing here is
 * thread-safe; use one device instance per thread.
 *
 * Reference citations are relative to the Xilinx/aiehlc source tree.
 */
#ifndef MIAIE_XAIE_H
#define MIAIE_XAIE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIAIE_XAIE_API __attribute__((visibility("default")))

/* The BSP's fixed-width names, which the harnesses use throughout
 * (aieml_mm.cc:124-127, multi_tile.cpp:89). */
#ifndef MIAIE_XAIE_NO_XIL_TYPES
typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;
#endif

/* ---- status ----------------------------------------------------------- */
typedef enum {
  XAIE_OK = 0,                 /* the only value the harnesses test (aieml_perf.cc:283-310) */
  XAIE_ERR = 1,                /* HIP failure or internal error */
  XAIE_INVALID_DEVICE = 2,     /* instance not initialised, or no GPU */
  XAIE_INVALID_ARGS = 3,       /* null pointer, bad size, unknown address */
  XAIE_INVALID_TILE = 4,       /* location outside the partition, or wrong tile type */
  XAIE_INVALID_DATA_MEM_ADDR = 5, /* range outside the tile's data memory */
  XAIE_INVALID_ELF = 6,        /* LoadElfMem got something that is not an XAie_MiaieKernel */
  XAIE_CORE_STATUS_TIMEOUT = 7,/* CoreWaitForDone deadline passed */
  XAIE_ERR_NO_ROUTE = 8,       /* move between tiles with no XAie_Route between them */
  XAIE_NOT_SUPPORTED = 9
} AieRC;

/* Device generations as the harnesses select them (aieml_perf.cc:14-19,
 * :293: generation 5 is AIE2PS). */
#define XAIE_DEV_GEN_AIE 1
#define XAIE_DEV_GEN_AIEML 2
#define XAIE_DEV_GEN_AIE2IPU 3
#define XAIE_DEV_GEN_AIE2P 4
#define XAIE_DEV_GEN_AIE2PS 5

typedef enum { XAIE_MEM_NONCACHEABLE = 0, XAIE_MEM_CACHEABLE = 1 } XAie_MemCacheProp;

typedef enum {
  XAIE_IO_BACKEND_BAREMETAL = 0, /* what every example selects (aieml_perf.cc:286) */
  XAIE_IO_BACKEND_LINUX = 1,
  XAIE_IO_BACKEND_MIAIE_HIP = 2  /* what actually runs underneath */
} XAie_BackendType;

typedef struct {
  XAie_BackendType Type; /* read as DevInst.Backend->Type (aieml_perf.cc:289) */
  const char* Name;
} XAie_Backend;

/* Tile coordinate.  XAie_TileLoc(col, row) (aieml_mm.cc:113). */
typedef struct {
  u8 Row;
  u8 Col;
} XAie_LocType;

static inline XAie_LocType XAie_TileLoc(u8 col, u8 row) {
  XAie_LocType l;
  l.Row = row;
  l.Col = col;
  return l;
}

/* Array geometry, as XAie_SetupConfig lists it (aieml_perf.cc:265-269). */
typedef struct {
  u8 AieGen;
  u64 BaseAddr;
  u8 ColShift;
  u8 RowShift;
  u8 NumCols;
  u8 NumRows;
  u8 ShimRowNum;
  u8 MemTileRowStart;
  u8 MemTileNumRows;
  u8 AieTileRowStart;
  u8 AieTileNumRows;
} XAie_Config;

#define XAie_SetupConfig(Config, Gen, Base, ColSh, RowSh, NCols, NRows, ShimRow, MemStart, MemNum, AieStart, AieNum) \
  XAie_Config Config = {(u8)(Gen), (u64)(Base), (u8)(ColSh), (u8)(RowSh), (u8)(NCols), (u8)(NRows),                  \
                        (u8)(ShimRow), (u8)(MemStart), (u8)(MemNum), (u8)(AieStart), (u8)(AieNum)}

struct miaie_xaie_dev;

/* One AI Engine partition, here one GPU.  Declared by XAie_InstDeclare
 * (aieml_perf.cc:273) and set up by XAie_CfgInitialize. */
typedef struct {
  const XAie_Backend* Backend;
  u8 IsReady;
  u8 AieGen;
  u64 BaseAddr;
  u8 NumCols;
  u8 NumRows;
  u8 ShimRow;
  u8 MemTileRowStart;
  u8 MemTileNumRows;
  u8 AieTileRowStart;
  u8 AieTileNumRows;
  u8 StartCol;        /* partition: first column (XAie_SetupPartitionConfig) */
  u8 PartNumCols;     /* partition: columns; 0 = the whole array */
  u64 PartBaseAddr;
  struct miaie_xaie_dev* Priv; /* facade state: device, tile memories, cores */
} XAie_DevInst;

#ifdef __cplusplus
#define XAie_InstDeclare(Inst, ConfigPtr) XAie_DevInst Inst = {}
#else
#define XAie_InstDeclare(Inst, ConfigPtr) XAie_DevInst Inst = {0}
#endif

typedef struct XAie_MemInst XAie_MemInst;
typedef struct XAie_RoutingInstance XAie_RoutingInstance;

/* ---- kernels ("ELFs") --------------------------------------------------- */
/* What XAie_LoadElfMem loads.  In the reference the argument is the AIE ELF
 * that aiehlc compiled from a `__global__` function (aieml_mm.cc:115 passes
 * `(unsigned char *)mm`); here it is a descriptor of a gfx950 kernel that
 * runs on the tile's data memory.  Each parameter is a window whose ping
 * buffer address follows the reference's layout rule (see
 * XAie_MiaieWindowLayout). */
#define MIAIE_XAIE_KERNEL_MAGIC 0x4b45494du /* "MIEK" */
#define MIAIE_XAIE_MAX_PARAMS 4
#define MIAIE_XAIE_KERNEL_FOREVER 1u /* the reference body never returns (vek385_verification.cpp:58) */

/* Launch hook of a user kernel.  `tile_mem` is the device address of the
 * tile-memory slab, `tile_offsets` (host array, `ntiles` entries) the byte
 * offset of each participating tile's data memory in it, `ping` (host array,
 * `nparams` entries) the window addresses inside a tile memory, `stream` the
 * hipStream_t to launch on.  Returns 0 or a negative miaie status. */
typedef int (*XAie_MiaieLaunchFn)(void* stream, void* tile_mem, const u32* tile_offsets, u32 ntiles,
                                  const u32* ping, u32 nparams, u32 iterations, void* user);

typedef struct {
  u32 Magic;                              /* MIAIE_XAIE_KERNEL_MAGIC */
  const char* Name;
  u32 NumParams;
  u32 MemAddress[MIAIE_XAIE_MAX_PARAMS];  /* annotate("mem_address:...") or 0 */
  u32 SizeHint[MIAIE_XAIE_MAX_PARAMS];    /* annotate("size_hint:...") in words, or 0 (= 512) */
  u32 Flags;                              /* MIAIE_XAIE_KERNEL_FOREVER */
  XAie_MiaieLaunchFn Launch;              /* NULL for the built-in kernels below */
  void* User;
  u32 Builtin;                            /* internal id of a built-in, 0 for user kernels */
} XAie_MiaieKernel;

/* Built-in kernels: the reference examples' `__global__` functions.  A
 * harness swaps its kernel definition for e.g. `#define mm (&miaie_xaie_mm)`
 * and keeps `XAie_LoadElfMem(dev, loc, (unsigned char *)mm)`. */
MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_mm;     /* aieml_mm.cc:41-93: int32 16x16 NT, in 0x1000, out 0x6000 */
MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_mm8;    /* the same kernel built for 8x8 (MAT_SIZE 64, the "15us(8*8)" case of aieml_mm.cc:257): size_hint 128 */
MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_perf;   /* aieml_perf.cc:61-83: uint32 16x16 NT at DM 0x1000 -> 0x6000 */
MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_k1;     /* multi_tile.cpp:39-42: out[0..20) = in[0] + 1 */
MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_k2;     /* multi_tile.cpp:44-47: out[0..20) = in[0] + 10 */
MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_mm3_u64;/* vek385_verification.cpp:56-69: 3x3 A.A forever, counter at out[9] */

MIAIE_XAIE_API extern const XAie_MiaieKernel miaie_xaie_perf_u8;/* aie_nokernelload.cc:50-83: uint8 MAC probe, in[0] at 0x1000 -> 5 words at 0x6000 */

/* Iterations a FOREVER kernel runs per XAie_CoreEnable: the GPU runs a
 * bounded grid, so "until disabled" becomes this many passes, and the pass
 * counter the kernel keeps (out[9] for mm3_u64) ends at this value. */
#define MIAIE_XAIE_FOREVER_PASSES 1024u

/* Window placement of the reference compiler (src/mlir/mlirfront/
 * AieFrontEnd.cc:297-394): parameter i gets a ping buffer at its
 * mem_address annotation, else where parameter i-1's pong buffer ends
 * (0x1000 for the first); each buffer reserves 4*size_hint words (size_hint
 * defaults to 512), and the pong buffer follows the ping buffer.  Lock ids
 * are 2i (ping) and 2i+1 (pong).  Fills ping[] and pong[] (NumParams entries
 * each; either may be NULL).  Pure host computation. */
MIAIE_XAIE_API AieRC XAie_MiaieWindowLayout(const XAie_MiaieKernel* Kernel, u32* Ping, u32* Pong);

/* Run a two-window kernel on the Cols x Rows tiles from (ColStart, RowStart)
 * with DDR addresses as its arguments: the launch the reference's
 * `__kernel__` template call stands for, perf<1,1,4,4,256,16,64>(phy, phy_out)
 * (aie_nokernelload.cc:130), where phy / phy_out are XAie_MemGetDevAddr
 * values.  Each tile gets the input window from InAddr (as much as the
 * buffer holds); tile i's output (what the kernel writes) lands at
 * OutAddr + i * that size.  The addresses must lie in XAie_MemAllocate
 * buffers of one initialised instance; the tiles' cores are loaded with the
 * kernel and run once.  Returns when the output is in DDR. */
MIAIE_XAIE_API AieRC XAie_MiaieRunOnDdr(const XAie_MiaieKernel* Kernel, u32 Cols, u32 Rows, u32 ColStart, u32 RowStart,
                                        u64 InAddr, u64 OutAddr);

/* Text of the last failure on this instance ("" if none).  With a NULL or
 * uninitialised instance: the last failure of any instance on this thread. */
MIAIE_XAIE_API const char* XAie_MiaieLastError(const XAie_DevInst* DevInst);

/* Data memory bytes of a tile (0 for a shim tile, or outside the array). */
MIAIE_XAIE_API u32 XAie_MiaieTileMemBytes(const XAie_DevInst* DevInst, XAie_LocType Loc);

/* ---- partition set-up (aieml_perf.cc:265-325) --------------------------- */
/* XAie_SetupPartitionConfig(&DevInst, base, startcol, numcols) (aieml_perf.cc:276) */
MIAIE_XAIE_API AieRC XAie_SetupPartitionConfig(XAie_DevInst* DevInst, u64 PartBaseAddr, u32 StartCol, u32 NumCols);
/* XAie_CfgInitialize(&DevInst, &ConfigPtr) (aieml_perf.cc:283).  Opens GPU 0
 * (or $MIAIE_XAIE_DEVICE) and allocates the tile memories. */
MIAIE_XAIE_API AieRC XAie_CfgInitialize(XAie_DevInst* DevInst, const XAie_Config* ConfigPtr);
/* XAie_SetIOBackend(&DevInst, XAIE_IO_BACKEND_BAREMETAL) (aieml_perf.cc:286):
 * recorded; the work runs on HIP whatever is selected. */
MIAIE_XAIE_API AieRC XAie_SetIOBackend(XAie_DevInst* DevInst, XAie_BackendType Backend);
/* XAie_UpdateNpiAddr(&DevInst, 0xF6D10000) (aieml_perf.cc:295): no NPI here, accepted. */
MIAIE_XAIE_API AieRC XAie_UpdateNpiAddr(XAie_DevInst* DevInst, u64 NpiAddr);
/* XAie_PartitionInitialize(&DevInst, NULL) (aieml_perf.cc:304): zero every
 * tile memory, put every core in reset with no kernel loaded, drop routes. */
MIAIE_XAIE_API AieRC XAie_PartitionInitialize(XAie_DevInst* DevInst, void* Opts);
/* XAie_PmRequestTiles(&DevInst, NULL, 0) (aieml_perf.cc:307, AIE1 path): as PartitionInitialize. */
MIAIE_XAIE_API AieRC XAie_PmRequestTiles(XAie_DevInst* DevInst, XAie_LocType* Loc, u32 NumTiles);
/* XAie_PartitionTeardown(&DevInst) (aieml_perf.cc:321): drain, free everything. */
MIAIE_XAIE_API AieRC XAie_PartitionTeardown(XAie_DevInst* DevInst);
/* XAie_Finish(&DevInst): same as XAie_PartitionTeardown. */
MIAIE_XAIE_API AieRC XAie_Finish(XAie_DevInst* DevInst);

/* ---- cores (aieml_mm.cc:113-115, vek385_verification.cpp:78-161) -------- */
/* Status word bits of XAie_CoreGetStatus. */
#define XAIE_CORE_STATUS_ENABLE_BIT (1u << 0)
#define XAIE_CORE_STATUS_RESET_BIT (1u << 1)
#define XAIE_CORE_STATUS_DONE_BIT (1u << 20)

MIAIE_XAIE_API AieRC XAie_CoreReset(XAie_DevInst* DevInst, XAie_LocType Loc);
MIAIE_XAIE_API AieRC XAie_CoreUnreset(XAie_DevInst* DevInst, XAie_LocType Loc);
/* Bind a kernel to a core tile (aieml_mm.cc:115).  `ElfMem` must point at an
 * XAie_MiaieKernel; anything else is XAIE_INVALID_ELF. */
MIAIE_XAIE_API AieRC XAie_LoadElfMem(XAie_DevInst* DevInst, XAie_LocType Loc, const unsigned char* ElfMem);
/* Start one core on its own (vek385_verification.cpp:129).  The launch is
 * queued and issued, batched with other enabled cores, at the next call that
 * observes or moves data. */
MIAIE_XAIE_API AieRC XAie_CoreEnable(XAie_DevInst* DevInst, XAie_LocType Loc);
MIAIE_XAIE_API AieRC XAie_CoreDisable(XAie_DevInst* DevInst, XAie_LocType Loc);
/* XAIE_OK once the core's last run has finished; waits up to TimeOut
 * microseconds (0: 500 us), else XAIE_CORE_STATUS_TIMEOUT (aieml_mm.cc:172-182
 * polls this in a loop).  A core that never ran, or a FOREVER kernel still
 * enabled, is not done. */
MIAIE_XAIE_API AieRC XAie_CoreWaitForDone(XAie_DevInst* DevInst, XAie_LocType Loc, u32 TimeOut);
/* *DoneBit = 1 when the core's last run has finished (vek385_verification.cpp:78). */
MIAIE_XAIE_API AieRC XAie_CoreReadDoneBit(XAie_DevInst* DevInst, XAie_LocType Loc, u8* DoneBit);
/* Status word (seq_full_col.cpp:72): ENABLE, RESET and DONE bits.  Core
 * tiles come out of XAie_PartitionInitialize in reset, so their status is
 * non-zero; shim and memory tiles have no core and read 0. */
MIAIE_XAIE_API AieRC XAie_CoreGetStatus(XAie_DevInst* DevInst, XAie_LocType Loc, u32* CoreStatus);

/* ---- tile data memory (vek385_verification.cpp:86, :122) ---------------- */
MIAIE_XAIE_API AieRC XAie_DataMemBlockWrite(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, const void* Src, u32 Size);
MIAIE_XAIE_API AieRC XAie_DataMemBlockRead(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, void* Dst, u32 Size);
MIAIE_XAIE_API AieRC XAie_DataMemWrWord(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, u32 Data);
MIAIE_XAIE_API AieRC XAie_DataMemRdWord(XAie_DevInst* DevInst, XAie_LocType Loc, u64 Addr, u32* Data);

/* ---- DDR buffers (aieml_mm.cc:130-145, multi_tile.cpp:89-102) ----------- */
MIAIE_XAIE_API XAie_MemInst* XAie_MemAllocate(XAie_DevInst* DevInst, u64 Size, XAie_MemCacheProp Cache);
MIAIE_XAIE_API AieRC XAie_MemFree(XAie_MemInst* MemInst);
MIAIE_XAIE_API void* XAie_MemGetVAddr(XAie_MemInst* MemInst);
/* The address a harness passes to XAie_MoveData as a DDR address
 * (aieml_mm.cc:133, :149).  Equal to the virtual address. */
MIAIE_XAIE_API u64 XAie_MemGetDevAddr(XAie_MemInst* MemInst);
/* Cache maintenance of the reference's DDR; host memory here is coherent
 * with the copies, so these only validate the handle. */
MIAIE_XAIE_API AieRC XAie_MemSyncForDev(XAie_MemInst* MemInst);
MIAIE_XAIE_API AieRC XAie_MemSyncForCPU(XAie_MemInst* MemInst);

/* ---- routing and data movement (aieml_mm.cc:117-187) -------------------- */
MIAIE_XAIE_API XAie_RoutingInstance* XAie_InitRoutingHandler(XAie_DevInst* DevInst);
/* XAie_Route(ri, NULL, src, dst) (aieml_mm.cc:119): record a route.  Either
 * end may be a shim tile (DDR side) or a core/memory tile. */
MIAIE_XAIE_API AieRC XAie_Route(XAie_RoutingInstance* RoutingInstance, void* RouteConstraints, XAie_LocType Source,
                                XAie_LocType Destination);
/* XAie_MoveData(ri, src, srcAddr, size, dstAddr, dst) (aieml_mm.cc:149-151,
 * :184-186, multi_tile.cpp:125-127).  With a shim source, SrcAddr is a DDR
 * address inside an XAie_MemInst; with a shim destination, DstAddr is.
 * Otherwise both are tile data-memory addresses. */
MIAIE_XAIE_API AieRC XAie_MoveData(XAie_RoutingInstance* RoutingInstance, XAie_LocType Source, void* SrcAddr, u32 Size,
                                   void* DstAddr, XAie_LocType Destination);
/* DDR buffer -> tile memory at DstAddr (multi_tile.cpp:106-108). */
MIAIE_XAIE_API AieRC XAie_MoveDataExternal2Aie(XAie_RoutingInstance* RoutingInstance, XAie_LocType Source,
                                               XAie_MemInst* MemInst, u32 Size, u64 DstAddr,
                                               XAie_LocType Destination);
/* Tile memory at SrcAddr -> DDR buffer (multi_tile.cpp:148-150). */
MIAIE_XAIE_API AieRC XAie_MoveDataAie2External(XAie_RoutingInstance* RoutingInstance, XAie_LocType Source, u64 SrcAddr,
                                               u32 Size, XAie_MemInst* MemInst, XAie_LocType Destination);
/* Checks the route (aieml_perf.cc:163).  Moves out of a tile are complete on
 * return; a move into a tile counts as complete once its bytes are staged
 * (every later access to tile memory is ordered after the device copy), so
 * there is nothing left to wait for. */
MIAIE_XAIE_API AieRC XAie_RouteDmaWait(XAie_RoutingInstance* RoutingInstance, XAie_LocType Source,
                                       XAie_LocType Destination, u8 IsMm2s);
/* XAie_Run(ri, 1) (aieml_mm.cc:167): run every loaded, out-of-reset core on
 * the instance's routes `Iterations` times; asynchronous. */
MIAIE_XAIE_API AieRC XAie_Run(XAie_RoutingInstance* RoutingInstance, u32 Iterations);
MIAIE_XAIE_API AieRC XAie_RoutingInstanceFree(XAie_RoutingInstance* RoutingInstance);

/* ---- kernel-instance API of example/other/aieoob.c:88-95 ---------------
 * That example is written against a placeholder header (xaie_placeholder.h,
 * absent from the reference); the calls below give its flow a meaning on
 * an implicit AIE-ML partition (38 columns x 11 rows) opened on first use.
 * Window arguments are numbered from 1 among the kernel's inputs (MoveDataToAie)
 * and among its outputs (MoveAieToData). */
typedef struct XAie_Kernel_Inst XAie_Kernel_Inst;
MIAIE_XAIE_API XAie_Kernel_Inst* XAie_LoadKernel(const char* Name, int Col, int Row);
MIAIE_XAIE_API AieRC XAie_RoutingHostToAie(XAie_Kernel_Inst* Kernel, XAie_LocType Shim);
MIAIE_XAIE_API AieRC XAie_RoutingAieToHost(XAie_Kernel_Inst* Kernel, XAie_LocType Shim);
MIAIE_XAIE_API AieRC XAie_MoveDataToAie(XAie_Kernel_Inst* Kernel, int Input, const void* Src, size_t Bytes);
MIAIE_XAIE_API AieRC XAie_RunCore(XAie_Kernel_Inst* Kernel);
MIAIE_XAIE_API AieRC XAie_WaitOutData(XAie_Kernel_Inst* Kernel);
MIAIE_XAIE_API AieRC XAie_MoveAieToData(XAie_Kernel_Inst* Kernel, int Output, void* Dst, size_t Bytes);
MIAIE_XAIE_API AieRC XAie_KernelFree(XAie_Kernel_Inst* Kernel);

#ifdef __cplusplus
}
#endif

#endif /* MIAIE_XAIE_H */
