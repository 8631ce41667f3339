// gfx950 device helpers shared by the MFMA kernels: LDS DMA, explicit
// waits and barriers, LDS transpose reads, and the XCD-aware tile order.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "dbg_checks.hpp"

#define MIAIE_LDS __attribute__((address_space(3)))

typedef int miaie_v2i __attribute__((ext_vector_type(2)));
typedef short miaie_v4s __attribute__((ext_vector_type(4)));

namespace miaie {
namespace dev {

// LDS byte address of a pointer into a __shared__ array (the value M0 and
// the ds_* instructions take).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const MIAIE_LDS void*)p;
}

// 16-byte global -> LDS copy (global_load_lds_dwordx4, saddr form): lane l
// reads 16 bytes at sbase + voff and the wave's 64 x 16 bytes land
// contiguously at LDS address m0 + 16*l.  Written as inline asm so that the
// compiler's wait insertion does not treat every later LDS read as aliasing
// the copy (it would put a vmcnt(0) in front of each); callers therefore
// wait for their own copies with wait_vmcnt<N>() before the barrier that
// publishes them.  m0 must be wave-uniform.
// (In the debug build a lane whose 16 bytes lie outside `span`, the buffer
// of the copied operand, is left out of the copy and reported; line is the
// caller's.  In the product build span is empty and unused.)
__device__ __forceinline__ void gload_lds16(const void* sbase, uint32_t voff, uint32_t m0, dbg::Span span,
                                            int line = __builtin_LINE(),
                                            uint32_t file = dbg::file_id(__builtin_FILE_NAME())) {
#if MIAIE_DEVICE_CHECKS
  const void* p = static_cast<const char*>(sbase) + voff;
  if (!dbg::in_span(span, p, 16)) {
    dbg::report(p, 16, 2, line, file);
    return;
  }
#else
  (void)span;
  (void)line;
  (void)file;
#endif
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// s_waitcnt through the builtin, so that the compiler's own wait insertion
// sees it (and keeps it: waits written by the program are never dropped).
// gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14].
template <int VM, int LGKM>
__device__ __forceinline__ void waitcnt() {
  static_assert(VM >= 0 && VM <= 63 && LGKM >= 0 && LGKM <= 15, "waitcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LGKM << 8));
}
// Wait until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() { waitcnt<N, 15>(); }

// s_waitcnt vmcnt((n - 1) * CP) for a run-time 1 <= n <= N, with the count
// as the immediate it must be: the copies of all but the first of n tiles or
// stages (CP per tile) may stay in flight.
template <int CP, int N>
__device__ __forceinline__ void wait_tiles_behind(int n) {
  if constexpr (N > 1) {
    if (n == N)
      wait_vmcnt<(N - 1) * CP>();
    else
      wait_tiles_behind<CP, N - 1>(n);
  } else {
    wait_vmcnt<0>();
  }
}

// Workgroup barrier with no implied memory waits (callers wait explicitly).
// The empty asm statements keep the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Keep the scheduler from moving instructions across this point.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// ds_read_b64_tr_b8.  Within each 16-lane group, lane s supplies the address
// of 8 bytes C_s; lane i receives byte (i & 7) of C_{2j + (i >> 3)} as its
// byte j (j < 8).  So if lanes 2j and 2j+1 point at bytes [0, 8) and [8, 16)
// of row j of a row-major byte matrix, lane i receives column i of rows 0..7.
__device__ __forceinline__ miaie_v2i lds_read_tr8(const void* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((MIAIE_LDS miaie_v2i*)(p));
}

// ds_read_b64_tr_b16: the 16-bit analogue; lane i receives element (i & 3)
// of C_{4j + (i >> 2)} as its element j (j < 4), i.e. column i of four
// 16-element rows supplied by lanes 4j .. 4j+3.
__device__ __forceinline__ miaie_v4s lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((MIAIE_LDS miaie_v4s*)(p));
}

// Copy schedule of the pair-staged pipelines: A in three LDS stages of two
// k-tiles each, B in four per-k-tile stages.  In phases phi = 2t + h - 1
// (k-tile t, phase h = 1, 2), B k-tile k goes out in two halves, b_cp0
// copies at phi = 2k - 7 and b_cp1 at phi = 2k - 6; A pair p (k-tiles 2p,
// 2p+1) in quarters of qa copies at phi = 4p - 9 + q; phases before 0 belong
// to the prologue.  pair_phase_copies: copies issued in phase h of the
// k-tile d before the last (the k-tile count is even, so that k-tile is even
// exactly when d is odd); every k-tile with d >= 6 issues all of them.
constexpr int pair_phase_copies(int d, int h, int b_cp0, int b_cp1, int qa) {
  if (h == 1) return (d >= 3 ? b_cp1 : 0) + (((d & 1) ? d >= 5 : d >= 4) ? qa : 0);
  return (d >= 4 ? b_cp0 : 0) + (((d & 1) ? d >= 5 : d >= 6) ? qa : 0);
}
// Copies allowed in flight at the barrier of the k-tile d before the last:
// those of the four phases after the one that issued the next k-tile's last
// copy (B k-tile t+1 at phase 2t - 4, A pair (t+1)/2 no later).
constexpr int pair_vm(int d, int b_cp0, int b_cp1, int qa) {
  return pair_phase_copies(d + 2, 2, b_cp0, b_cp1, qa) + pair_phase_copies(d + 1, 1, b_cp0, b_cp1, qa) +
         pair_phase_copies(d + 1, 2, b_cp0, b_cp1, qa) + pair_phase_copies(d, 1, b_cp0, b_cp1, qa);
}
// Copies allowed in flight after the prologue (phases -5 .. -1), once B
// k-tile 0 and A pair 0 (issued by phase -6) have landed; valid for 6 or more
// k-tiles.
constexpr int pair_prologue_vm(int b_cp0, int b_cp1, int qa) { return 2 * (b_cp0 + b_cp1) + b_cp0 + 5 * qa; }

// MFMA order within a wave tile of NI x NJ blocks: slot x runs block
// (x / NJ, snake_j(x)), rows in order and columns serpentine (reversed on odd
// rows), so every MFMA shares one operand with the one before it (A within a
// row, B at a row turn).  Fewer operand bits toggle, and under the power
// limit the clock runs higher: register-only streams of random int8 operands
// ran 0.6% faster in this order than in plain row-major order, and 2.2%
// faster than with both operands changing every MFMA.
template <int NJ>
constexpr int snake_j(int x) {
  return ((x / NJ) & 1) ? NJ - 1 - x % NJ : x % NJ;
}

// Tile order.  Workgroups are dealt round-robin to the 8 XCDs, so workgroup
// b runs on XCD b % 8.  Give each XCD a contiguous run of logical tiles, and
// walk logical tiles in groups of GROUP_M tile-rows, column by column, so one
// XCD's run is a compact block of tiles sharing A rows and B columns in its L2.
template <int GROUP_M>
__device__ __forceinline__ void tile_coords(int b, int TM, int TN, int& tm, int& tn) {
  const int T = TM * TN;
  const int logical = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
  const int group_size = GROUP_M * TN;
  const int first_m = (logical / group_size) * GROUP_M;
  const int gm = min(TM - first_m, GROUP_M);
  tm = first_m + (logical % group_size) % gm;
  tn = (logical % group_size) / gm;
}

// First row (column) of tile t along a dimension of `extent` rows cut into
// tiles of `tile` (extent >= tile).  When the tile does not divide the
// extent, the last tile is moved back to end at the extent: it overlaps its
// neighbour, which computes the same exact sums for the shared rows, so both
// write identical bytes there and no load or store needs a bound.
__device__ __forceinline__ int tile_origin(int t, int tile, int extent) { return min(t * tile, extent - tile); }

}  // namespace dev
}  // namespace miaie
