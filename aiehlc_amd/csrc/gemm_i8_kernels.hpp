// int8 GEMM device code shared by the library (gemm_i8.hip) and the
// in-kernel clock probe (probes/gemm_span.hip): the requantize epilogues and
// the pipelined kernels gemm_i8_pipe, gemm_i8_pipe16 and
// gemm_i8_pipe16_mixed.  The kernel list, tiling and operand-role conventions
// are described at the top of gemm_i8.hip.
#pragma once

#include <type_traits>

#include "gfx950_ops.hpp"
#include "miaie_internal.hpp"

namespace miaie {
namespace gemm {

namespace dev = miaie::dev;


// ------------------------------------------------------------- epilogue
// y = sat_int8(floor((acc + 2^(s-1)) / 2^s)) for s in [1, 31], sat_int8(acc)
// for s == 0; ReLU after the shift.  floor((a + 2^(s-1)) / 2^s) equals
// (a >> s) + bit (s-1) of a, which cannot overflow.
__device__ __forceinline__ int requant1(int acc, int s, int relu) {
  int q = s ? (acc >> s) + ((acc >> (s - 1)) & 1) : acc;
  q = relu ? max(q, 0) : q;
  return min(max(q, -128), 127);
}

// The same requant in three instructions (add, arithmetic shift, med3) for
// accumulators with |acc| + 2^(s-1) < 2^31, which holds for any int8 GEMM
// with K < 2^16 (|acc| <= K * 2^14).  rnd = s ? 2^(s-1) : 0; lo = relu ? 0 : -128
// (ReLU after the shift is the same as raising the lower clamp to 0).
struct Requant {
  int s, rnd, lo, hi;  // hi == 127, kept in a register (VOP3 takes no literal)
  __device__ __forceinline__ int operator()(int acc) const {
    int r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"((acc + rnd) >> s), "s"(lo), "v"(hi));
    return r;
  }
  // four results packed little-endian into one dword (byte k = value k)
  __device__ __forceinline__ uint32_t pack4(int a0, int a1, int a2, int a3) const {
    const uint32_t lo2 = __builtin_amdgcn_perm((uint32_t)(*this)(a1), (uint32_t)(*this)(a0), 0x0c0c0400u);
    const uint32_t hi2 = __builtin_amdgcn_perm((uint32_t)(*this)(a3), (uint32_t)(*this)(a2), 0x04000c0cu);
    return lo2 | hi2;
  }
};

// The same requant for s >= 8 in 7 instructions per 4 values.  With
// u = (acc + rnd) >> (s - 8), floor division composes, so u >> 8 equals
// (acc + rnd) >> s, and the high byte of sat_int16(u) is that value clamped
// to [-128, 127]: in range it is u >> 8; above 32767 it is 127 = 32767 >> 8
// (and u >> 8 >= 128); below -32768 it is -128 (and u >> 8 <= -129).
// v_cvt_pk_i16_i32 saturates two such u into one dword, v_perm_b32 collects
// the four high bytes.  ReLU clamps the int16 pairs at 0 first.
typedef short miaie_v2s __attribute__((ext_vector_type(2)));
template <bool RELU>
struct RequantHi {
  int sh, rnd;  // sh = s - 8 (s >= 8)
  __device__ __forceinline__ uint32_t pair(int a, int b) const {
    miaie_v2s p = __builtin_amdgcn_cvt_pk_i16((a + rnd) >> sh, (b + rnd) >> sh);
    if constexpr (RELU) p = __builtin_elementwise_max(p, miaie_v2s{0, 0});
    return __builtin_bit_cast(uint32_t, p);
  }
  __device__ __forceinline__ uint32_t pack4(int a0, int a1, int a2, int a3) const {
    // bytes 1 and 3 of pair(a0, a1), then bytes 1 and 3 of pair(a2, a3)
    return __builtin_amdgcn_perm(pair(a2, a3), pair(a0, a1), 0x07050301u);
  }
};

// LDS tile rows are 64 bytes = four 16-byte chunks; chunk c of row r is
// stored at chunk c ^ swz(r).  gfx950 serves a ds_read_b128 16 lanes at a
// time from 64 four-byte banks; the MFMA fragment read has lanes 0..15 on
// 16 consecutive rows at one logical chunk, and XOR with row bits 2-3 makes
// those 16 reads cover all 64 banks (measured conflict-free with
// SQ_LDS_BANK_CONFLICT; XOR with row bits 1-2 measured 2-way conflicts).
__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 64 + ((chunk ^ swz(row)) << 4); }

// ---------------------------------------------------------- pipelined tile
// Workgroup tile BM x BN (256x256, 256x128 or 128x128), k-step 64, four LDS
// stages.  The stages are the AIE DMA ping-pong generalised to depth 4: tile
// t+4 is copied global -> LDS (global_load_lds_dwordx4, no register staging)
// while tiles t and t+1 are multiplied, half of it in each, so each copy has
// over two tiles of MFMA work to land.
// Each of the 4 waves owns a 128 x BN/2 quarter: 4 x (BN/64)
// v_mfma_i32_32x32x32_i8 per 32-wide k-step, fragments double-buffered in
// registers so the LDS reads of one k-step overlap the MFMAs of the other.
// One barrier per tile.  BN = 128 halves the work per tile, for shapes whose
// 256-wide tiles would leave CUs idle.
//
// LDS layouts (per stage):
//   A  [256 rows][64 B]: 16-byte chunk c of row r at chunk c ^ swz(r).
//   B NT [BN rows][64 B]: as A.
//   B NN [64 k-rows][BN B] (row-major, as stored in memory): 16-byte chunk
//      c of k-row k at chunk c ^ bswz(k).  MFMA fragments (16 consecutive k
//      of one column per lane) are read with two ds_read_b64_tr_b8, which
//      transpose 8x16 byte blocks on the fly; bswz spreads the 8 k-rows x 2
//      column halves one 32-lane half reads over all banks.
constexpr int BK = 64, STAGES = 4;

// NW waves (4 or 8) tile the BM x BN workgroup tile as 2 x (NW/2): each
// wave owns WM = BM/2 rows (NI = WM/32 A fragments) and WN = BN / (NW/2)
// columns (NJ = WN/32 B fragments).
template <int BM, int BN, int NW>
struct PipeGeom {
  static constexpr int THREADS = 64 * NW;
  static constexpr int WAVES_N = NW / 2;
  static constexpr int WM = BM / 2;                    // rows per wave
  static constexpr int WN = BN / WAVES_N;              // columns per wave
  static constexpr int NI = WM / 32;                   // A fragments per wave per k-step
  static constexpr int A_BYTES = BM * BK;             // 16 or 8 KiB
  static constexpr int B_BYTES = BN * BK;             // 16 or 8 KiB
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
  static constexpr int CP_BYTES = 1024 * NW;          // one 16-byte copy by every thread
  static constexpr int A_CP = A_BYTES / CP_BYTES;     // A copies per thread per tile
  static constexpr int B_CP = B_BYTES / CP_BYTES;     // B copies per thread per tile
  static constexpr int CP_PER_TILE = A_CP + B_CP;     // 16-byte LDS copies per thread per tile
  static constexpr int NJ = WN / 32;                   // B fragments per wave per k-step
  static constexpr int NMF = NI * NJ;                  // MFMAs per wave per k-step
  static_assert(NI >= 1 && NJ >= 1 && A_CP >= 1 && B_CP >= 1, "tile too small for this many waves");
  static_assert(BM * BN <= LDS_BYTES, "Y staging fits in the stages");
};

template <int BN>
__device__ __forceinline__ int bswz(int k) {
  return BN == 256 ? (k & 7) << 1 : ((k >> 1) & 3) << 1;
}

// Issue order of one k-step's LDS reads.  Reads are numbered as in
// read_one (A fragment i -> i; NT B fragment j -> NI + j; NN B fragment j ->
// NI + 2j and NI + 2j + 1, its two transposing halves), and go out in the
// order the MFMA sequence (i, j) = (x / NJ, dev::snake_j<NJ>(x)) first needs
// them: B0, A0, B1 .. B(NJ-1), A1 .. A(NI-1).  With reads issued RPS per MFMA slot
// from the start of a phase, every fragment has landed several MFMAs before
// the next phase consumes it, and the last read of a phase is far from the
// wait that precedes the tile barrier.
template <int NI, int NJ, bool B_NT>
constexpr int read_order(int n) {
  if (B_NT) {
    if (n == 0) return NI;
    if (n == 1) return 0;
    if (n <= NJ) return NI + n - 1;
    return n - NJ;
  }
  if (n < 2) return NI + n;
  if (n == 2) return 0;
  if (n <= 2 * NJ) return NI + n - 1;
  return n - 2 * NJ;
}
constexpr int RPS = 2;  // LDS reads issued per MFMA slot

// Requantized-output modes (the YQ template argument): no Y; the med3 form
// for any shift; the int16-saturation form for shifts >= 8, without and with
// ReLU.
enum YMode { Y_NONE = 0, Y_MED3 = 1, Y_HI = 2, Y_HI_RELU = 3 };

// Epilogue of the pipelined kernels.  acc[i][j][4g + t] holds row
// m = wm*WM + 32i + lane%32, column n = wn*WN + 32j + 8g + 4*(lane/32) + t of
// the BM x BN tile.  C (int32) is stored straight from the accumulators; Y is
// requantized, staged in LDS (16-byte chunk index XOR row%16, within the row's
// BN/16 chunks) and written with fully coalesced 16-byte stores.  Both stores
// are non-temporal: nothing in the kernel reads them back, and lines left
// dirty in L2 are written back when the kernel ends.  `lds` must be free (every
// LDS read and copy of the main loop completed before its last barrier) and
// hold BM * BN bytes; rnd_add is the rounding term still to be added.
template <int BM, int BN, int NW, int YQ, bool WRITE_C, int NI, int NJ>
__device__ __forceinline__ void pipe_epilogue(v16i (&acc)[NI][NJ], int8_t* lds, int tid, int wm, int wn, int fr,
                                              int fh, int m0, int n0, int8_t* __restrict__ Y,
                                              int32_t* __restrict__ C, int ldy, int ldc, int shift, int relu,
                                              int rnd_add) {
  constexpr int WM = BM / 2, WN = BN / (NW / 2), THREADS = 64 * NW;
  const dbg::Span y_span = dbg::span_of(Y), c_span = dbg::span_of(C);  // (debug build only)
  if constexpr (WRITE_C) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = m0 + wm * WM + 32 * i + fr;
          const int n = n0 + wn * WN + 32 * j + 8 * g + 4 * fh;
          v4i v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          MIAIE_ST_NT_IN(c_span, reinterpret_cast<v4i*>(C + (size_t)m * ldc + n), v);
        }
  }
  if constexpr (YQ != Y_NONE) {
    // Y leaves in NI chunks of 64 rows (row block i of both wave rows, all BN
    // columns), through two LDS buffers: chunk i is requantized into buffer
    // i % 2, then, after a barrier, written with coalesced 16-byte stores
    // while the waves go on to requantize chunk i + 1.  Every workgroup of a
    // launch reaches its epilogue at about the same time, so the stores of
    // one chunk drain while the next chunk's VALU work (accumulator reads,
    // shifts, saturating packs) runs, instead of after all of it.  Buffer
    // i % 2 is rewritten for chunk i + 2 only after the barrier of chunk
    // i + 1, which every wave reaches after its own loads of chunk i.
    constexpr int CH = BN / 16;  // 16-byte chunks per row
    constexpr int CR = 64;       // rows per chunk
    constexpr int CB = CR * BN;  // bytes per chunk buffer
    static_assert(2 * CB <= BM * BN && (CR * CH) % THREADS == 0, "two chunk buffers fit the stages");
    auto stage_rows = [&](const auto& rq, int i, int8_t* buf) {
      const int ml = 32 * wm + fr;  // row within the chunk
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = wn * WN + 32 * j + 8 * g + 4 * fh;
          const uint32_t packed = rq.pack4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                           acc[i][j][4 * g + 3]);
          const int off = ml * BN + ((((n >> 4) ^ (ml & (CH - 1)))) << 4) + (n & 15);
          *reinterpret_cast<uint32_t*>(buf + off) = packed;
        }
    };
    auto store_rows = [&](int i, const int8_t* buf) {
#pragma unroll
      for (int it = 0; it < CR * CH / THREADS; ++it) {
        const int flat = it * THREADS + tid;
        const int ml = flat / CH, c = flat % CH;
        const int m = (ml / 32) * WM + 32 * i + (ml % 32);  // row within the tile
        const v4i v = *reinterpret_cast<const v4i*>(buf + ml * BN + ((c ^ (ml & (CH - 1))) << 4));
        MIAIE_ST_NT_IN(y_span, reinterpret_cast<v4i*>(Y + (size_t)(m0 + m) * ldy + n0 + c * 16), v);
      }
    };
    auto run = [&](const auto& rq) {
      __syncthreads();  // the main loop's last LDS reads are done
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        int8_t* const buf = lds + (i & 1) * CB;
        stage_rows(rq, i, buf);
        __syncthreads();
        store_rows(i, buf);
      }
    };
    if constexpr (YQ == Y_HI_RELU)
      run(RequantHi<true>{shift - 8, rnd_add});
    else if constexpr (YQ == Y_HI)
      run(RequantHi<false>{shift - 8, rnd_add});
    else
      run(Requant{shift, rnd_add, relu ? 0 : -128, 127});
  }
}

// The last S k-tiles of an S-stage pipeline, D = KT - kt of them left when
// tile kt runs: tile kt+S-1 (whose second half this tile issues) exists for
// D == S, tile kt+1 for D >= 2, and the D - 2 whole tiles after kt+1 stay in
// flight at the wait for it.  Tile(kt, PRE, MORE, NEXT, VM) as in
// gemm_i8_pipe.
template <int D, int S, int CP, class Tile>
__device__ __forceinline__ void pipe_tail(Tile& tile, int& kt, int KT) {
  if (kt == KT - D)
    tile(kt++, std::bool_constant<D == S>{}, std::false_type{}, std::bool_constant<(D >= 2)>{},
         std::integral_constant<int, (D >= 2 ? (D - 2) * CP : 0)>{});
  if constexpr (D > 1) pipe_tail<D - 1, S, CP>(tile, kt, KT);
}

template <int BM, int BN, int NW, bool B_NT, int YQ, bool WRITE_C>
__global__ __launch_bounds__(64 * NW, 1) void gemm_i8_pipe(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int8_t* __restrict__ Y,
    int32_t* __restrict__ C, int M, int N, int K, int lda, int ldb, int ldy, int ldc, int shift,
    int relu) {
  using G = PipeGeom<BM, BN, NW>;
  constexpr int S = STAGES;
  constexpr bool WRITE_Y = YQ != Y_NONE;
  __shared__ __attribute__((aligned(1024))) int8_t lds[G::LDS_BYTES];
  const uint32_t lds0 = dev::lds_addr(lds);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tm, tn;
  dev::tile_coords<4>(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = dev::tile_origin(tm, BM, M), n0 = dev::tile_origin(tn, BN, N);
  const int KT = K / BK;

  // ---- LDS copy assignment.  Copy i of wave w fills the 1 KiB block NW*i + w
  // of an operand's stage region:
  //   A (and NT B): rows 16*(NW*i + w) + lane/4, physical chunk lane%4;
  //   NN B: k-rows (NW*i + w) * (1024 / BN) + lane / (BN / 16), physical
  //   chunk lane % (BN / 16).
  const int a_r = 16 * wave + (lane >> 2);
  const uint32_t a_voff = (uint32_t)a_r * lda + 16 * ((lane & 3) ^ swz(a_r));  // swz(a_r + 16*NW*i) == swz(a_r)
  const int8_t* const a_base = A + (size_t)m0 * lda;
  const dbg::Span a_span = dbg::span_of(A), b_span = dbg::span_of(B);  // (debug build only)
  uint32_t b_voff;
  const int8_t* b_base;
  constexpr int B_ROWS_PER_CP = B_NT ? 16 * NW : 1024 * NW / BN;  // operand rows between copies i and i+1
  if constexpr (B_NT) {
    b_voff = (uint32_t)a_r * ldb + 16 * ((lane & 3) ^ swz(a_r));
    b_base = B + (size_t)n0 * ldb;
  } else {
    constexpr int CPR = BN / 16;  // 16-byte chunks per k-row
    const int b_r = (1024 / BN) * wave + lane / CPR;  // bswz(b_r + B_ROWS_PER_CP * i) == bswz(b_r)
    b_voff = (uint32_t)b_r * ldb + 16 * ((lane % CPR) ^ bswz<BN>(b_r));
    b_base = B + n0;
  }

  // copy x (< CP_PER_TILE) of tile kt into stage `stage`
  auto copy = [&](int kt, int stage, int x) {
    const uint32_t st = lds0 + stage * G::STAGE_BYTES + 1024 * wave;
    if (x < G::A_CP) {
      dev::gload_lds16(a_base + (size_t)kt * BK + (size_t)(16 * NW * x) * lda, a_voff, st + G::CP_BYTES * x, a_span);
    } else {
      const int i = x - G::A_CP;
      const int8_t* bb = B_NT ? b_base + (size_t)kt * BK : b_base + (size_t)kt * BK * ldb;
      dev::gload_lds16(bb + (size_t)(B_ROWS_PER_CP * i) * ldb, b_voff, st + G::A_BYTES + G::CP_BYTES * i, b_span);
    }
  };

  // ---- fragment offsets within a stage.
  // A fragment (ks, i): row wm*128 + 32i + lane%32, logical chunk 2ks + lane/32.
  const int wm = wave / G::WAVES_N, wn = wave % G::WAVES_N;
  const int fr = lane & 31, fh = lane >> 5;
  int a_fo[2], b_fo[G::NJ > 2 ? G::NJ : 2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) a_fo[ks] = (wm * G::WM + fr) * 64 + (((2 * ks + fh) ^ swz(fr)) << 4);
  if constexpr (B_NT) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      b_fo[ks] = G::A_BYTES + (wn * G::WN + fr) * 64 + (((2 * ks + fh) ^ swz(fr)) << 4);
  } else {
    // tr8 read (ks, j, r): lane 16g + 2jj + h supplies k-row 32ks + 16(g>>1) + 8r + jj,
    // columns wn*WN + 32j + 16(g&1) + 8h .. +8; it receives column
    // wn*WN + 32j + lane%32, k = 32ks + 16*(lane/32) + 8r + (0..7).
    // bswz of those k-rows depends on jj only.
    const int g = lane >> 4, jj = (lane >> 1) & 7, h = lane & 1;
#pragma unroll
    for (int j = 0; j < G::NJ; ++j) {
      const int c = wn * (G::WN / 16) + 2 * j + (g & 1);
      b_fo[j] = G::A_BYTES + (16 * (g >> 1) + jj) * BN + ((c ^ bswz<BN>(jj)) << 4) + 8 * h;
    }
  }

  // One k-step's fragments: NI A fragments, and NJ B fragments (NT: one
  // ds_read_b128 each; NN: two tr8 halves each).
  struct Frags {
    v4i a[G::NI];
    v4i b[G::NJ];                  // NT
    miaie_v2i lo[G::NJ], hi[G::NJ];  // NN
  };
  constexpr int NREAD = G::NI + (B_NT ? 1 : 2) * G::NJ;  // LDS read instructions per k-step
  // q-th LDS read of k-step ks of `stage` into f
  auto read_one = [&](int stage, int ks, int q, Frags& f) {
    const int8_t* s = lds + stage * G::STAGE_BYTES;
    if (q < G::NI) {
      f.a[q] = *reinterpret_cast<const v4i*>(s + a_fo[ks] + 2048 * q);
    } else if constexpr (B_NT) {
      f.b[q - G::NI] = *reinterpret_cast<const v4i*>(s + b_fo[ks] + 2048 * (q - G::NI));
    } else {
      const int j = (q - G::NI) >> 1;
      if (((q - G::NI) & 1) == 0)
        f.lo[j] = dev::lds_read_tr8(s + b_fo[j] + ks * 32 * BN);
      else
        f.hi[j] = dev::lds_read_tr8(s + b_fo[j] + ks * 32 * BN + 8 * BN);
    }
  };
  auto bfrag = [&](const Frags& f, int j) -> v4i {
    if constexpr (B_NT)
      return f.b[j];
    else
      return v4i{f.lo[j][0], f.lo[j][1], f.hi[j][0], f.hi[j][1]};
  };

  // When only the requantized output is wanted, the accumulators start at
  // the rounding term 2^(shift-1) so the epilogue needs no add.
  const int rnd = shift ? 1 << (shift - 1) : 0;
  const int acc0 = (WRITE_Y && !WRITE_C) ? rnd : 0;
  v16i acc[G::NI][G::NJ];
#pragma unroll
  for (int i = 0; i < G::NI; ++i)
#pragma unroll
    for (int j = 0; j < G::NJ; ++j)
      acc[i][j] = v16i{acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0, acc0};

  constexpr int CP = G::CP_PER_TILE;
  // A tile's CP copies go out in two halves, each spread evenly over the
  // MFMA slots of one phase: the first CP_A in phase 2 of the tile four
  // earlier (right after the barrier that frees their stage), the other CP_B
  // in phase 1 of the tile three earlier.  Issuing a whole tile's copies in
  // one phase saturates the vector-memory path (each copy moves 1 KiB), and
  // the in-order wave then stalls its MFMAs behind them.
  constexpr int CP_A = (CP + 1) / 2, CP_B = CP - CP_A;

  // ---- prologue: tiles 0..S-2 and the first half of tile S-1 in flight
  // (tile 0's phase 1 sends the second half), wait for tile 0
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) {
#pragma unroll
      for (int x = 0; x < (s == S - 1 ? CP_A : CP); ++x) copy(s, s, x);
    }
  if (KT >= S)
    dev::wait_vmcnt<(S - 2) * CP + CP_A>();
  else  // KT < S tiles, all issued whole: the KT - 1 after tile 0 may stay in flight
    dev::wait_tiles_behind<CP, S - 1>(KT);
  dev::barrier();

  Frags f0, f1;
#pragma unroll
  for (int n = 0; n < NREAD; ++n) read_one(0, 0, read_order<G::NI, G::NJ, B_NT>(n), f0);

  // reads of slot x of a phase (RPS per slot, in read_order)
  auto read_slot = [&](int stage, int ks, int x, Frags& f) {
#pragma unroll
    for (int r = 0; r < RPS; ++r)
      if (RPS * x + r < NREAD) read_one(stage, ks, read_order<G::NI, G::NJ, B_NT>(RPS * x + r), f);
  };
  constexpr int READ_SLOTS = (NREAD + RPS - 1) / RPS;

  auto copy_slot = [&](int kt_dst, int stage, int x, int first, int count) {
#pragma unroll
    for (int c = 0; c < count; ++c)
      if ((c * G::NMF) / count == x) copy(kt_dst, stage, first + c);
  };

  // Per tile: phase 1 multiplies k-step 0 (f0) while the reads of k-step 1
  // (f1) and the second half of tile kt+S-1's copies go out between the
  // MFMAs; then the tile barrier; phase 2 multiplies k-step 1 while the first
  // half of tile kt+S's copies and the k-step-0 reads of tile kt+1 go out
  // between the MFMAs.  sched_fence() pins this interleave.
  // PRE: tile kt+S-1 exists (its first half went out in phase 2 of tile
  // kt-1, or in the prologue for tile S-1); MORE: tile kt+S exists; NEXT:
  // tile kt+1 exists; VM: copies still allowed in flight once tile kt+1 has
  // landed (those of tiles kt+2 .. kt+S-1, the last ones issued).
  auto tile = [&](int kt, auto pre_c, auto more_c, auto next_c, auto vm_c) {
    constexpr bool PRE = decltype(pre_c)::value, MORE = decltype(more_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    constexpr int VM = decltype(vm_c)::value;
    const int cur = kt & (S - 1);
    // stage of tile kt+S-1 = stage of tile kt-1, whose last reads completed
    // before tile kt-1's barrier (for kt = 0: stage S-1, not read yet)
    const int pre_stage = (kt + S - 1) & (S - 1);
#pragma unroll
    for (int x = 0; x < G::NMF; ++x) {
      const int i = x / G::NJ, j = dev::snake_j<G::NJ>(x);
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bfrag(f0, j), f0.a[i], acc[i][j], 0, 0, 0);
      read_slot(cur, 1, x, f1);
      if constexpr (PRE) copy_slot(kt + S - 1, pre_stage, x, CP_A, CP_B);
      dev::sched_fence();
    }
    if constexpr (READ_SLOTS > G::NMF) {
#pragma unroll
      for (int x = G::NMF; x < READ_SLOTS; ++x) read_slot(cur, 1, x, f1);
    }
    // Tile kt+1 must have landed (own copies, then everyone's via the
    // barrier); after the barrier no wave reads stage `cur` again, so the
    // copies of tile kt+S may overwrite it.
    dev::waitcnt<VM, 0>();
    dev::barrier();
    const int nxt = (kt + 1) & (S - 1);
#pragma unroll
    for (int x = 0; x < G::NMF; ++x) {
      const int i = x / G::NJ, j = dev::snake_j<G::NJ>(x);
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bfrag(f1, j), f1.a[i], acc[i][j], 0, 0, 0);
      if constexpr (MORE) copy_slot(kt + S, cur, x, 0, CP_A);
      if constexpr (NEXT) read_slot(nxt, 0, x, f0);
      dev::sched_fence();
    }
    if constexpr (NEXT && READ_SLOTS > G::NMF) {
#pragma unroll
      for (int x = G::NMF; x < READ_SLOTS; ++x) read_slot(nxt, 0, x, f0);
    }
  };
  using T_ = std::true_type;
  int kt = 0;
  for (; kt + S < KT; ++kt) tile(kt, T_{}, T_{}, T_{}, std::integral_constant<int, (S - 2) * CP>{});
  pipe_tail<S, S, CP>(tile, kt, KT);

  pipe_epilogue<BM, BN, NW, YQ, WRITE_C>(acc, lds, tid, wm, wn, fr, fh, m0, n0, Y, C, ldy, ldc, shift, relu,
                                        rnd - acc0);
}

// ------------------------------------------------------ pair-staged tiles
// The pipeline of gemm_i8_pipe with A staged two k-tiles at a time.  A row-major A tile
// row contributes 64 bytes per k-tile, so a per-k-tile copy touches every
// 128-byte line at half use; the L1 fetches whole lines, the address path
// handles 16 lines per 1 KiB copy, and the A stream costs twice its bytes on
// the L2 -> L1 path.  Here A lives in NA2 = 3 pair stages of BM rows x 128
// bytes (k-tiles 2p and 2p+1 of pair p in stage p % 3) and each 1 KiB copy
// moves 8 whole lines; B keeps its four per-k-tile stages.  Needs K % 128 == 0.
//
// Copy schedule, in phases phi = 2t + (h - 1) (tile t, phase h = 1, 2):
//   B tile k: first half at phi = 2k - 7 (phase 2 of tile k-4, after the
//     barrier that retires tile k-4's reads of its stage), second half at
//     phi = 2k - 6 (phase 1 of tile k-3);
//   A pair p: quarter q at phi = 4p - 9 + q (phase 2 of tile 2p-5, after the
//     barrier that retires pair p-3's reads of its stage, through phase 1 of
//     tile 2p-3).
// Copies with phi < 0 go out in the prologue, in phi order.  Tile t's data
// (B tile t, A pair t/2) was issued by phase 2t - 6, so the barrier of tile
// t-1 (end of phase 2t - 2) waits until at most the copies of the four phases
// after it are in flight: 2 * (copies per tile) in steady state, fewer in the
// last tiles (dev::pair_vm).
constexpr int NA2 = 3;

// Stages and copy geometry of the pair-staged pipeline (NW waves).
template <int BM, int BN, int NW>
struct PairGeom {
  static constexpr int A2_BYTES = BM * 128;                 // one A pair stage
  static constexpr int A_REGION = NA2 * A2_BYTES;
  static constexpr int B_BYTES = BN * BK;                   // one B stage
  static constexpr int LDS_BYTES = A_REGION + STAGES * B_BYTES;
  static constexpr int CP_BYTES = 1024 * NW;                // one 16-byte copy by every thread
  static constexpr int A_CP2 = A2_BYTES / CP_BYTES;         // A copies per thread per pair
  static constexpr int QA = A_CP2 / 4;                      // ... per quarter (per phase)
  static constexpr int B_CP = B_BYTES / CP_BYTES;           // B copies per thread per k-tile
  static constexpr int B_CP0 = (B_CP + 1) / 2, B_CP1 = B_CP - B_CP0;
  static_assert(B_CP >= 1 && A_CP2 % 4 == 0 && QA >= 1, "pair-staged geometry");
  static_assert(LDS_BYTES <= 163840 && BM * BN <= LDS_BYTES, "pair-staged LDS budget");
};

// Clock probe records per wave (TIMED instantiations only): shader clock at
// the start, after the prologue's barrier, after the last k-tile and at the
// end, then the 100 MHz wall clock at the start and the end.
constexpr int PROBE_WORDS = 6;

// ---------------------------------------- pair-staged tile on 16x16x64 MFMA
// One BM x BN output tile (256 x 256 or 256 x 128; 4 waves of BM/2 x BN/2)
// of the pair-staged pipeline above, multiplied on v_mfma_i32_16x16x64_i8.
// v_mfma_i32_32x32x32_i8 does the same MACs per cycle, but the 16x16 form
// reads and writes half as many accumulator bits per MAC, and these boxes run
// power-limited: register-only streams of random int8 operands sustained
// 3.8 POP/s at a 1.9 GHz shader clock on the 16x16 form against 3.3 POP/s at
// 1.65 GHz on the 32x32 form, same GPU, same run (probes/mfma_ceiling).
//
// Copies (global_load_lds_dwordx4, 1 KiB per wave): A copy x of wave w fills
// the 1 KiB block NW*x + w of a pair stage, rows 8(NW*x + w) + lane/8,
// physical chunk lane%8 of the row's 128 bytes, holding logical chunk
// (lane%8) ^ ((row >> 1) & 7); B copies as in gemm_i8_pipe, with the NN
// swizzle bswz16 below.
//
// A wave's WM x WN quarter is NI x NJ blocks of 16 x 16 (NI = WM/16, NJ =
// WN/16), and one 64-wide k-tile is one k-step.  Block (i, j) of k-tile t is
// multiplied in phase 1 of tile t for i < NI/2 and in phase 2 for i >= NI/2,
// column-block-major (j outer, i inner, i reversed on odd j, so consecutive
// MFMAs always share an operand: 1.2% faster at 4096^3 under the power
// limit than restarting i at every column block) in both phases:
//   phase 1: A fragments 0 .. NI/2-1 (alo) and the B fragments, while A
//            fragments NI/2 .. NI-1 of tile t (ahi) are read;
//   barrier (tile t+1 landed);
//   phase 2: ahi and the B fragments, while alo and the B fragments of tile
//            t+1 are read, B fragment j right after the last MFMA that uses
//            tile t's B fragment j, into the same registers.
// One set of A and B fragment registers then suffices (64 VGPRs), which
// keeps the 256 accumulators in the AGPRs.  Tile t's fragments are read
// between phase 2 of tile t-1 and phase 1 of tile t, and the copy schedule
// above overwrites a stage only after the barrier that follows its last read.
//
// Fragments: lane l holds, for A fragment i, row 16i + l%16 of the wave's
// rows, k = 16(l/16) .. +16 (logical 16-byte chunk l/16 of the k-tile); for B
// fragment j, column 16j + l%16, the same k.  The accumulator of block (i, j)
// (srcA = B fragment, srcB = A fragment) holds in lane l row 16i + l%16,
// columns 16j + 4(l/16) + 0..3.  NN B fragments are two ds_read_b64_tr_b8
// halves (k 16(l/16) + 0..7 and + 8..15); a 32-lane read then spans k-rows
// r and r + 16, so the B stage swizzle also XORs k-row bit 4 into the chunk
// index (bswz16), which keeps those reads conflict-free.
template <int BN>
__device__ __forceinline__ int bswz16(int k) {
  return bswz<BN>(k) | ((k >> 4) & 1);
}

// acc += srcA x srcB in place.  The compiler's own form of this instruction
// writes a result register set distinct from the accumulator's, and with all
// 256 AGPRs holding a 128x128 wave tile it then shuttles accumulators through
// VGPRs (hundreds of extra moves per k-tile, and spills); written out, the
// accumulator is updated in place.  Operands come straight from LDS reads
// (the compiler's lgkmcnt waits see the asm's register uses); the end of the
// main loop waits out the last MFMAs' latency before any accumulator is read
// (mfma16_drain).
__device__ __forceinline__ void mfma16(v4i& acc, v4i a, v4i b) {
#if MIAIE_DEVICE_CHECKS
  // debug build: the checks' extra registers let the compiler move
  // accumulators inside the loop, so it gets its own MFMA, whose hazards it
  // tracks (slower, same sums)
  acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
#else
  asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
#endif
}
// 8-pass MFMA results are readable by VALU after 11 wait states (gfx950);
// 24 here, with nothing scheduled across.
__device__ __forceinline__ void mfma16_drain() {
  dev::sched_fence();
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  dev::sched_fence();
}

template <int BM, int BN, int NW>
struct Pipe16Geom {
  using G2 = PairGeom<BM, BN, NW>;  // stages and copy geometry
  static constexpr int WAVES_N = NW / 2;
  static constexpr int WM = BM / 2, WN = BN / WAVES_N;
  static constexpr int NI = WM / 16, NJ = WN / 16, HI = NI / 2;
  static constexpr int PH = HI * NJ;  // MFMAs per phase
  static_assert(NI % 2 == 0 && NJ >= 1 && HI * 16 * 2 == WM, "16x16 blocks per wave");
};

// KEEP_Y: Y written with ordinary stores, which leave it in the caches for
// a kernel that reads it next (the MLP's H); otherwise non-temporal.
template <int BM, int BN, int NW, bool B_NT, int YQ, bool WRITE_C, bool TIMED, bool KEEP_Y = false>
__device__ __forceinline__ void pipe16_tile(int8_t* lds, int m0, int n0, const int8_t* __restrict__ A,
                                            const int8_t* __restrict__ B, int8_t* __restrict__ Y,
                                            int32_t* __restrict__ C, int K, int lda, int ldb, int ldy, int ldc,
                                            int shift, int relu, unsigned long long* __restrict__ probe,
                                            unsigned long long t0, unsigned long long r0) {
  unsigned long long t1 = 0, t2 = 0;
  using G = typename Pipe16Geom<BM, BN, NW>::G2;
  using H = Pipe16Geom<BM, BN, NW>;
  constexpr int NI = H::NI, NJ = H::NJ, HI = H::HI, PH = H::PH;
  constexpr bool WRITE_Y = YQ != Y_NONE;
  // LDS: the four B stages first, then the three A pair stages.  A B
  // fragment read is then its lane's base address plus a compile-time offset
  // below 2^16 (the ds_read offset field) wherever the stage is known.
  constexpr int B_REGION = STAGES * G::B_BYTES;
  constexpr int B_MASK = B_REGION - 1;
  static_assert(B_REGION + G::A_REGION == G::LDS_BYTES && (B_REGION & B_MASK) == 0, "B stages first");
  const uint32_t lds0 = dev::lds_addr(lds);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int KT = K / BK;  // even

  // ---- copies.  A copy is one global_load_lds_dwordx4 from a wave-uniform
  // source pointer (per operand and k-tile) plus a per-lane offset; NN B
  // copies whose k-rows differ in bit 4 differ in bswz16.
  const int a_r = 8 * wave + (lane >> 3);
  const uint32_t a_voff = (uint32_t)a_r * lda + 16 * ((lane & 7) ^ ((a_r >> 1) & 7));
  constexpr int B_ROWS_PER_CP = B_NT ? 16 * NW : 1024 * NW / BN;
  uint32_t b_voff[2];
  if constexpr (B_NT) {
    const int b_r = 16 * wave + (lane >> 2);
    b_voff[0] = b_voff[1] = (uint32_t)b_r * ldb + 16 * ((lane & 3) ^ swz(b_r));
  } else {
    static_assert(B_ROWS_PER_CP == 16 || B_ROWS_PER_CP % 32 == 0, "k-row bit 4 per NN B copy");
    constexpr int CPR = BN / 16;
    const int b_r = (1024 / BN) * wave + lane / CPR;
#pragma unroll
    for (int e = 0; e < 2; ++e)
      b_voff[e] = (uint32_t)b_r * ldb + 16 * ((lane % CPR) ^ bswz16<BN>(b_r + (B_ROWS_PER_CP == 16 ? 16 * e : 0)));
  }
  const int8_t* const a_base = A + (size_t)m0 * lda;
  const int8_t* const b_base = B_NT ? B + (size_t)n0 * ldb : B + n0;
  const dbg::Span a_span = dbg::span_of(A), b_span = dbg::span_of(B);  // (debug build only)
  const size_t b_kstep = B_NT ? (size_t)BK : (size_t)BK * ldb;  // B source per k-tile
  const uint32_t ldsw = lds0 + 1024 * wave;
  // copy x of an A pair (source src) into the pair stage at byte st of the A region
  auto copy_a = [&](const int8_t* src, uint32_t st, int x) __attribute__((always_inline)) {
    dev::gload_lds16(src + (size_t)(8 * NW * x) * lda, a_voff, ldsw + B_REGION + st + G::CP_BYTES * x, a_span);
  };
  // copy x of a B k-tile (source src) into the B stage at byte st
  auto copy_b = [&](const int8_t* src, uint32_t st, int x) __attribute__((always_inline)) {
    dev::gload_lds16(src + (size_t)(B_ROWS_PER_CP * x) * ldb, b_voff[B_ROWS_PER_CP == 16 ? (x & 1) : 0],
                     ldsw + st + G::CP_BYTES * x, b_span);
  };

  // ---- fragments.  A fragment i of k-tile 2p + par: row wm*WM + 16i +
  // lane%16 of pair stage p % 3, logical chunk 4par + lane/16, physical chunk
  // XOR (row >> 1) & 7 = (lane%16 >> 1) & 7.
  const int wm = wave / H::WAVES_N, wn = wave % H::WAVES_N;
  const int fr = lane & 15, fg = lane >> 4;
  int a_fo[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) a_fo[par] = (wm * H::WM + fr) * 128 + (((4 * par + fg) ^ ((fr >> 1) & 7)) << 4);
  int b_fo[B_NT ? 1 : NJ];
  if constexpr (B_NT) {
    b_fo[0] = (wn * H::WN + fr) * 64 + ((fg ^ swz(fr)) << 4);
  } else {
    // tr8 half r of fragment j: lane 16g + 2jj + h supplies k-row 16g + 8r +
    // jj, columns wn*WN + 16j + 8h .. +8; lane 16g + c receives column
    // wn*WN + 16j + c, k = 16g + 8r + (0..7).  bswz16 of those k-rows depends
    // on jj and g only.
    const int jj = (lane >> 1) & 7, h = lane & 1;
    const int kr = 16 * fg + jj;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = wn * (H::WN / 16) + j;
      b_fo[j] = kr * BN + ((c ^ bswz16<BN>(kr)) << 4) + 8 * h;
    }
  }

  struct BFrags {
    v4i b[NJ];
    miaie_v2i lo[NJ], hi[NJ];
  };
  v4i alo[HI], ahi[HI];
  BFrags bs;
  // A fragment i (parity par) from the pair stage at byte st of the A region
  auto read_a = [&](uint32_t st, int par, int i) __attribute__((always_inline)) -> v4i {
    // (the stage's byte address goes through readfirstlane so that the
    // compiler keeps it in the base register: only 2048 i, below 2^16, is
    // left for the instruction's offset field)
    const uint32_t sbase = __builtin_amdgcn_readfirstlane(B_REGION + st);
    return *reinterpret_cast<const v4i*>(lds + sbase + a_fo[par] + 2048 * i);
  };
  constexpr int BPF = B_NT ? 1 : 2;  // B reads per fragment
  // read r of B fragment j from the B stage at byte st
  auto read_b = [&](int st, int j, int r) __attribute__((always_inline)) {
    if constexpr (B_NT) {
      bs.b[j] = *reinterpret_cast<const v4i*>(lds + st + b_fo[0] + 1024 * j);
    } else if (r == 0) {
      bs.lo[j] = dev::lds_read_tr8(lds + st + b_fo[j]);
    } else {
      bs.hi[j] = dev::lds_read_tr8(lds + st + b_fo[j] + 8 * BN);
    }
  };
  auto bfrag = [&](int j) __attribute__((always_inline)) -> v4i {
    if constexpr (B_NT)
      return bs.b[j];
    else
      return v4i{bs.lo[j][0], bs.lo[j][1], bs.hi[j][0], bs.hi[j][1]};
  };

  const int rnd = shift ? 1 << (shift - 1) : 0;
  const int acc0 = (WRITE_Y && !WRITE_C) ? rnd : 0;
  v4i acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = v4i{acc0, acc0, acc0, acc0};

  // ---- prologue: the copies of phases -9 .. -1 in phase order
  const int KP = KT / 2;
#pragma unroll
  for (int phi = -9; phi < 0; ++phi) {
    if ((phi & 1) != 0) {
      const int k = (phi + 7) / 2;
      if (phi >= -7 && k < KT)
#pragma unroll
        for (int x = 0; x < G::B_CP0; ++x) copy_b(b_base + k * b_kstep, k * G::B_BYTES, x);
    } else {
      const int k = (phi + 6) / 2;
      if (phi >= -6 && k < KT)
#pragma unroll
        for (int x = G::B_CP0; x < G::B_CP; ++x) copy_b(b_base + k * b_kstep, k * G::B_BYTES, x);
    }
    const int p = (phi + 9) / 4, q = (phi + 9) % 4;
    if (p < KP)
#pragma unroll
      for (int x = 0; x < G::QA; ++x) copy_a(a_base + p * 128, p * G::A2_BYTES, G::QA * q + x);
  }
  if (KT >= 6)
    dev::wait_vmcnt<dev::pair_prologue_vm(G::B_CP0, G::B_CP1, G::QA)>();
  else
    dev::wait_vmcnt<0>();
  dev::barrier();
  if constexpr (TIMED) t1 = __builtin_amdgcn_s_memtime();

#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < BPF; ++r) read_b(0, j, r);
#pragma unroll
  for (int i = 0; i < HI; ++i) alo[i] = read_a(0, 0, i);

  // ---- per-tile state (wave-uniform), for tile t of pair P = t / 2:
  uint32_t sa0 = 0, sa1 = G::A2_BYTES, sa2 = 2 * G::A2_BYTES;  // stages of pairs P, P+1, P+2
  const int8_t* a_src = a_base + 2 * 128;                       // A source of pair P+2
  const int8_t* b_src = b_base + 3 * b_kstep;                   // B source of k-tile t+3
  int sb_rt = 0;                                                // B stage of tile t

  // Tile t (parity PAR; D tiles before the last; SB = t % 4, or -1 where only
  // known at run time), copies in the schedule above: phase 1 sends the
  // second half of B k-tile t+3 and a quarter of A pair P+2; phase 2 the first
  // half of B k-tile t+4 (into tile t's stage) and a quarter of A pair P+2 (t
  // even) or P+3 (t odd, into pair P's stage).
  auto tile = [&](auto par_c, auto d_c, auto sb_c) __attribute__((always_inline)) {
    constexpr int PAR = decltype(par_c)::value, D = decltype(d_c)::value, SB = decltype(sb_c)::value;
    constexpr int NB1 = D >= 3 ? G::B_CP1 : 0, NB2 = D >= 4 ? G::B_CP0 : 0;
    constexpr int NA1 = (PAR == 0 ? D >= 5 : D >= 4) ? G::QA : 0;
    constexpr int NA2_ = (PAR == 0 ? D >= 5 : D >= 6) ? G::QA : 0;
    constexpr bool NEXT = D >= 1;
    constexpr int VM = dev::pair_vm(D, G::B_CP0, G::B_CP1, G::QA);
    const int sbc = SB >= 0 ? SB * G::B_BYTES : sb_rt;                                   // tile t
    const int sb1 = SB >= 0 ? ((SB + 1) & 3) * G::B_BYTES : (sb_rt + G::B_BYTES) & B_MASK;  // tile t+1
    const int sb3 = SB >= 0 ? ((SB + 3) & 3) * G::B_BYTES : (sb_rt + 3 * G::B_BYTES) & B_MASK;  // tile t+3
    constexpr int qa1 = PAR == 0 ? 1 : 3;
#pragma unroll
    for (int x = 0; x < PH; ++x) {
      const int j = x / HI, i = dev::snake_j<HI>(x);
      mfma16(acc[i][j], bfrag(j), alo[i]);
      if (x < HI) ahi[x] = read_a(sa0, PAR, HI + x);
#pragma unroll
      for (int c = 0; c < NB1 + NA1; ++c)
        if ((c * PH) / (NB1 + NA1 > 0 ? NB1 + NA1 : 1) == x) {
          if (c < NB1)
            copy_b(b_src, sb3, G::B_CP0 + c);
          else
            copy_a(a_src, sa2, G::QA * qa1 + c - NB1);
        }
      dev::sched_fence();
    }
    // tile t+1 has landed (own copies, then everyone's via the barrier);
    // after the barrier no wave reads tile t's B stage or, for t odd, pair
    // P's stage again
    dev::waitcnt<VM, 0>();
    dev::barrier();
    constexpr int qa2 = PAR == 0 ? 2 : 0;
    const int8_t* const a_src2 = PAR == 0 ? a_src : a_src + 128;
    const uint32_t sa_cp2 = PAR == 0 ? sa2 : sa0;
    const uint32_t sa_next = PAR == 0 ? sa0 : sa1;  // pair of tile t+1
#pragma unroll
    for (int x = 0; x < PH; ++x) {
      const int j = x / HI, i = dev::snake_j<HI>(x);
      mfma16(acc[HI + i][j], bfrag(j), ahi[i]);
#pragma unroll
      for (int c = 0; c < NB2 + NA2_; ++c)
        if ((c * PH) / (NB2 + NA2_ > 0 ? NB2 + NA2_ : 1) == x) {
          if (c < NB2)
            copy_b(b_src + b_kstep, sbc, c);
          else
            copy_a(a_src2, sa_cp2, G::QA * qa2 + c - NB2);
        }
      if constexpr (NEXT) {
        if (x < HI) alo[x] = read_a(sa_next, 1 - PAR, x);
        if (x % HI == HI - 1) {  // last use of tile t's B fragment j
#pragma unroll
          for (int r = 0; r < BPF; ++r) read_b(sb1, j, r);
        }
      }
      dev::sched_fence();
    }
    b_src += b_kstep;
    sb_rt = (sb_rt + G::B_BYTES) & B_MASK;
    if constexpr (PAR == 1) {
      const uint32_t s = sa0;
      sa0 = sa1;
      sa1 = sa2;
      sa2 = s;
      a_src += 128;
    }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using DS = std::integral_constant<int, 64>;  // steady state
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using SR = std::integral_constant<int, -1>;
  // steady tiles 0 .. KT-7, then the last six.  (With the steady loops
  // inside the KT >= 6 branch instead, the register allocator moves the
  // accumulators between AGPRs and VGPRs around them.)
  int t = 0;
  for (; t + 10 <= KT; t += 4) {  // four at a time: B stages known at compile time
    tile(P0{}, DS{}, S0{});
    tile(P1{}, DS{}, S1{});
    tile(P0{}, DS{}, S2{});
    tile(P1{}, DS{}, S3{});
  }
  for (; t + 6 < KT; t += 2) {
    tile(P0{}, DS{}, SR{});
    tile(P1{}, DS{}, SR{});
  }
  if (KT >= 6) {
    tile(P0{}, std::integral_constant<int, 5>{}, SR{});
    tile(P1{}, std::integral_constant<int, 4>{}, SR{});
  }
  if (KT >= 4) {
    tile(P0{}, std::integral_constant<int, 3>{}, SR{});
    tile(P1{}, std::integral_constant<int, 2>{}, SR{});
  }
  tile(P0{}, std::integral_constant<int, 1>{}, SR{});
  tile(P1{}, std::integral_constant<int, 0>{}, SR{});
  mfma16_drain();
  if constexpr (TIMED) t2 = __builtin_amdgcn_s_memtime();

  // ---- epilogue.  acc[i][j][e]: row wm*WM + 16i + lane%16, column
  // wn*WN + 16j + 4(lane/16) + e.
  constexpr int WM = H::WM, WN = H::WN, THREADS = 64 * NW;
  const dbg::Span y_span = dbg::span_of(Y), c_span = dbg::span_of(C);  // (debug build only)
  const int rnd_add = rnd - acc0;
  if constexpr (WRITE_C) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int m = m0 + wm * WM + 16 * i + fr;
        const int n = n0 + wn * WN + 16 * j + 4 * fg;
        MIAIE_ST_NT_IN(c_span, reinterpret_cast<v4i*>(C + (size_t)m * ldc + n), acc[i][j]);
      }
  }
  if constexpr (WRITE_Y) {
    // Y leaves in NI/2 chunks of 64 rows (blocks 2c and 2c+1 of both wave
    // rows, all BN columns) through two LDS buffers, as in pipe_epilogue.
    constexpr int CH = BN / 16, CR = 64, CB = CR * BN;
    static_assert(2 * CB <= BM * BN && (CR * CH) % THREADS == 0, "two chunk buffers fit the stages");
    auto stage_rows = [&](const auto& rq, int c, int8_t* buf) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = 2 * c + u;
        const int ml = 32 * wm + 16 * u + fr;  // row within the chunk
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int n = wn * WN + 16 * j + 4 * fg;
          const uint32_t packed = rq.pack4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
          const int off = ml * BN + (((n >> 4) ^ (ml & (CH - 1))) << 4) + (n & 15);
          *reinterpret_cast<uint32_t*>(buf + off) = packed;
        }
      }
    };
    auto store_rows = [&](int c, const int8_t* buf) {
#pragma unroll
      for (int it = 0; it < CR * CH / THREADS; ++it) {
        const int flat = it * THREADS + tid;
        const int ml = flat / CH, ch = flat % CH;
        const int m = (ml / 32) * WM + 32 * c + (ml % 32);  // row within the tile
        const v4i v = *reinterpret_cast<const v4i*>(buf + ml * BN + ((ch ^ (ml & (CH - 1))) << 4));
        v4i* const dst = reinterpret_cast<v4i*>(Y + (size_t)(m0 + m) * ldy + n0 + ch * 16);
        if constexpr (KEEP_Y)
          MIAIE_ST_IN(y_span, dst, v);
        else
          MIAIE_ST_NT_IN(y_span, dst, v);
      }
    };
    auto run = [&](const auto& rq) {
      __syncthreads();  // the main loop's last LDS reads are done
#pragma unroll
      for (int c = 0; c < NI / 2; ++c) {
        int8_t* const buf = lds + (c & 1) * CB;
        stage_rows(rq, c, buf);
        __syncthreads();
        store_rows(c, buf);
      }
    };
    if constexpr (YQ == Y_HI_RELU)
      run(RequantHi<true>{shift - 8, rnd_add});
    else if constexpr (YQ == Y_HI)
      run(RequantHi<false>{shift - 8, rnd_add});
    else
      run(Requant{shift, rnd_add, relu ? 0 : -128, 127});
  }
  if constexpr (TIMED) {
    const unsigned long long t3 = __builtin_amdgcn_s_memtime(), r3 = __builtin_amdgcn_s_memrealtime();
    const unsigned long long rec[PROBE_WORDS] = {t0, t1, t2, t3, r0, r3};
    unsigned long long v = 0;
#pragma unroll
    for (int i = 0; i < PROBE_WORDS; ++i) v = lane == i ? rec[i] : v;
    if (lane < PROBE_WORDS) probe[((size_t)blockIdx.x * NW + wave) * PROBE_WORDS + lane] = v;
  }
}

template <int BM, int BN, int NW, bool B_NT, int YQ, bool WRITE_C, bool TIMED = false, bool KEEP_Y = false>
__global__ __launch_bounds__(64 * NW, 1) void gemm_i8_pipe16(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int8_t* __restrict__ Y,
    int32_t* __restrict__ C, int M, int N, int K, int lda, int ldb, int ldy, int ldc, int shift,
    int relu, unsigned long long* __restrict__ probe) {
  unsigned long long t0 = 0, r0 = 0;
  if constexpr (TIMED) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  __shared__ __attribute__((aligned(1024))) int8_t lds[PairGeom<BM, BN, NW>::LDS_BYTES];
  int tm, tn;
  dev::tile_coords<4>(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  pipe16_tile<BM, BN, NW, B_NT, YQ, WRITE_C, TIMED, KEEP_Y>(lds, dev::tile_origin(tm, BM, M),
                                                             dev::tile_origin(tn, BN, N), A, B, Y, C, K, lda, ldb,
                                                             ldy, ldc, shift, relu, probe, t0, r0);
}

// Mixed tile widths in one launch: the first ceil(M/256) * nw workgroups
// take the 256 x 256 tiles of output columns [0, 256 nw), the rest the
// 256 x 128 tiles of columns [256 nw, N) (N - 256 nw >= 128; the last tile
// row and the last narrow column are moved back as dev::tile_origin says).  Workgroups are dispatched in order, so the
// narrow tiles fill the CUs the wide ones leave idle and then the CUs they
// free.  For shapes whose 256-wide tiles would leave most of a round empty
// (the MLP's 2048 x 11008 up-projection: 344 wide tiles on 256 CUs, or 688
// narrow ones, 2.7 rounds) the planner picks the split (plan_pipe).
template <bool B_NT, int YQ, bool WRITE_C, bool KEEP_Y = false>
__global__ __launch_bounds__(256, 1) void gemm_i8_pipe16_mixed(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int8_t* __restrict__ Y,
    int32_t* __restrict__ C, int M, int N, int K, int lda, int ldb, int ldy, int ldc, int shift,
    int relu, int nw) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[PairGeom<256, 256, 4>::LDS_BYTES];
  const int TM = (M + 255) / 256, nwide = TM * nw;
  const int b = blockIdx.x;
  int tm, tn;
  if (b < nwide) {
    dev::tile_coords<4>(b, TM, nw, tm, tn);
    pipe16_tile<256, 256, 4, B_NT, YQ, WRITE_C, false, KEEP_Y>(lds, dev::tile_origin(tm, 256, M), 256 * tn, A, B, Y,
                                                                C, K, lda, ldb, ldy, ldc, shift, relu, nullptr, 0, 0);
  } else {
    const int nn = N - 256 * nw;  // columns of the narrow tiles (>= 128)
    dev::tile_coords<4>(b - nwide, TM, (nn + 127) / 128, tm, tn);
    const size_t c0 = (size_t)256 * nw;  // first column of the narrow tiles
    pipe16_tile<256, 128, 4, B_NT, YQ, WRITE_C, false, KEEP_Y>(
        lds, dev::tile_origin(tm, 256, M), dev::tile_origin(tn, 128, nn), A, B_NT ? B + c0 * ldb : B + c0,
        Y ? Y + c0 : nullptr, C ? C + c0 : nullptr, K, lda, ldb, ldy, ldc, shift, relu, nullptr, 0, 0);
  }
}

}  // namespace gemm
}  // namespace miaie
