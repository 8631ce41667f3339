// bf16 x bf16 -> fp32 GEMM on gfx950 MFMA (v_mfma_f32_16x16x32_bf16 and
// v_mfma_f32_32x32x16_bf16).
//
// The benchmark's bf16 -> fp32 path; the reference has no bf16 kernel (its
// only float check is the elementwise square of example/other/
// aieml_apu.cc:149-156 with an absolute tolerance of 1e-2 at :190).
//
// Same geometry as the int8 kernel: a row of an LDS tile is 64 bytes
// (32 bf16 of k), read as 16-byte MFMA fragments with the same XOR swizzle;
// the row-major B operand is transposed by ds_read_b64_tr_b16 on its way out
// of LDS.
// M and N need not be multiples of 256 (the launcher's conditions): the last
// tile row and column are moved back to end at M and N.
//   gemm_bf16_pair16   256x256, K % 64 == 0: A staged two k-tiles at a time,
//                      v_mfma_f32_16x16x32_bf16 (a higher clock than the
//                      32x32x16 form under the power limit).
//   gemm_bf16_tile256  256x256x32, 4 waves x (4x4 MFMA 32x32x16), four LDS stages.
//   gemm_bf16_tile64p  64x64x32 fallback for K % 8 == 0 and an aligned A:
//                      vector A loads, next k-tile prefetched into registers.
//   gemm_bf16_tile64   64x64x32 bounds-checked fallback.
// The 256x256 kernels write C through whole-row stores staged in LDS.
#include <type_traits>

#include "gfx950_ops.hpp"
#include "miaie_internal.hpp"

namespace {

namespace dev = miaie::dev;
namespace dbg = miaie::dbg;

// 64-byte LDS rows: chunk c of row r at chunk c ^ swz(r).  gfx950 serves a
// ds_read_b128 16 lanes at a time from 64 four-byte banks; XOR with row
// bits 2-3 puts the 16 rows one fragment read touches on distinct banks.
__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 64 + ((chunk ^ swz(row)) << 4); }

__device__ __forceinline__ v8bf as_bf(v4i x) { return __builtin_bit_cast(v8bf, x); }

// fp32 epilogue of a 256x256 tile held as acc[i][j][4g + t] = C[m0 + wm*128
// + 32i + lane%32][n0 + wn*128 + 32j + 8g + 4*(lane/32) + t], staged through
// 128 KiB of LDS in two halves so that every store instruction writes one
// whole 1 KiB row (eight full 128-byte lines).  Direct stores from the
// accumulators write 32 bytes per row per instruction; with every workgroup
// of a round storing at once, that burst cost 5% of the 8192^3 GEMM, this one
// half of that.  Half h holds each wave's row blocks i = 2h, 2h+1: LDS row
// R = wm*64 + 32(i - 2h) + lane%32 (tile row wm*128 + 64h + R%64), logical
// 16-byte chunk c at physical chunk c ^ (R & 15), so both the column writes
// (16 rows, one chunk) and the row reads (one row, 16 chunks) touch 16
// distinct bank groups.  Stores are non-temporal: nothing reads C back.
__device__ __forceinline__ void store_tile_f32(const v16f (&acc)[4][4], int8_t* lds, int wave, int lane, float* C,
                                               int m0, int n0, int N) {
  const int wm = wave >> 1, wn = wave & 1, fr = lane & 31, fh = lane >> 5;
  const dbg::Span c_span = dbg::span_of(C);  // (debug build only)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    dev::barrier();  // the other waves' last reads of this LDS (k-loop fragments or the previous half)
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const v16f& a = acc[2 * h + ii][j];
          const int R = wm * 64 + 32 * ii + fr;
          const int c = wn * 32 + 8 * j + 2 * g + fh;
          const v4f v = {a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
          *reinterpret_cast<v4f*>(lds + R * 1024 + ((c ^ (R & 15)) << 4)) = v;
        }
    dev::barrier();
#pragma unroll
    for (int rr = 0; rr < 32; ++rr) {
      const int R = wave * 32 + rr;
      const v4f v = *reinterpret_cast<const v4f*>(lds + R * 1024 + ((lane ^ (R & 15)) << 4));
      const int m = m0 + (R >> 6) * 128 + 64 * h + (R & 63);
      MIAIE_ST_NT_IN(c_span, reinterpret_cast<v4f*>(C + (size_t)m * N + n0 + 4 * lane), v);
    }
  }
}

// 256x256 workgroup tile, k-step 32, four 32 KiB LDS stages fed by
// global_load_lds_dwordx4 (the AIE ping-pong generalised to depth 4), one
// barrier per tile; each wave owns a 128x128 quarter (4x4
// v_mfma_f32_32x32x16_bf16 per 16-wide k-step) with register-double-buffered
// fragments.  Same schedule as the int8 kernel.
//
// LDS layouts (per stage):
//   A  [256 rows][32 bf16 = 64 B]: 16-byte chunk c of row r at c ^ swz(r).
//   B  [32 k-rows][256 bf16 = 512 B] (row-major as in memory): 16-byte chunk
//      c of k-row k at c ^ ((k & 3) << 2).  Fragments (8 consecutive k of
//      one column per lane) come from two ds_read_b64_tr_b16, each
//      transposing a 4 x 16 block; the XOR puts the 4 k-rows x 64 bytes that
//      one 32-lane half reads on distinct banks.
constexpr int BM = 256, BN = 256, BK = 32, STAGES = 4;
constexpr int TILE_BYTES = BM * BK * 2;       // 16 KiB per operand per stage
constexpr int STAGE_BYTES = 2 * TILE_BYTES;   // 32 KiB
constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
constexpr int CP_PER_TILE = 8;                // 16-byte LDS copies per thread per tile

__global__ __launch_bounds__(256, 1) void gemm_bf16_tile256(const uint16_t* __restrict__ A,
                                                            const uint16_t* __restrict__ B,
                                                            float* __restrict__ C, int M, int N, int K) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];
  const uint32_t lds0 = dev::lds_addr(lds);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tm, tn;
  dev::tile_coords<4>(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = dev::tile_origin(tm, BM, M), n0 = dev::tile_origin(tn, BN, N);
  const size_t lda = (size_t)K * 2, ldb = (size_t)N * 2;  // row pitches in bytes

  // Copy i (< 4) of wave w fills 1 KiB of a stage: A rows 64i + 16w + lane/4
  // (physical chunk lane%4); B k-rows 8i + 2w + lane/32 (physical chunk lane%32).
  const int a_r = 16 * wave + (lane >> 2);
  const uint32_t a_voff = (uint32_t)(a_r * lda) + 16 * ((lane & 3) ^ swz(a_r));
  const int8_t* const a_base = reinterpret_cast<const int8_t*>(A) + (size_t)m0 * lda;
  const int b_r = 2 * wave + (lane >> 5);  // (b_r + 8i) & 3 == b_r & 3
  const uint32_t b_voff = (uint32_t)(b_r * ldb) + 16 * ((lane & 31) ^ ((b_r & 3) << 2));
  const int8_t* const b_base = reinterpret_cast<const int8_t*>(B) + (size_t)n0 * 2;
  const dbg::Span a_span = dbg::span_of(A), b_span = dbg::span_of(B);  // (debug build only)

  auto issue = [&](int kt, int stage, int i) {
    const uint32_t st = lds0 + stage * STAGE_BYTES + 1024 * wave;
    if (i < 4)
      dev::gload_lds16(a_base + (size_t)kt * BK * 2 + (size_t)(64 * i) * lda, a_voff, st + 4096 * i, a_span);
    else
      dev::gload_lds16(b_base + (size_t)kt * BK * ldb + (size_t)(8 * (i - 4)) * ldb, b_voff,
                       st + TILE_BYTES + 4096 * (i - 4), b_span);
  };

  // fragment offsets within a stage
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  int a_fo[2], b_fo[4];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) a_fo[ks] = (wm * 128 + fr) * 64 + (((2 * ks + fh) ^ swz(fr)) << 4);
  {
    // tr16 read (ks, j, r): lane 16g + 4jj + q supplies k-row 16ks + 8(g>>1) + 4r + jj,
    // columns wn*128 + 32j + 16(g&1) + 4q .. +4; it receives column
    // wn*128 + 32j + lane%32 at k = 16ks + 8*(lane/32) + 4r + (0..3).
    const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = wn * 16 + 4 * j + 2 * (g & 1) + (q >> 1);
      b_fo[j] = TILE_BYTES + (8 * (g >> 1) + jj) * 512 + ((c ^ (jj << 2)) << 4) + 8 * (q & 1);
    }
  }

  struct Frags {
    v4i a[4];
    miaie_v4s lo[4], hi[4];
  };
  auto read_one = [&](int stage, int ks, int qd, Frags& f) {
    const int8_t* s = lds + stage * STAGE_BYTES;
    if (qd < 4) {
      f.a[qd] = *reinterpret_cast<const v4i*>(s + a_fo[ks] + 2048 * qd);
    } else {
      const int j = (qd - 4) >> 1;
      if ((qd & 1) == 0)
        f.lo[j] = dev::lds_read_tr16(s + b_fo[j] + ks * 8192);
      else
        f.hi[j] = dev::lds_read_tr16(s + b_fo[j] + ks * 8192 + 2048);
    }
  };
  auto bfrag = [&](const Frags& f, int j) -> v8bf {
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s v = {f.lo[j][0], f.lo[j][1], f.lo[j][2], f.lo[j][3], f.hi[j][0], f.hi[j][1], f.hi[j][2], f.hi[j][3]};
    return __builtin_bit_cast(v8bf, v);
  };
  constexpr int NREAD = 12;

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16f{0.f};

  const int KT = K / BK;
  // A tile's 8 copies go out in two halves spread over the MFMA slots of one
  // phase each: the first 4 in phase 2 of the tile four earlier (after the
  // barrier that frees their stage), the other 4 in phase 1 of the tile three
  // earlier; a whole tile's copies in one phase saturate the vector-memory
  // path and stall the in-order wave's MFMAs.  The prologue sends tiles 0..2
  // and the first half of tile 3; tile 0's phase 1 sends the rest.
  constexpr int CP_A = CP_PER_TILE / 2;
  static_assert(CP_PER_TILE == 2 * CP_A, "a tile's copies go out in two equal halves");
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    if (s < KT) {
#pragma unroll
      for (int i = 0; i < (s == STAGES - 1 ? CP_A : CP_PER_TILE); ++i) issue(s, s, i);
    }
  if (KT >= 4)
    dev::wait_vmcnt<2 * CP_PER_TILE + CP_A>();
  else if (KT == 3)
    dev::wait_vmcnt<2 * CP_PER_TILE>();
  else if (KT == 2)
    dev::wait_vmcnt<CP_PER_TILE>();
  else
    dev::wait_vmcnt<0>();
  dev::barrier();

  // Reads go out two per MFMA slot in the order the MFMA sequence
  // first needs them: B0 (two halves), A0, B1 .. B3, A1 .. A3.
  auto read_n = [](int n) { return n < 2 ? 4 + n : n == 2 ? 0 : n <= 8 ? 3 + n : n - 8; };
  Frags f0, f1;
#pragma unroll
  for (int n = 0; n < NREAD; ++n) read_one(0, 0, read_n(n), f0);
  auto read_slot = [&](int stage, int ks, int x, Frags& f) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (2 * x + r < NREAD) read_one(stage, ks, read_n(2 * x + r), f);
  };
  auto copy_slot = [&](int kt_dst, int stage, int x, int first) {
#pragma unroll
    for (int c = 0; c < CP_A; ++c)
      if (c * 16 / CP_A == x) issue(kt_dst, stage, first + c);
  };

  // Phase 1 multiplies k-step 0 while the k-step-1 reads and the second half
  // of tile kt+3's copies go out; tile barrier; phase 2 multiplies k-step 1
  // while the first half of tile kt+4's copies and the k-step-0 reads of tile
  // kt+1 go out.  PRE: tile kt+3 exists; MORE: tile kt+4 exists; NEXT: tile
  // kt+1 exists; VM: copies allowed in flight once tile kt+1 has landed.
  auto tile = [&](int kt, auto pre_c, auto more_c, auto next_c, auto vm_c) {
    constexpr bool PRE = decltype(pre_c)::value, MORE = decltype(more_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    constexpr int VM = decltype(vm_c)::value;
    const int cur = kt & (STAGES - 1);
    // stage of tile kt+3 = stage of tile kt-1, whose reads ended before tile
    // kt-1's barrier (for kt = 0: stage 3, not read yet)
    const int pre_stage = (kt + 3) & (STAGES - 1);
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int i = x >> 2, j = dev::snake_j<4>(x);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfrag(f0, j), __builtin_bit_cast(v8bf, f0.a[i]),
                                                          acc[i][j], 0, 0, 0);
      read_slot(cur, 1, x, f1);
      if constexpr (PRE) copy_slot(kt + 3, pre_stage, x, CP_A);
      dev::sched_fence();
    }
    dev::waitcnt<VM, 0>();
    dev::barrier();
    const int nxt = (kt + 1) & (STAGES - 1);
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int i = x >> 2, j = dev::snake_j<4>(x);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfrag(f1, j), __builtin_bit_cast(v8bf, f1.a[i]),
                                                          acc[i][j], 0, 0, 0);
      if constexpr (MORE) copy_slot(kt + STAGES, cur, x, 0);
      if constexpr (NEXT) read_slot(nxt, 0, x, f0);
      dev::sched_fence();
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using V2 = std::integral_constant<int, 2 * CP_PER_TILE>;
  using V1 = std::integral_constant<int, CP_PER_TILE>;
  using V0 = std::integral_constant<int, 0>;
  int kt = 0;
  for (; kt + STAGES < KT; ++kt) tile(kt, T_{}, T_{}, T_{}, V2{});
  if (kt == KT - 4) tile(kt++, T_{}, F_{}, T_{}, V2{});
  if (kt == KT - 3) tile(kt++, F_{}, F_{}, T_{}, V1{});
  if (kt == KT - 2) tile(kt++, F_{}, F_{}, T_{}, V0{});
  tile(kt, F_{}, F_{}, F_{}, V0{});

  store_tile_f32(acc, lds, wave, lane, C, m0, n0, N);
}

// Pair-staged geometry (K % 64 == 0): A in three LDS stages of 256 rows x 128
// bytes (two k-tiles, 64 bf16 of k), so each A copy moves whole 128-byte lines
// instead of touching 16 lines at half use; B keeps four per-k-tile stages
// (32 k-rows of 512 bytes, whole lines already).  160 KiB of LDS.  The copy
// schedule is the int8 pair-staged kernel's (dev::pair_vm): B k-tile k in two
// halves at phases 2k-7 and 2k-6, A pair p in quarters at phases 4p-9+q.
// A copy x of wave w: rows 8(4x + w) + lane/8, physical chunk lane%8 of the
// row's 128 bytes, holding logical chunk (lane%8) ^ ((row >> 1) & 7), so a
// fragment read (16 consecutive rows, one logical chunk) touches 16 distinct
// bank groups.  B copy i: k-rows 8i + 2w + lane/32, physical chunk lane%32.
constexpr int NA2 = 3;
constexpr int A2_BYTES = BM * 128;                  // one A pair stage (32 KiB)
constexpr int A_REGION = NA2 * A2_BYTES;            // 96 KiB
constexpr int B_BYTES = BK * BN * 2;                // one B stage (16 KiB)
constexpr int PAIR_LDS = A_REGION + STAGES * B_BYTES;
constexpr int A_CP2 = A2_BYTES / 4096, QA = A_CP2 / 4;  // A copies per thread per pair / per phase
constexpr int B_CP = B_BYTES / 4096, B_CP0 = (B_CP + 1) / 2, B_CP1 = B_CP - B_CP0;
static_assert(PAIR_LDS <= 163840, "pair-staged LDS budget");

// ------------------------------------------- pair-staged, 16x16x32 MFMA
// The pair-staged geometry above with the multiplies on
// v_mfma_f32_16x16x32_bf16: the same MACs per cycle as the 32x32x16 form,
// half the accumulator bits per MAC, and under the power limit a higher clock
// (register-only random bf16 operands: 1.86 PFLOP/s at 1.82 GHz against 1.63
// at 1.60 GHz on the 32x32x16 form, same GPU, same run).  The k-loop follows
// the int8 kernel gemm_i8_pipe16 (gemm_i8_kernels.hpp): each wave's 128x128
// quarter is 8 x 8 blocks of 16 x 16, a 32-wide k-tile is one k-step, block
// rows 0-3 are multiplied in phase 1 and 4-7 in phase 2 (column-block-major,
// rows reversed on odd column blocks so consecutive MFMAs share an operand),
// one set of fragment registers, accumulators updated in place by inline
// MFMAs (the int8 kernel's notes on why, and the CPU check of the generated
// assembly, apply here too).
//
// LDS: the four B stages first (so a B fragment read is a base register plus
// a compile-time offset where the stage is known), then the three A pair
// stages.  B k-row k (512 bytes) holds logical 16-byte chunk c at
// c ^ bswz16(k), bswz16(k) = ((k & 3) << 2) | (((k >> 3) & 1) << 1): a
// fragment half (ds_read_b64_tr_b16) has lane 16g + 4jj + q supply k-row
// 8g + 4r + jj, 8 bytes of chunk (16 wn + 2j) + q/2, and lane 16g + c
// receives column c of the 16-column block, k = 8g + 4r + (0..3); the 32
// lanes of a read half (g = 0, 1) then touch 16 distinct 16-byte bank groups.
// A fragment i: row 16i + lane%16 of the wave's rows, logical chunk lane/16 of
// the k-tile (k = 8(lane/16) .. +8), as in the int8 kernel.
__device__ __forceinline__ int bswz16(int k) { return ((k & 3) << 2) | (((k >> 3) & 1) << 1); }

__device__ __forceinline__ void mfma16_bf16(v4f& acc, v4i a, v4i b) {
#if MIAIE_DEVICE_CHECKS
  // debug build: the compiler's own MFMA, whose hazards it tracks (see mfma16)
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(a), as_bf(b), acc, 0, 0, 0);
#else
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
#endif
}

// fp32 epilogue of a 256x256 tile held as acc[i][j][e] = C[m0 + wm*128 + 16i +
// lane%16][n0 + wn*128 + 16j + 4(lane/16) + e], staged through LDS in two
// halves of 64 rows per wave row (block rows i = 4h .. 4h+3) so that every
// store writes one whole 1 KiB row: LDS row R = wm*64 + 16(i - 4h) + lane%16,
// 16-byte chunk c = 32 wn + 4j + lane/16 at physical chunk c ^ (R & 15).
__device__ __forceinline__ void store_tile16_f32(const v4f (&acc)[8][8], int8_t* lds, int wave, int lane, float* C,
                                                 int m0, int n0, int N) {
  const int wm = wave >> 1, wn = wave & 1, fr = lane & 15, fg = lane >> 4;
  const dbg::Span c_span = dbg::span_of(C);  // (debug build only)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    dev::barrier();  // the other waves' last reads of this LDS
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int R = wm * 64 + 16 * ii + fr;
        const int c = wn * 32 + 4 * j + fg;
        *reinterpret_cast<v4f*>(lds + R * 1024 + ((c ^ (R & 15)) << 4)) = acc[4 * h + ii][j];
      }
    dev::barrier();
#pragma unroll
    for (int rr = 0; rr < 32; ++rr) {
      const int R = wave * 32 + rr;
      const v4f v = *reinterpret_cast<const v4f*>(lds + R * 1024 + ((lane ^ (R & 15)) << 4));
      const int m = m0 + (R >> 6) * 128 + 64 * h + (R & 63);
      MIAIE_ST_NT_IN(c_span, reinterpret_cast<v4f*>(C + (size_t)m * N + n0 + 4 * lane), v);
    }
  }
}

__global__ __launch_bounds__(256, 1) void gemm_bf16_pair16(const uint16_t* __restrict__ A,
                                                           const uint16_t* __restrict__ B,
                                                           float* __restrict__ C, int M, int N, int K) {
  constexpr int B_REGION = STAGES * B_BYTES;  // 64 KiB, first
  constexpr int B_MASK = B_REGION - 1;
  static_assert((B_REGION & B_MASK) == 0 && B_REGION + A_REGION == PAIR_LDS, "B stages first");
  constexpr int NI = 8, NJ = 8, HI = 4, PH = HI * NJ;
  __shared__ __attribute__((aligned(1024))) int8_t lds[PAIR_LDS];
  const uint32_t lds0 = dev::lds_addr(lds);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tm, tn;
  dev::tile_coords<4>(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = dev::tile_origin(tm, BM, M), n0 = dev::tile_origin(tn, BN, N);
  const size_t lda = (size_t)K * 2, ldb = (size_t)N * 2;  // row pitches in bytes
  const int KT = K / BK;                                   // even

  // copies (B with bswz16, whose bit 1 is k-row bit 3 = the copy's parity)
  const int a_r = 8 * wave + (lane >> 3);
  const uint32_t a_voff = (uint32_t)(a_r * lda) + 16 * ((lane & 7) ^ ((a_r >> 1) & 7));
  const int8_t* const a_base = reinterpret_cast<const int8_t*>(A) + (size_t)m0 * lda;
  const int b_r = 2 * wave + (lane >> 5);
  uint32_t b_voff[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) b_voff[e] = (uint32_t)(b_r * ldb) + 16 * ((lane & 31) ^ bswz16(b_r + 8 * e));
  const int8_t* const b_base = reinterpret_cast<const int8_t*>(B) + (size_t)n0 * 2;
  const size_t b_kstep = (size_t)BK * ldb;
  const uint32_t ldsw = lds0 + 1024 * wave;
  const dbg::Span a_span = dbg::span_of(A), b_span = dbg::span_of(B);  // (debug build only)
  auto copy_a = [&](const int8_t* src, uint32_t st, int x) __attribute__((always_inline)) {
    dev::gload_lds16(src + (size_t)(32 * x) * lda, a_voff, ldsw + B_REGION + st + 4096 * x, a_span);
  };
  auto copy_b = [&](const int8_t* src, uint32_t st, int x) __attribute__((always_inline)) {
    dev::gload_lds16(src + (size_t)(8 * x) * ldb, b_voff[x & 1], ldsw + st + 4096 * x, b_span);
  };

  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 15, fg = lane >> 4;
  int a_fo[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) a_fo[par] = (wm * 128 + fr) * 128 + (((4 * par + fg) ^ ((fr >> 1) & 7)) << 4);
  int b_fo[NJ];
  {
    const int jj = (lane >> 2) & 3, q = lane & 3;
    const int kr = 8 * fg + jj;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = wn * 16 + 2 * j + (q >> 1);
      b_fo[j] = kr * 512 + ((c ^ bswz16(kr)) << 4) + 8 * (q & 1);
    }
  }
  v4i alo[HI], ahi[HI];
  miaie_v4s blo[NJ], bhi[NJ];
  auto read_a = [&](uint32_t st, int par, int i) __attribute__((always_inline)) -> v4i {
    const uint32_t sbase = __builtin_amdgcn_readfirstlane(B_REGION + st);
    return *reinterpret_cast<const v4i*>(lds + sbase + a_fo[par] + 2048 * i);
  };
  auto read_b = [&](int st, int j) __attribute__((always_inline)) {
    blo[j] = dev::lds_read_tr16(lds + st + b_fo[j]);
    bhi[j] = dev::lds_read_tr16(lds + st + b_fo[j] + 2048);
  };
  auto bfrag = [&](int j) __attribute__((always_inline)) -> v4i {
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s v = {blo[j][0], blo[j][1], blo[j][2], blo[j][3], bhi[j][0], bhi[j][1], bhi[j][2], bhi[j][3]};
    return __builtin_bit_cast(v4i, v);
  };

  v4f acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // prologue: phases -9 .. -1 in order, then wait for B k-tile 0 and A pair 0
  const int KP = KT / 2;
#pragma unroll
  for (int phi = -9; phi < 0; ++phi) {
    if ((phi & 1) != 0) {
      const int k = (phi + 7) / 2;
      if (phi >= -7 && k < KT)
#pragma unroll
        for (int x = 0; x < B_CP0; ++x) copy_b(b_base + k * b_kstep, k * B_BYTES, x);
    } else {
      const int k = (phi + 6) / 2;
      if (phi >= -6 && k < KT)
#pragma unroll
        for (int x = B_CP0; x < B_CP; ++x) copy_b(b_base + k * b_kstep, k * B_BYTES, x);
    }
    const int p = (phi + 9) / 4, q = (phi + 9) % 4;
    if (p < KP)
#pragma unroll
      for (int x = 0; x < QA; ++x) copy_a(a_base + p * 128, p * A2_BYTES, QA * q + x);
  }
  if (KT >= 6)
    dev::wait_vmcnt<dev::pair_prologue_vm(B_CP0, B_CP1, QA)>();
  else
    dev::wait_vmcnt<0>();
  dev::barrier();
#pragma unroll
  for (int j = 0; j < NJ; ++j) read_b(0, j);
#pragma unroll
  for (int i = 0; i < HI; ++i) alo[i] = read_a(0, 0, i);

  uint32_t sa0 = 0, sa1 = A2_BYTES, sa2 = 2 * A2_BYTES;  // stages of pairs P, P+1, P+2
  const int8_t* a_src = a_base + 2 * 128;                 // A source of pair P+2
  const int8_t* b_src = b_base + 3 * b_kstep;             // B source of k-tile t+3
  int sb_rt = 0;                                          // B stage of tile t

  auto tile = [&](auto par_c, auto d_c, auto sb_c) __attribute__((always_inline)) {
    constexpr int PAR = decltype(par_c)::value, D = decltype(d_c)::value, SB = decltype(sb_c)::value;
    constexpr int NB1 = D >= 3 ? B_CP1 : 0, NB2 = D >= 4 ? B_CP0 : 0;
    constexpr int NA1 = (PAR == 0 ? D >= 5 : D >= 4) ? QA : 0;
    constexpr int NA2_ = (PAR == 0 ? D >= 5 : D >= 6) ? QA : 0;
    constexpr bool NEXT = D >= 1;
    constexpr int VM = dev::pair_vm(D, B_CP0, B_CP1, QA);
    const int sbc = SB >= 0 ? SB * B_BYTES : sb_rt;
    const int sb1 = SB >= 0 ? ((SB + 1) & 3) * B_BYTES : (sb_rt + B_BYTES) & B_MASK;
    const int sb3 = SB >= 0 ? ((SB + 3) & 3) * B_BYTES : (sb_rt + 3 * B_BYTES) & B_MASK;
    constexpr int qa1 = PAR == 0 ? 1 : 3;
#pragma unroll
    for (int x = 0; x < PH; ++x) {
      const int j = x / HI, i = dev::snake_j<HI>(x);
      mfma16_bf16(acc[i][j], bfrag(j), alo[i]);
      if (x < HI) ahi[x] = read_a(sa0, PAR, HI + x);
#pragma unroll
      for (int c = 0; c < NB1 + NA1; ++c)
        if ((c * PH) / (NB1 + NA1 > 0 ? NB1 + NA1 : 1) == x) {
          if (c < NB1)
            copy_b(b_src, sb3, B_CP0 + c);
          else
            copy_a(a_src, sa2, QA * qa1 + c - NB1);
        }
      dev::sched_fence();
    }
    dev::waitcnt<VM, 0>();
    dev::barrier();
    constexpr int qa2 = PAR == 0 ? 2 : 0;
    const int8_t* const a_src2 = PAR == 0 ? a_src : a_src + 128;
    const uint32_t sa_cp2 = PAR == 0 ? sa2 : sa0;
    const uint32_t sa_next = PAR == 0 ? sa0 : sa1;
#pragma unroll
    for (int x = 0; x < PH; ++x) {
      const int j = x / HI, i = dev::snake_j<HI>(x);
      mfma16_bf16(acc[HI + i][j], bfrag(j), ahi[i]);
#pragma unroll
      for (int c = 0; c < NB2 + NA2_; ++c)
        if ((c * PH) / (NB2 + NA2_ > 0 ? NB2 + NA2_ : 1) == x) {
          if (c < NB2)
            copy_b(b_src + b_kstep, sbc, c);
          else
            copy_a(a_src2, sa_cp2, QA * qa2 + c - NB2);
        }
      if constexpr (NEXT) {
        if (x < HI) alo[x] = read_a(sa_next, 1 - PAR, x);
        if (x % HI == HI - 1) read_b(sb1, j);  // after the last use of tile t's B fragment j
      }
      dev::sched_fence();
    }
    b_src += b_kstep;
    sb_rt = (sb_rt + B_BYTES) & B_MASK;
    if constexpr (PAR == 1) {
      const uint32_t s3 = sa0;
      sa0 = sa1;
      sa1 = sa2;
      sa2 = s3;
      a_src += 128;
    }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using DS = std::integral_constant<int, 64>;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using SR = std::integral_constant<int, -1>;
  int t = 0;
  for (; t + 10 <= KT; t += 4) {
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
  // the last MFMAs' results are read only after their latency
  dev::sched_fence();
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  dev::sched_fence();

  store_tile16_f32(acc, lds, wave, lane, C, m0, n0, N);
}

__global__ __launch_bounds__(256) void gemm_bf16_tile64(const uint16_t* __restrict__ A,
                                                        const uint16_t* __restrict__ B,
                                                        float* __restrict__ C, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) int8_t as[64 * 64];
  __shared__ __attribute__((aligned(16))) int8_t bs[64 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  v16f acc = v16f{0.f};
  for (int k0 = 0; k0 < K; k0 += 32) {
    {
      const int row = tid >> 2, ch = tid & 3;
      const int m = m0 + row, k = k0 + ch * 8;
      uint16_t tmp[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) tmp[t] = (m < M && k + t < K) ? MIAIE_LD(A + (size_t)m * K + k + t) : 0;
      v4i v;
      __builtin_memcpy(&v, tmp, 16);
      *reinterpret_cast<v4i*>(as + lds_off(row, ch)) = v;
    }
    {
      const int col = tid & 63, ch = tid >> 6;
      const int n = n0 + col;
      uint16_t tmp[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int k = k0 + ch * 8 + t;
        tmp[t] = (n < N && k < K) ? MIAIE_LD(B + (size_t)k * N + n) : 0;
      }
      v4i v;
      __builtin_memcpy(&v, tmp, 16);
      *reinterpret_cast<v4i*>(bs + lds_off(col, ch)) = v;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const v4i af = *reinterpret_cast<const v4i*>(as + lds_off(wm * 32 + fr, 2 * ks + fh));
      const v4i bf = *reinterpret_cast<const v4i*>(bs + lds_off(wn * 32 + fr, 2 * ks + fh));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(bf), as_bf(af), acc, 0, 0, 0);
    }
    __syncthreads();
  }
  const int m = m0 + wm * 32 + fr;
  if (m >= M) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int n = n0 + wn * 32 + 8 * (e >> 2) + 4 * fh + (e & 3);
    if (n < N) MIAIE_ST(C + (size_t)m * N + n, acc[e]);
  }
}

// The 64x64 kernel for K % 8 == 0 and a 16-byte aligned A (a ragged M, N
// or K): A rows are loaded as full vectors and B columns gathered from clamped,
// always valid addresses, zeroed when written to LDS if outside the matrix,
// and the next k-tile's loads are issued before this k-tile's LDS reads and
// MFMAs, so their latency overlaps the MFMAs.
__global__ __launch_bounds__(256) void gemm_bf16_tile64p(const uint16_t* __restrict__ A,
                                                         const uint16_t* __restrict__ B,
                                                         float* __restrict__ C, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) int8_t as[64 * 64];
  __shared__ __attribute__((aligned(16))) int8_t bs[64 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  // A: thread -> row tid/4, 8-element chunk tid%4; B: column tid%64, k-chunk tid/64
  const int row = tid >> 2, ch = tid & 3, col = tid & 63, bch = tid >> 6;
  // K % 8 == 0: an 8-element k-chunk lies wholly inside or wholly past K; one
  // past K loads the row's last chunk instead and is zeroed
  const bool a_in = m0 + row < M, b_in = n0 + col < N;
  const uint16_t* const a_p = A + (size_t)min(m0 + row, M - 1) * K;
  const uint16_t* const b_p = B + min(n0 + col, N - 1);
  auto load = [&](int k0, v4i& va, v4i& vb) {
    va = MIAIE_LD(reinterpret_cast<const v4i*>(a_p + min(k0 + 8 * ch, K - 8)));
    const uint16_t* const p = b_p + (size_t)min(k0 + 8 * bch, K - 8) * N;
    uint16_t tmp[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) tmp[t] = MIAIE_LD(p + (size_t)t * N);
    __builtin_memcpy(&vb, tmp, 16);
  };
  v16f acc = v16f{0.f};
  v4i va, vb;
  load(0, va, vb);
  for (int k0 = 0; k0 < K; k0 += 32) {
    *reinterpret_cast<v4i*>(as + lds_off(row, ch)) = a_in && k0 + 8 * ch < K ? va : v4i{0};
    *reinterpret_cast<v4i*>(bs + lds_off(col, bch)) = b_in && k0 + 8 * bch < K ? vb : v4i{0};
    __syncthreads();
    if (k0 + 32 < K) load(k0 + 32, va, vb);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const v4i af = *reinterpret_cast<const v4i*>(as + lds_off(wm * 32 + fr, 2 * ks + fh));
      const v4i bf = *reinterpret_cast<const v4i*>(bs + lds_off(wn * 32 + fr, 2 * ks + fh));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf(bf), as_bf(af), acc, 0, 0, 0);
    }
    __syncthreads();
  }
  const int m = m0 + wm * 32 + fr;
  if (m >= M) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int n = n0 + wn * 32 + 8 * (e >> 2) + 4 * fh + (e & 3);
    if (n < N) MIAIE_ST(C + (size_t)m * N + n, acc[e]);
  }
}

}  // namespace

namespace miaie {

int launch_gemm_bf16(miaie_ctx* ctx, const uint16_t* A, const uint16_t* B, float* C, int M, int N, int K) {
  // 256x256 kernels: 16-byte aligned operands, per-lane copy offsets of up
  // to 64 rows in 32 bits, and whole tiles, or else the last tile row
  // (column) moved back over its neighbour (dev::tile_origin; N % 8 == 0
  // keeps B and C rows on 16-byte chunks) when the tiles fill at least half
  // the CUs (fewer, and the 64x64 kernel's wider grid is the faster one).
  const long tiles = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const bool whole = M % BM == 0 && N % BN == 0;
  const bool overlap = M >= BM && N >= BN && N % 8 == 0 && 2 * tiles >= ctx->cus;
  const bool big = (whole || overlap) && K % BK == 0 && aligned(A, 16) && aligned(B, 16) && aligned(C, 16) &&
                   K < (1 << 24) && N < (1 << 24);
  if (big && K % (2 * BK) == 0) {
    return check_launch(ctx, launch<gemm_bf16_pair16>(ctx->device, dim3(tiles), dim3(256), 0, ctx->stream, A, B, C, M, N, K),
                        "gemm_bf16_pair16");
  }
  if (big) {
    return check_launch(ctx, launch<gemm_bf16_tile256>(ctx->device, dim3(tiles), dim3(256), 0, ctx->stream, A, B, C, M, N, K),
                        "gemm_bf16_tile256");
  }
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  if (grid.y > 65535) return fail(ctx, MIAIE_EINVAL, "gemm_bf16: M too large for the 64x64 fallback");
  if (K % 8 == 0 && aligned(A, 16)) {
    return check_launch(ctx, launch<gemm_bf16_tile64p>(ctx->device, grid, dim3(256), 0, ctx->stream, A, B, C, M, N, K),
                        "gemm_bf16_tile64p");
  }
  return check_launch(ctx, launch<gemm_bf16_tile64>(ctx->device, grid, dim3(256), 0, ctx->stream, A, B, C, M, N, K),
                      "gemm_bf16_tile64");
}

}  // namespace miaie
