// Row-block int8 conv2d kernel (device code), shared by the library
// (conv2d_i8.hip) and the in-kernel clock probe (probes/conv_span.hip).
//
// For stride-1 convolutions (instantiated for 3x3 filters and Cin in {32,
// 64, 128}).  A workgroup owns ROWS output rows of one image, 64 columns of
// them (padded; wider rows are cut into blocks of 64 columns), and one block
// of WCO output channels, with ROWS * WCO = 128 so that its 8 waves each own
// 32 pixels x 32 channels.  It stages in LDS
// once, with every global load of the staging in flight together:
//   X  the ROWS+R-1 input rows the output rows touch, with the zero padding
//      columns and rows materialised, [row][col][Cin bytes], 16-byte chunk
//      c of column col at c ^ xswz(col) (conflict-free fragment reads);
//   W  the WCO output channels' OHWI rows, pitch R*S*Cin + 16 bytes.
// Each wave then runs the whole k = (r, s, ci) reduction from LDS (one
// v_mfma_i32_32x32x32_i8 per 32-wide k-step, fully unrolled), so there is no
// im2col buffer and no cross-wave reduction.  The requantized int8 results
// go through a third LDS region: each wave writes its 32 pixels x 32
// channels there and reads them back as 16-byte pieces, two lanes per pixel,
// so every pixel's 32 channels leave as one 32-byte run, with an LDS wait and
// no workgroup barrier.  (Stored straight from the accumulators, each lane
// wrote 4-byte pieces of 8 different 64-byte pixel runs, and the lines left
// partially written in L2 made the end of every launch 0.3-0.4 us longer.
// A workgroup-wide store of whole ROWS x Wo x WCO runs after a barrier
// measured 0.6% slower per launch than the per-wave store.)
//
// Tile order: with N a multiple of 8 the grid is (8, row blocks, N/8 *
// channel blocks) and workgroup (x, y, z) takes image 8*(z mod N/8) + x.
// Workgroups are dealt round-robin to the 8 XCDs in linear order, so XCD x
// runs every workgroup of its images and the ROWS+2 staged rows of
// neighbouring row blocks, which overlap in 2 rows, are fetched into its L2
// once (measured: 1.98 MB read per launch at config 4 against 3.52 MB with
// neighbouring row blocks on different XCDs; X + W is 1.64 MB).  Otherwise
// the grid is (row blocks, channel blocks, N).
#pragma once

#include <type_traits>

#include "dbg_checks.hpp"
#include "miaie_internal.hpp"

namespace miaie {
namespace conv {

constexpr int PB = 64;  // output columns per row (padded)

template <int CIN>
__device__ __forceinline__ int xswz(int col) {
  return (col * CIN / 256) & (CIN / 16 - 1);
}

// BW: output columns per block (64, or 32 for narrow layers).
template <int R, int S, int CIN, int ROWS, int WCO, int BW = PB>
struct RowsGeom {
  static_assert(ROWS * WCO % 128 == 0 && WCO % 32 == 0, "8 waves of 32 pixels x 32 channels (or a multiple)");
  static constexpr int NWC = WCO / 32;                      // 32-channel blocks per workgroup
  static constexpr int XR = ROWS + R - 1, XC = BW + S - 1;  // staged input rows / columns
  static constexpr int NCH = CIN / 16;                      // 16-byte chunks per pixel
  static constexpr int BW_ = BW;
  // X staging map: one pass covers RPP whole rows of the first BW staged
  // columns (thread -> chunk tid % NCH of column tid / NCH % BW), XQ passes
  // cover the XR rows, and one more load per thread (the first XE threads)
  // covers the last S - 1 columns of every row.
  static constexpr int RPP = 512 / (BW * NCH);              // rows per pass
  static constexpr int XQ = (XR + RPP - 1) / RPP;           // passes
  static constexpr int XE = XR * (XC - BW) * NCH;           // chunks of the last S - 1 columns
  static constexpr int RSC = R * S * CIN, WP = RSC + 16;    // weight row length / LDS pitch
  static constexpr int WTOT = WCO * RSC / 16;               // W chunks
  static constexpr int WQ = (WTOT + 511) / 512;
  static constexpr int WREM = WTOT - 512 * (WQ - 1);        // W chunks of the last pass
  static_assert(512 % (BW * NCH) == 0 && XE <= 512, "row-block conv staging map");
  static constexpr int X_BYTES = XR * XC * CIN;
  static constexpr int W_BYTES = WCO * WP;
  static constexpr int YP = WCO + 16;                       // LDS pitch of one staged output pixel
  static constexpr int Y_BYTES = ROWS * BW * YP;
  static constexpr int LDS = X_BYTES + W_BYTES + Y_BYTES;
  static constexpr int T = R * S * CIN / 32;                // 32-wide k-steps
  static_assert(LDS <= 163840, "row-block conv LDS budget (160 KiB per workgroup on gfx950)");
};

// Requantize one wave's 32 pixels x 32 channels into its part of the Y
// region and store them.  acc[4g + tt]: channel 32wc + 8g + 4*(lane/32) + tt
// of pixel 32pb + lane%32 (four consecutive channels of one pixel per
// dword), started at the rounding term 2^(s-1) of its channel.  Each wave
// then stores its own 32 pixels x 32 channels from its own part of the Y
// region, after an LDS wait and no workgroup barrier: lane l takes pixel
// 32pb + l/2, 16 channels 32wc + 16(l%2), so a pixel's 32 channels leave as
// one 32-byte run.  (Padding columns px >= Wo land in LDS and stay there.)
template <class G>
__device__ __forceinline__ void rows_epilogue(const v16i& acc, const uint32_t (&sh4)[4], bool hi_form, int8_t* ys,
                                              int rr, int pb, int wc, int fr, int fh, int lane, int n, int ho0,
                                              int wc0, int co0, int Ho, int Wo, int Cout, int8_t* __restrict__ Y) {
  const int px = 32 * pb + fr;
  int8_t* const yl = ys + (rr * G::BW_ + px) * G::YP + 32 * wc + 4 * fh;
  if (hi_form) {
    // every shift of the wave >= 8: y is the high byte of
    // sat_int16(acc >> (s - 8)) (floor shifts compose; saturating at 16 bits
    // clamps the high byte exactly at -128 and 127), 7 instructions per 4
    // channels
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t sm8 = sh4[g] - 0x08080808u;  // bytewise s - 8 (no borrow: every byte >= 8)
      const int u0 = acc[4 * g] >> (sm8 & 31), u1 = acc[4 * g + 1] >> ((sm8 >> 8) & 31);
      const int u2 = acc[4 * g + 2] >> ((sm8 >> 16) & 31), u3 = acc[4 * g + 3] >> ((sm8 >> 24) & 31);
      const uint32_t p01 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(u0, u1));
      const uint32_t p23 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(u2, u3));
      *reinterpret_cast<uint32_t*>(yl + 8 * g) = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
    }
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t packed = 0;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int q = min(max(acc[4 * g + tt] >> ((sh4[g] >> (8 * tt)) & 31), -128), 127);
        packed |= (uint32_t)(q & 0xFF) << (8 * tt);
      }
      *reinterpret_cast<uint32_t*>(yl + 8 * g) = packed;
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
  __builtin_amdgcn_wave_barrier();
  const int sp = 32 * pb + (lane >> 1), sh = lane & 1;
  if (wc0 + sp < Wo && ho0 + rr < Ho) {
    const v4i v = *reinterpret_cast<const v4i*>(ys + (rr * G::BW_ + sp) * G::YP + 32 * wc + 16 * sh);
    MIAIE_ST(reinterpret_cast<v4i*>(Y + (uint32_t)(((n * Ho + ho0 + rr) * Wo + wc0 + sp) * Cout + co0 + 32 * wc + 16 * sh)), v);
  }
}

// Clock probe records per wave (TIMED instantiations only): shader clock at
// the start, after the staging barrier, after the MFMA loop and at the end,
// then the 100 MHz wall clock at the start and the end.
constexpr int PROBE_WORDS = 6;

// xg: 0 for the (row blocks, channel blocks, N) grid, else N / 8 for the
// image-per-XCD grid.  ncb: blocks of PB output columns per row (rows wider
// than PB are split; the row-block grid index counts row block x ncb +
// column block).  probe: PROBE_WORDS words per wave (TIMED only).
// The arguments fit the 14 dwords that arrive in SGPRs at wave launch (four
// pointers, then six ints with no alignment gap; the output size is
// H + 2 pad - 2 by W + 2 pad - 2), so nothing waits for a load from the
// argument segment; probe (TIMED only) comes after them.
template <int R, int S, int CIN, int ROWS, int WCO, bool TIMED>
__global__ __launch_bounds__(512) void conv2d_i8_rows(const int8_t* __restrict__ X, const int8_t* __restrict__ W,
                                                      const uint8_t* __restrict__ shifts, int8_t* __restrict__ Y,
                                                      int H, int Wd, int pad, int xg, int ncb, int Cout,
                                                      unsigned long long* __restrict__ probe) {
  using G = RowsGeom<R, S, CIN, ROWS, WCO>;
  const int Ho = H + 2 * pad - (R - 1), Wo = Wd + 2 * pad - (S - 1);
  __shared__ __attribute__((aligned(16))) int8_t smem[G::LDS];
  unsigned long long t0 = 0, r0 = 0;
  if constexpr (TIMED) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  int n, rb, cb;
  if (xg) {
    rb = blockIdx.y;
    const int z = blockIdx.z;
    cb = xg == 1 ? z : z / xg;
    n = 8 * (z - cb * xg) + blockIdx.x;
  } else {
    rb = blockIdx.x;
    cb = blockIdx.y;
    n = blockIdx.z;
  }
  int wc0 = 0;  // first output column of this block
  if (ncb > 1) {
    const int cbk = rb % ncb;
    rb /= ncb;
    wc0 = cbk * PB;
  }
  const int ho0 = rb * ROWS;
  const int co0 = cb * WCO;
  int8_t* const xs = smem;
  int8_t* const ws = smem + G::X_BYTES;
  int8_t* const ys = smem + G::X_BYTES + G::W_BYTES;

  // wave: output row rr, pixels 32pb .. +32, channels 32wc .. +32
  const int wc = wave % G::NWC, pb = (wave / G::NWC) & 1, rr = wave / (2 * G::NWC);

  // the wave's 32 output channels' shifts (4 per dword): one wave-uniform
  // load through the scalar cache, so the staging below is the only
  // vector-memory work ahead of the first wait (four per-lane loads of them
  // measured 1-2% slower per launch: the staging is bound by the issue of its
  // load instructions, not by their bytes)
  uint32_t s8[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) s8[q] = MIAIE_LD(reinterpret_cast<const uint32_t*>(shifts + co0 + 32 * wc) + q);
  // a wave-uniform value the compiler cannot see through: the conditional
  // last W pass below stays a branch around its load and its LDS write
  // instead of being merged into one block with a wait for the load
  auto opaque = [](int v) {
    asm volatile("" : "+s"(v));
    return v;
  };
  constexpr int WRW = (G::WREM + 63) / 64;  // waves that have chunks in the last W pass

  // ---- stage X (zero outside the image) and W.  Every load is issued before
  // any is waited for: positions outside the image load the nearest chunk
  // inside it and are zeroed by a select afterwards (a branch around the load would
  // make the zero write wait for the load in flight to the same registers).
  // Offsets are 32-bit from the tensor base: the launcher keeps X, W and Y
  // below 2^31 bytes.
  const int xc = tid % G::NCH, xcol = (tid / G::NCH) % PB, xrow = tid / (G::NCH * PB);
  // (threads past XE repeat an earlier thread's chunk: the same value to the
  // same LDS address, so the load and the write need no branch)
  const int et = tid % G::XE;
  const int ec = et % G::NCH, ecol = PB + (et / G::NCH) % (G::XC - PB), erow = et / (G::NCH * (G::XC - PB));
  auto x_off = [&](int row, int col, int c, bool& in) -> uint32_t {
    const int hi = ho0 + row - pad, wi = wc0 + col - pad;
    in = (unsigned)hi < (unsigned)H && (unsigned)wi < (unsigned)Wd;
    // clamped into the image: a valid address without a branch
    const int hc = min(max(hi, 0), H - 1), wcl = min(max(wi, 0), Wd - 1);
    return (uint32_t)(((n * H + hc) * Wd + wcl) * CIN + 16 * c);
  };
  v4i xv[G::XQ], xe, wv[G::WQ];
  bool xin[G::XQ], ein;
  // (a pass that runs past the last staged row repeats that row's chunks)
  auto xrow_of = [&](int u) { return min(G::RPP * u + xrow, G::XR - 1); };
#pragma unroll
  for (int u = 0; u < G::XQ; ++u)
    xv[u] = MIAIE_LD(reinterpret_cast<const v4i*>(X + x_off(xrow_of(u), xcol, xc, xin[u])));
  xe = MIAIE_LD(reinterpret_cast<const v4i*>(X + x_off(erow, ecol, ec, ein)));
  // (the last W pass is issued by the WRW waves that have chunks in it; the
  // lanes of a partial wave past its end repeat that pass's chunks)
  auto wq_of = [&](int u) { return u < G::WQ - 1 ? tid + 512 * u : 512 * (G::WQ - 1) + tid % G::WREM; };
#pragma unroll
  for (int u = 0; u < G::WQ - 1; ++u)
    wv[u] = MIAIE_LD(reinterpret_cast<const v4i*>(W + (uint32_t)(co0 * G::RSC + 16 * wq_of(u))));
  if (opaque(wave) < WRW)
    wv[G::WQ - 1] = MIAIE_LD(reinterpret_cast<const v4i*>(W + (uint32_t)(co0 * G::RSC + 16 * wq_of(G::WQ - 1))));
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait

  // This lane's 16 channels' shifts: channels 32wc + 8g + 4fh + tt.  (The
  // values pass through an empty asm so that the select stays a select of
  // two registers and does not become a lane-indexed read of s8.)
  uint32_t sh4[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint32_t lo = s8[2 * g], hi = s8[2 * g + 1];
    asm("" : "+s"(lo), "+s"(hi));
    sh4[g] = fh ? hi : lo;
  }
  // The accumulators start at the rounding term 2^(s-1) of their channel
  // (|acc| <= R*S*CIN * 2^14 < 2^30 keeps acc + 2^30 inside int32), so the
  // epilogue only shifts and saturates.  Computed here, while the staging
  // loads are in flight (the shifts were issued first).
  v16i acc;
  int smin = 31;
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int sc = (sh4[g] >> (8 * tt)) & 31;
      acc[4 * g + tt] = (int)((1u << sc) >> 1);
      smin = min(smin, sc);
    }
  const bool hi_form = __builtin_amdgcn_ballot_w64(smin < 8) == 0;  // every shift of the wave >= 8
  __builtin_amdgcn_sched_barrier(0);

  auto x_put = [&](int row, int col, int c, bool in, v4i v) {
    *reinterpret_cast<v4i*>(xs + (row * G::XC + col) * CIN + ((c ^ xswz<CIN>(col)) << 4)) = in ? v : v4i{0};
  };
#pragma unroll
  for (int u = 0; u < G::XQ; ++u) x_put(xrow_of(u), xcol, xc, xin[u], xv[u]);
  x_put(erow, ecol, ec, ein, xe);
  auto w_put = [&](int q, v4i v) {
    *reinterpret_cast<v4i*>(ws + (q / (G::RSC / 16)) * G::WP + 16 * (q % (G::RSC / 16))) = v;
  };
#pragma unroll
  for (int u = 0; u < G::WQ - 1; ++u) w_put(wq_of(u), wv[u]);
  if (opaque(wave) < WRW) w_put(wq_of(G::WQ - 1), wv[G::WQ - 1]);
  __syncthreads();
  unsigned long long t1 = 0;
  if constexpr (TIMED) t1 = __builtin_amdgcn_s_memtime();

  const int px = 32 * pb + fr;
  const int8_t* wrow = ws + (32 * wc + fr) * G::WP + 16 * fh;
#pragma unroll
  for (int t = 0; t < G::T; ++t) {
    const int cib = t % (CIN / 32), rs = t / (CIN / 32);
    const int r = rs / S, s = rs % S;
    const int col = px + s;
    const v4i xf = *reinterpret_cast<const v4i*>(xs + ((rr + r) * G::XC + col) * CIN +
                                                 (((2 * cib + fh) ^ xswz<CIN>(col)) << 4));
    const v4i wf = *reinterpret_cast<const v4i*>(wrow + 32 * t);
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf, xf, acc, 0, 0, 0);
  }
  unsigned long long t2 = 0;
  if constexpr (TIMED) t2 = __builtin_amdgcn_s_memtime();

  rows_epilogue<G>(acc, sh4, hi_form, ys, rr, pb, wc, fr, fh, lane, n, ho0, wc0, co0, Ho, Wo, Cout, Y);
  if constexpr (TIMED) {
    const unsigned long long t3 = __builtin_amdgcn_s_memtime(), r3 = __builtin_amdgcn_s_memrealtime();
    const unsigned long long rec[PROBE_WORDS] = {t0, t1, t2, t3, r0, r3};
    unsigned long long v = 0;
#pragma unroll
    for (int i = 0; i < PROBE_WORDS; ++i) v = lane == i ? rec[i] : v;
    const size_t wg = ((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    if (lane < PROBE_WORDS) probe[(wg * 8 + wave) * PROBE_WORDS + lane] = v;
  }
}

// Grid and launch of the row-block kernel (shapes already checked by the
// caller: rows_ok in conv2d_kernel_for).
template <int CIN, int ROWS, int WCO, bool TIMED>
inline hipError_t launch_rows_as(int device, hipStream_t st, const int8_t* X, const int8_t* W, const uint8_t* shifts,
                                 int8_t* Y, int N, int H, int Wd, int Cout, int pad, int Ho, int Wo,
                                 unsigned long long* probe = nullptr) {
  const int ncb = (Wo + PB - 1) / PB;
  const unsigned rbs = (unsigned)((Ho + ROWS - 1) / ROWS * ncb), cbs = (unsigned)(Cout / WCO);
  const bool by_xcd = N % 8 == 0 && rbs <= 65535 && (size_t)(N / 8) * cbs <= 65535;
  const dim3 grid = by_xcd ? dim3(8, rbs, (unsigned)(N / 8) * cbs) : dim3(rbs, cbs, (unsigned)N);
  return launch<conv2d_i8_rows<3, 3, CIN, ROWS, WCO, TIMED>>(device, grid, dim3(512), 0, st, X, W, shifts, Y, H, Wd,
                                                             pad, by_xcd ? N / 8 : 0, ncb, Cout, probe);
}


// Row-block kernel over input-channel chunks, for 3x3 stride-1 layers whose
// Cin (a multiple of CK = 64) is too deep to stage whole.  The workgroup
// owns an output block as conv2d_i8_rows does (ROWS rows x BW columns x WCO
// channels; BW = 32 for narrow layers), its 8 waves each 32 pixels x 32*NJ
// channels (NJ MFMAs share each X fragment, so NJ = 2 reads 3/4 of the LDS
// bytes per MAC of NJ = 1), and walks Cin in chunks of 64 channels: each
// chunk stages what conv2d_i8_rows<3,3,64> stages for its whole input (the
// ROWS+2 padded input rows, 64 channels of them, and the WCO channels'
// 3x3x64 weights), into one of two LDS buffers.  The next chunk's loads go
// out into registers before the current chunk's 18*NJ MFMAs per wave run
// from the other buffer, and are written to LDS one load at a time between
// the second half of those MFMAs, so the writes run under the MFMAs and one
// workgroup barrier per chunk suffices.  The launcher keeps X, W and Y below
// 2^31 bytes (the Y store offset is 32-bit), and the accumulators start at
// the rounding term: |acc| <= 9*Cin*2^14 < 2^30 for Cin <= 4096.
template <int ROWS, int WCO, int NJ, int BW>
__global__ __launch_bounds__(512) void conv2d_i8_rowsk(const int8_t* __restrict__ X, const int8_t* __restrict__ W,
                                                       const uint8_t* __restrict__ shifts, int8_t* __restrict__ Y,
                                                       int H, int Wd, int Cin, int Cout, int pad, int Ho, int Wo,
                                                       int xg, int ncb) {
  constexpr int CK = 64;
  using G = RowsGeom<3, 3, CK, ROWS, WCO, BW>;
  constexpr int BUF = G::X_BYTES + G::W_BYTES;  // one chunk's X and W
  constexpr int WPC = 9 * CK / 16;              // 16-byte W chunks per output channel per input chunk
  static_assert(2 * BUF + G::Y_BYTES <= 163840, "chunked row-block conv LDS budget");
  constexpr int NPB = BW / 32;  // 32-pixel halves of a block row
  static_assert(ROWS * NPB * (WCO / (32 * NJ)) == 8, "8 waves of 32 pixels x 32*NJ channels");
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * BUF + G::Y_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  int n, rb, cb;
  if (xg) {
    rb = blockIdx.y;
    const int z = blockIdx.z;
    cb = xg == 1 ? z : z / xg;
    n = 8 * (z - cb * xg) + blockIdx.x;
  } else {
    rb = blockIdx.x;
    cb = blockIdx.y;
    n = blockIdx.z;
  }
  int wc0 = 0;
  if (ncb > 1) {
    const int cbk = rb % ncb;
    rb /= ncb;
    wc0 = cbk * BW;
  }
  const int ho0 = rb * ROWS;
  const int co0 = cb * WCO;
  int8_t* const ys = smem + 2 * BUF;
  // wave: output row rr, pixels 32pb .. +32, channels 32*NJ*wj .. +32*NJ
  constexpr int NWJ = WCO / (32 * NJ);
  const int wj = wave % NWJ, pb = (wave / NWJ) % NPB, rr = wave / (NPB * NWJ);

  // Staging map of conv2d_i8_rows<3,3,64>, with each source offset computed
  // once; chunk kc adds kc * CK.  Positions outside the image load the
  // nearest pixel inside it and are zeroed when written to LDS.  The offsets
  // are 64-bit: formed in 32 bits, each became a v_mad_u64_u32 whose unused
  // high addend half the compiler took from any register, at times one still
  // waiting for a load, so the next load waited for it.
  const int xc = tid % G::NCH, xcol = (tid / G::NCH) % BW, xrow = tid / (G::NCH * BW);
  const int et = tid % G::XE;
  const int ec = et % G::NCH, ecol = BW + (et / G::NCH) % (G::XC - BW), erow = et / (G::NCH * (G::XC - BW));
  auto x_src = [&](int row, int col, int c, bool& in) -> uint64_t {
    const int hi = ho0 + row - pad, wi = wc0 + col - pad;
    in = (unsigned)hi < (unsigned)H && (unsigned)wi < (unsigned)Wd;
    const int hc = min(max(hi, 0), H - 1), wcl = min(max(wi, 0), Wd - 1);
    return (uint64_t)((n * H + hc) * Wd + wcl) * (uint64_t)Cin + 16 * c;
  };
  auto xrow_of = [&](int u) { return min(G::RPP * u + xrow, G::XR - 1); };
  auto wq_of = [&](int u) { return u < G::WQ - 1 ? tid + 512 * u : 512 * (G::WQ - 1) + tid % G::WREM; };
  uint64_t xo[G::XQ], eo, wo[G::WQ];
  bool xin[G::XQ], ein;
#pragma unroll
  for (int u = 0; u < G::XQ; ++u) xo[u] = x_src(xrow_of(u), xcol, xc, xin[u]);
  eo = x_src(erow, ecol, ec, ein);
#pragma unroll
  for (int u = 0; u < G::WQ; ++u) {
    const int q = wq_of(u), co = q / WPC, rem = q % WPC;  // rem: tap (rem / 4) x 16-byte chunk (rem % 4)
    wo[u] = (uint64_t)(co0 + co) * (uint64_t)(9 * Cin) + (uint64_t)((rem >> 2) * Cin + 16 * (rem & 3));
  }
  v4i xv[G::XQ], xe, wv[G::WQ];
  auto load = [&](int kc) {
    const uint64_t k0 = (uint64_t)(kc * CK);
#pragma unroll
    for (int u = 0; u < G::XQ; ++u) xv[u] = MIAIE_LD(reinterpret_cast<const v4i*>(X + xo[u] + k0));
    xe = MIAIE_LD(reinterpret_cast<const v4i*>(X + eo + k0));
#pragma unroll
    for (int u = 0; u < G::WQ; ++u) wv[u] = MIAIE_LD(reinterpret_cast<const v4i*>(W + wo[u] + k0));
  };
  // Write load i (in issue order: X passes, the last columns, W passes) of
  // the staged chunk into LDS buffer buf.
  constexpr int NPUT = G::XQ + 1 + G::WQ;
  auto put_one = [&](int8_t* buf, int i) {
    auto x_put = [&](int row, int col, int c, bool in, v4i v) {
      *reinterpret_cast<v4i*>(buf + (row * G::XC + col) * CK + ((c ^ xswz<CK>(col)) << 4)) = in ? v : v4i{0};
    };
    if (i < G::XQ) {
      x_put(xrow_of(i), xcol, xc, xin[i], xv[i]);
    } else if (i == G::XQ) {
      x_put(erow, ecol, ec, ein, xe);
    } else {
      const int u = i - G::XQ - 1, q = wq_of(u);
      *reinterpret_cast<v4i*>(buf + G::X_BYTES + (q / WPC) * G::WP + 16 * (q % WPC)) = wv[u];
    }
  };
  static_assert(NPUT <= G::T, "one staged load written per k-step at most");

  uint32_t sh4[NJ][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      sh4[j][g] = MIAIE_LD(reinterpret_cast<const uint32_t*>(shifts + co0 + 32 * (NJ * wj + j) + 8 * g + 4 * fh));
  const int nk = Cin / CK;
  load(0);
  __builtin_amdgcn_sched_barrier(0);
  v16i acc[NJ];
  int smin = 31;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int sc = (sh4[j][g] >> (8 * tt)) & 31;
        acc[j][4 * g + tt] = (int)((1u << sc) >> 1);
        smin = min(smin, sc);
      }
  const bool hi_form = __builtin_amdgcn_ballot_w64(smin < 8) == 0;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NPUT; ++i) put_one(smem, i);
  if (nk > 1) load(1);
  __syncthreads();

  const int px = 32 * pb + fr;
  // One chunk's MFMAs from buffer xs; with PUT, the staged next chunk goes
  // into buffer nbuf, load i after k-step T - NPUT + i (the loads have had
  // the first half of the chunk to land).  nbuf was last read in the chunk
  // before, which the barrier that ended it retired.
  auto chunk = [&](auto put_next, const int8_t* xs, int8_t* nbuf) {
    constexpr bool PUT = decltype(put_next)::value;
    const int8_t* const wrow = xs + G::X_BYTES + (32 * NJ * wj + fr) * G::WP + 16 * fh;
    // fragments of k-step t in set t % 2.  At NJ = 2, step t+1's are read
    // before step t's MFMAs issue, so an LDS read's latency passes under the
    // MFMAs (2-4% faster); at NJ = 1 the compiler's own order measured 1-2%
    // faster (fewer registers, two waves per SIMD hide more).
    constexpr bool AHEAD = NJ > 1;
    v4i xf[2], wf[2][NJ];
    auto read = [&](int t) {
      const int cib = t % (CK / 32), rs = t / (CK / 32);
      const int r = rs / 3, s = rs % 3;
      const int col = px + s, f = t & 1;
      xf[f] = *reinterpret_cast<const v4i*>(xs + ((rr + r) * G::XC + col) * CK +
                                            (((2 * cib + fh) ^ xswz<CK>(col)) << 4));
#pragma unroll
      for (int j = 0; j < NJ; ++j) wf[f][j] = *reinterpret_cast<const v4i*>(wrow + 32 * j * G::WP + 32 * t);
    };
    if constexpr (AHEAD) read(0);
#pragma unroll
    for (int t = 0; t < G::T; ++t) {
      if constexpr (AHEAD) {
        if (t + 1 < G::T) read(t + 1);
        __builtin_amdgcn_sched_barrier(0);
      } else {
        read(t);
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[t & 1][j], xf[t & 1], acc[j], 0, 0, 0);
      if constexpr (PUT) {
        if (t >= G::T - NPUT) put_one(nbuf, t - (G::T - NPUT));
      }
    }
  };
  for (int kc = 0; kc + 1 < nk; ++kc) {
    chunk(std::true_type{}, smem + (kc & 1) * BUF, smem + ((kc + 1) & 1) * BUF);
    if (kc + 2 < nk) load(kc + 2);
    __syncthreads();
  }
  chunk(std::false_type{}, smem + ((nk - 1) & 1) * BUF, nullptr);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    rows_epilogue<G>(acc[j], sh4[j], hi_form, ys, rr, pb, NJ * wj + j, fr, fh, lane, n, ho0, wc0, co0, Ho, Wo, Cout, Y);
}

// Grid and launch of the chunked row-block kernel (shapes already checked by
// the caller: deep_ok in conv2d_kernel_for).
template <int ROWS, int WCO, int NJ, int BW>
inline hipError_t launch_rowsk_as(int device, hipStream_t st, const int8_t* X, const int8_t* W, const uint8_t* shifts,
                                  int8_t* Y, int N, int H, int Wd, int Cin, int Cout, int pad, int Ho, int Wo) {
  const int ncb = (Wo + BW - 1) / BW;
  const unsigned rbs = (unsigned)((Ho + ROWS - 1) / ROWS * ncb), cbs = (unsigned)(Cout / WCO);
  const bool by_xcd = N % 8 == 0 && rbs <= 65535 && (size_t)(N / 8) * cbs <= 65535;
  const dim3 grid = by_xcd ? dim3(8, rbs, (unsigned)(N / 8) * cbs) : dim3(rbs, cbs, (unsigned)N);
  return launch<conv2d_i8_rowsk<ROWS, WCO, NJ, BW>>(device, grid, dim3(512), 0, st, X, W, shifts, Y, H, Wd, Cin, Cout,
                                                    pad, Ho, Wo, by_xcd ? N / 8 : 0, ncb);
}


}  // namespace conv
}  // namespace miaie
