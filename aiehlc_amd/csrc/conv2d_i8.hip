// int8 conv2d (NHWC x OHWI -> NHWC) with a per-output-channel requantize
// epilogue, as an im2col-free implicit GEMM on gfx950 MFMA.
//
// The reference's conv exists only as the generated control code of an AIE
// graph (thirdparty/adf/aie_control.cpp:854-1524: 8 `conv` kernels with
// ping/pong activation windows); no kernel source ships.  Semantics are the
// benchmark's: zero padding, stride, int32 accumulation, then
// y = sat_int8((acc + 2^(s_c-1)) >> s_c) per output channel c.
//
// GEMM view: rows = output pixels (n, ho, wo), columns = output channels,
// k = (r, s, ci).  A workgroup owns 64 consecutive pixels x 64 channels.
// Each of its 4 waves takes every 4th k-step of 32 (one (r, s, ci-block)),
// loading X and W fragments straight from global memory in MFMA operand
// layout (W rows are k-contiguous in OHWI; X pixels are ci-contiguous in
// NHWC), so no im2col buffer and no LDS staging of the operands.  The four
// partial 64x64 int32 tiles are summed through LDS, requantized and written
// as one contiguous 4 KiB run of NHWC output.
//
// Split K: when the tiles cover at most a third of the CUs (the deep layers
// of a CNN: few output pixels, long k = 9 * Cin), each tile's k-steps are divided
// among ksplit workgroups (grid.z), which write int32 partial sums to the
// context's workspace; conv2d_i8_splitk_reduce adds them and requantizes.
// The two kernels are ordered by the stream, so no atomics are involved and
// the sums are exact in any order.
#include <algorithm>

#include "conv2d_i8_rows.hpp"
#include "gfx950_ops.hpp"
#include "miaie_internal.hpp"

namespace {

__device__ __forceinline__ int requant1(int acc, int s) {
  int q = s ? (acc >> s) + ((acc >> (s - 1)) & 1) : acc;
  return min(max(q, -128), 127);
}

constexpr int PIX = 64;    // pixels per workgroup
constexpr int COB = 64;    // output channels per workgroup
constexpr int BATCH = 6;   // k-steps whose fragments are in flight per wave

// PARTIAL: k-steps [T z / ksplit, T (z+1) / ksplit) of the tile, z =
// blockIdx.z, summed into psum[z][pixel][channel] (int32, no requantize).
template <bool PARTIAL>
__global__ __launch_bounds__(256) void conv2d_i8_igemm(
    const int8_t* __restrict__ X, const int8_t* __restrict__ W, const uint8_t* __restrict__ shifts,
    int8_t* __restrict__ Y, int32_t* __restrict__ psum, int N, int H, int Wd, int Cin, int Cout, int R, int S,
    int stride, int pad, int Ho, int Wo, int ksplit) {
  __shared__ __attribute__((aligned(16))) int32_t part[4][PIX * COB];  // 64 KiB

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  const int P = N * Ho * Wo;
  const int p0 = blockIdx.x * PIX;
  const int co0 = blockIdx.y * COB;

  // the two pixels this lane feeds (one per 32-pixel block)
  int pn[2], phb[2], pwb[2];
  bool pvalid[2];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int p = p0 + 32 * pb + fr;
    pvalid[pb] = p < P;
    const int pp = pvalid[pb] ? p : 0;
    const int wo = pp % Wo;
    const int t = pp / Wo;
    const int ho = t % Ho;
    pn[pb] = t / Ho;
    phb[pb] = ho * stride - pad;
    pwb[pb] = wo * stride - pad;
  }
  const int KW = R * S * Cin;  // weight row length (OHWI)
  const int8_t* wrow[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) wrow[cb] = W + (size_t)(co0 + 32 * cb + fr) * KW + 16 * fh;

  const int CBI = Cin / 32;
  const int T = R * S * CBI;
  const int tb = PARTIAL ? (int)((long long)T * blockIdx.z / ksplit) : 0;
  const int te = PARTIAL ? (int)((long long)T * (blockIdx.z + 1) / ksplit) : T;

  v16i acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = v16i{0};

  for (int t0 = tb + wave; t0 < te; t0 += 4 * BATCH) {
    v4i xf[BATCH][2], wf[BATCH][2];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int t = t0 + 4 * u;
      if (t < te) {
        const int rs = t / CBI, cib = t - rs * CBI;
        const int r = rs / S, s = rs - r * S;
        const int koff = rs * Cin + cib * 32;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) wf[u][cb] = MIAIE_LD(reinterpret_cast<const v4i*>(wrow[cb] + koff));
#pragma unroll
        for (int pb = 0; pb < 2; ++pb) {
          const int hi = phb[pb] + r, wi = pwb[pb] + s;
          const bool ok = pvalid[pb] && hi >= 0 && hi < H && wi >= 0 && wi < Wd;
          const int8_t* src = X + (((size_t)pn[pb] * H + hi) * Wd + wi) * Cin + cib * 32 + 16 * fh;
          xf[u][pb] = ok ? MIAIE_LD(reinterpret_cast<const v4i*>(src)) : v4i{0};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      if (t0 + 4 * u < te) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
          for (int pb = 0; pb < 2; ++pb)
            acc[cb][pb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[u][cb], xf[u][pb], acc[cb][pb], 0, 0, 0);
      }
    }
  }

  // acc[cb][pb][4g + t]: channel co = 32cb + 8g + 4*(lane/32) + t, pixel p = 32pb + lane%32.
  // Partial tile layout: [pixel][16-byte channel quad, XOR pixel%16].
  int32_t* mine = part[wave];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int p = 32 * pb + fr;
        const int cq = (32 * cb + 8 * g + 4 * fh) >> 2;
        v4i v = {acc[cb][pb][4 * g], acc[cb][pb][4 * g + 1], acc[cb][pb][4 * g + 2], acc[cb][pb][4 * g + 3]};
        *reinterpret_cast<v4i*>(mine + p * COB + ((cq ^ (p & 15)) << 2)) = v;
      }
  __syncthreads();

  // thread -> pixel tid/4, channels 16*(tid%4) .. +16
  const int p = tid >> 2, c16 = (tid & 3) * 16;
  if (p0 + p >= P) return;
  int sum[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int cq = (c16 >> 2) + q;
    v4i s = v4i{0};
#pragma unroll
    for (int w = 0; w < 4; ++w) s += *reinterpret_cast<const v4i*>(part[w] + p * COB + ((cq ^ (p & 15)) << 2));
    sum[4 * q] = s[0];
    sum[4 * q + 1] = s[1];
    sum[4 * q + 2] = s[2];
    sum[4 * q + 3] = s[3];
  }
  if constexpr (PARTIAL) {
    int32_t* const dst = psum + ((size_t)blockIdx.z * P + p0 + p) * Cout + co0 + c16;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      MIAIE_ST(reinterpret_cast<v4i*>(dst + 4 * q), (v4i{sum[4 * q], sum[4 * q + 1], sum[4 * q + 2], sum[4 * q + 3]}));
    return;
  }
  uint32_t out[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int c = co0 + c16 + 4 * q + t;
      v |= (uint32_t)(requant1(sum[4 * q + t], MIAIE_LD(shifts + c)) & 0xFF) << (8 * t);
    }
    out[q] = v;
  }
  MIAIE_ST(reinterpret_cast<uint4*>(Y + (size_t)(p0 + p) * Cout + co0 + c16), make_uint4(out[0], out[1], out[2], out[3]));
}

// ------------------------------------------------------------ taps kernel
// LDS-staged implicit GEMM for Cin a multiple of 128 and Cout of 64 (the
// deep layers of a CNN, which the row-block kernel does not take).  The
// workgroup tile is 64 output pixels x 64 output channels, as in
// conv2d_i8_igemm, but the k loop runs over stages of one filter tap (r, s)
// and CK = 128 input channels, and each stage's two operands (the 64
// pixels' 128 channels at that tap, and the 64 channels' weights for it) are
// copied into an NS-stage LDS ring by global_load_lds_dwordx4 with eight
// lanes per 128-byte row: a copy instruction touches 8 cache lines, against
// 32 for a fragment loaded straight into MFMA layout.  The tap position is
// walked forward without division (a runtime division per stage cost more
// than the copies).  At Cin = 64 (two MFMAs per wave per stage) the per-stage
// barrier and waits outweigh this, and conv2d_i8_igemm is faster.  Positions
// outside the image are copied from a clamped address and their X fragments
// zeroed when read.  Each of the 4 waves owns 32 pixels x 32 channels (one
// v_mfma_i32_32x32x32_i8 accumulator), so there is no cross-wave reduction;
// with split K (grid.z) the tile's stages are divided among workgroups whose
// int32 partials conv2d_i8_splitk_reduce adds.
template <int TP, int TC>
struct TapsGeom {
  static constexpr int CK = 128;                    // input channels per stage
  static constexpr int NS = TP * TC > 64 * 64 ? 4 : 8;  // LDS stages in the ring
  static constexpr int CPR = CK / 16;               // 16-byte chunks per staged row
  static constexpr int XB = TP * CK, WB = TC * CK;  // the two operands of one stage
  static constexpr int STAGE = XB + WB;             // X rows, then W rows
  static constexpr int CPX = XB / 4096, CPW = WB / 4096;  // copies per thread per stage (256 x 16 bytes each)
  static constexpr int CPS = CPX + CPW;
  static constexpr int KS = CK / 32;                // 32-wide k-steps per stage
  static constexpr int NI = TP / 64, NJ = TC / 64;  // 32x32 blocks per wave (4 waves, 2 x 2)
  static constexpr int YP = TC / 2 + 16;            // epilogue: LDS pitch of a pixel's TC/2 output channels
  static constexpr int YW = TP / 2 * YP;            // one wave's output block
  static constexpr int LDS = NS * STAGE + 4 * YW;
  static_assert(CPX >= 1 && CPW >= 1 && NI >= 1 && NJ >= 1 && LDS <= 163840, "taps kernel staging");
  static_assert((NS - 2) * CPS <= 63, "copies in flight fit the vmcnt counter");
};

// Chunk swizzle of a staged 128-byte row: the 16 rows one half-wave
// fragment read touches land on distinct bank groups.
__device__ __forceinline__ int taps_swz(int row) { return (row >> 1) & 7; }

// Workgroup tile TP output pixels x TC output channels (64 x 64 for small
// grids, 128 x 128 otherwise); each wave owns TP/2 x TC/2, NI x NJ blocks of
// 32 x 32.
template <int TP, int TC, bool PARTIAL>
__global__ __launch_bounds__(256) void conv2d_i8_taps(
    const int8_t* __restrict__ X, const int8_t* __restrict__ W, const uint8_t* __restrict__ shifts,
    int8_t* __restrict__ Y, int32_t* __restrict__ psum, int N, int H, int Wd, int Cin, int Cout, int R, int S,
    int stride, int pad, int Ho, int Wo, int ksplit) {
  using G = TapsGeom<TP, TC>;
  constexpr int CK = G::CK, NI = G::NI, NJ = G::NJ;
  __shared__ __attribute__((aligned(1024))) int8_t lds[G::LDS];
  const uint32_t lds0 = miaie::dev::lds_addr(lds);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int pb = wave & 1, cb = wave >> 1;  // this wave's pixel half and channel half
  const int P = N * Ho * Wo;
  const int p0 = blockIdx.x * TP, co0 = blockIdx.y * TC;
  const int CB = Cin / CK, T = R * S * CB;
  const int sb = PARTIAL ? (int)((long long)T * blockIdx.z / ksplit) : 0;
  const int nst = (PARTIAL ? (int)((long long)T * (blockIdx.z + 1) / ksplit) : T) - sb;
  const int KW = R * S * Cin;

  // ---- copy geometry.  Copy i of wave w moves 1 KiB block q = 4i + w of an
  // operand: rows 8q + lane / 8, logical chunk (lane % 8) ^ swz(row), landing
  // at LDS byte 1024 q + 16 lane of the operand.
  int xhb[G::CPX], xwb[G::CPX];
  uint32_t xbase[G::CPX], wbase[G::CPW];
  const uint32_t rowx = (uint32_t)Wd * Cin;  // bytes per input row
#pragma unroll
  for (int i = 0; i < G::CPX; ++i) {
    const int row = (4 * i + wave) * 8 + lane / G::CPR;
    const int gc = (lane % G::CPR) ^ taps_swz(row);
    const int p = min(p0 + row, P - 1);  // rows past the last pixel copy a real one (never stored)
    const int wo = p % Wo, t = p / Wo;
    xhb[i] = (t % Ho) * stride - pad;
    xwb[i] = wo * stride - pad;
    xbase[i] = (uint32_t)((t / Ho) * H) * rowx + (uint32_t)(16 * gc);
  }
#pragma unroll
  for (int i = 0; i < G::CPW; ++i) {
    const int row = (4 * i + wave) * 8 + lane / G::CPR;
    wbase[i] = (uint32_t)((co0 + row) * KW + 16 * ((lane % G::CPR) ^ taps_swz(row)));
  }
  // this lane's fragment pixels (X rows TP/2 pb + 32 i + fr)
  bool pvalid[NI];
  int fhb[NI], fwb[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int pf = p0 + TP / 2 * pb + 32 * i + fr;
    pvalid[i] = pf < P;
    const int pp = pvalid[i] ? pf : 0;
    const int wo = pp % Wo, t = pp / Wo;
    fhb[i] = (t % Ho) * stride - pad;
    fwb[i] = wo * stride - pad;
  }

  // A stage position (filter row r, column s, channel chunk c) walked
  // forward without division.
  struct Tap {
    int r, s, c;
  };
  auto step = [&](Tap& t) {
    if (++t.c == CB) {
      t.c = 0;
      if (++t.s == S) {
        t.s = 0;
        ++t.r;
      }
    }
  };
  Tap at_issue, at_use;
  {
    const int rs = sb / CB;
    at_issue = Tap{rs / S, rs % S, sb % CB};
    at_use = at_issue;
  }
  const miaie::dbg::Span x_span = miaie::dbg::span_of(X), w_span = miaie::dbg::span_of(W);  // (debug build only)
  // copies of the stage at `t` into ring slot `slot`
  auto issue = [&](const Tap& t, int slot) {
    const uint32_t base = lds0 + slot * G::STAGE + 1024 * wave;
    const uint32_t wk = (uint32_t)((t.r * S + t.s) * Cin + t.c * CK), xk = (uint32_t)(t.c * CK);
    // X and W copies alternate (issuing all of one operand first measured 6%
    // slower at 64 x 64)
#pragma unroll
    for (int i = 0; i < (G::CPX > G::CPW ? G::CPX : G::CPW); ++i) {
      if (i < G::CPX) {
        const int hi = min(max(xhb[i] + t.r, 0), H - 1), wi = min(max(xwb[i] + t.s, 0), Wd - 1);
        miaie::dev::gload_lds16(X, xbase[i] + (uint32_t)hi * rowx + (uint32_t)wi * Cin + xk, base + 4096 * i, x_span);
      }
      if (i < G::CPW) miaie::dev::gload_lds16(W, wbase[i] + wk, base + G::XB + 4096 * i, w_span);
    }
  };

  v16i acc[NJ][NI];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[j][i] = v16i{0};
  const int8_t* const wfrag = lds + G::XB + (TC / 2 * cb + fr) * CK;
  const int8_t* const xfrag = lds + (TP / 2 * pb + fr) * CK;
  // the swizzle of rows r and r + 32 is the same: one per operand
  const int wsw = taps_swz(TC / 2 * cb + fr), xsw = taps_swz(TP / 2 * pb + fr);

#pragma unroll
  for (int i = 0; i < G::NS - 1; ++i)
    if (i < nst) {
      issue(at_issue, i);
      step(at_issue);
    }
  for (int s = 0; s < nst; ++s) {
    // this wave's copies of stage s have landed once only the stages issued
    // after it (at most NS - 2) are in flight; the barrier publishes everyone's
    // and frees the slot of stage s - 1 for stage s + NS - 1
    miaie::dev::wait_tiles_behind<G::CPS, G::NS - 1>(min(G::NS - 2, nst - 1 - s) + 1);
    miaie::dev::barrier();
    if (s + G::NS - 1 < nst) {
      issue(at_issue, (s + G::NS - 1) % G::NS);
      step(at_issue);
    }
    bool xin[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
      xin[i] = pvalid[i] && (unsigned)(fhb[i] + at_use.r) < (unsigned)H && (unsigned)(fwb[i] + at_use.s) < (unsigned)Wd;
    step(at_use);
    const int slot = (s % G::NS) * G::STAGE;
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) {
      const int cw = ((2 * ks + fh) ^ wsw) << 4, cx = ((2 * ks + fh) ^ xsw) << 4;
      v4i wf[NJ], xf[NI];
#pragma unroll
      for (int j = 0; j < NJ; ++j) wf[j] = *reinterpret_cast<const v4i*>(wfrag + slot + 32 * CK * j + cw);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        xf[i] = *reinterpret_cast<const v4i*>(xfrag + slot + 32 * CK * i + cx);
        xf[i] = xin[i] ? xf[i] : v4i{0};
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < NI; ++i) acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[j], xf[i], acc[j][i], 0, 0, 0);
    }
  }

  // acc[j][i][4g + t]: channel TC/2 cb + 32j + 8g + 4fh + t, pixel TP/2 pb + 32i + fr
  if constexpr (PARTIAL) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int pf = p0 + TP / 2 * pb + 32 * i + fr;
      if (!pvalid[i]) continue;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        int32_t* const dst = psum + ((size_t)blockIdx.z * P + pf) * Cout + co0 + TC / 2 * cb + 32 * j + 4 * fh;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          MIAIE_ST(reinterpret_cast<v4i*>(dst + 8 * g),
                   (v4i{acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]}));
      }
    }
    return;
  }
  // requantize into this wave's own LDS block (TP/2 pixels x TC/2 channels),
  // then 16-byte stores of whole pixel runs (an LDS wait, no workgroup barrier)
  int8_t* const yb = lds + G::NS * G::STAGE + wave * G::YW;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int cl = 32 * j + 4 * fh;  // channel within the wave's half
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t sh = MIAIE_LD(reinterpret_cast<const uint32_t*>(shifts + co0 + TC / 2 * cb + cl + 8 * g));
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          v |= (uint32_t)(requant1(acc[j][i][4 * g + t], (sh >> (8 * t)) & 0xFF) & 0xFF) << (8 * t);
        *reinterpret_cast<uint32_t*>(yb + (32 * i + fr) * G::YP + cl + 8 * g) = v;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
  __builtin_amdgcn_wave_barrier();
  constexpr int CPP = TC / 32;  // 16-byte chunks per pixel of the wave's half
#pragma unroll
  for (int it = 0; it < TP / 2 * CPP / 64; ++it) {
    const int flat = 64 * it + lane, sp = flat / CPP, ch = flat % CPP;
    const int p = p0 + TP / 2 * pb + sp;
    if (p < P) {
      const v4i v = *reinterpret_cast<const v4i*>(yb + sp * G::YP + 16 * ch);
      MIAIE_ST(reinterpret_cast<v4i*>(Y + (size_t)p * Cout + co0 + TC / 2 * cb + 16 * ch), v);
    }
  }
}

// The split-K epilogue: part[z][e] summed over z < ksplit for element e =
// pixel * Cout + channel, then the per-channel requantize.  One thread per 16
// channels of one pixel (Cout % 64 == 0).
__global__ __launch_bounds__(256) void conv2d_i8_splitk_reduce(const int32_t* __restrict__ part,
                                                               const uint8_t* __restrict__ shifts,
                                                               int8_t* __restrict__ Y, long long PC, int Cout,
                                                               int ksplit) {
  const long long e = ((long long)blockIdx.x * 256 + threadIdx.x) * 16;
  if (e >= PC) return;
  v4i s[4] = {v4i{0}, v4i{0}, v4i{0}, v4i{0}};
  for (int z = 0; z < ksplit; ++z) {
    const int32_t* src = part + (size_t)z * PC + e;
#pragma unroll
    for (int q = 0; q < 4; ++q) s[q] += MIAIE_LD(reinterpret_cast<const v4i*>(src + 4 * q));
  }
  const int c0 = (int)(e % Cout);
  uint32_t out[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) v |= (uint32_t)(requant1(s[q][t], MIAIE_LD(shifts + c0 + 4 * q + t)) & 0xFF) << (8 * t);
    out[q] = v;
  }
  MIAIE_ST(reinterpret_cast<uint4*>(Y + e), make_uint4(out[0], out[1], out[2], out[3]));
}

// Any-shape fallback: one thread per output element.
__global__ __launch_bounds__(256) void conv2d_i8_direct(const int8_t* __restrict__ X, const int8_t* __restrict__ W,
                                                        const uint8_t* __restrict__ shifts, int8_t* __restrict__ Y,
                                                        int N, int H, int Wd, int Cin, int Cout, int R, int S,
                                                        int stride, int pad, int Ho, int Wo) {
  const size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const size_t total = (size_t)N * Ho * Wo * Cout;
  if (idx >= total) return;
  const int co = (int)(idx % Cout);
  size_t t = idx / Cout;
  const int wo = (int)(t % Wo);
  t /= Wo;
  const int ho = (int)(t % Ho);
  const int n = (int)(t / Ho);
  uint32_t acc = 0;
  for (int r = 0; r < R; ++r) {
    const int hi = ho * stride + r - pad;
    if (hi < 0 || hi >= H) continue;
    for (int s = 0; s < S; ++s) {
      const int wi = wo * stride + s - pad;
      if (wi < 0 || wi >= Wd) continue;
      const int8_t* x = X + (((size_t)n * H + hi) * Wd + wi) * Cin;
      const int8_t* w = W + (((size_t)co * R + r) * S + s) * Cin;
      for (int ci = 0; ci < Cin; ++ci) acc += (uint32_t)((int)MIAIE_LD(x + ci) * (int)MIAIE_LD(w + ci));
    }
  }
  MIAIE_ST(Y + idx, (int8_t)requant1((int)acc, MIAIE_LD(shifts + co)));
}

}  // namespace

namespace miaie {

// Row-block shape: 4 output rows x 32 channels; 2 rows x 64 channels where
// Cout is a multiple of 64 and there are fewer than 8 output rows (a 4-row
// block would leave more of its rows empty).  Both shapes run the same
// number of workgroups; 4 x 32 stages 1.5 input rows per output row against
// 2, and half the weights, in fewer load instructions per workgroup, and
// measured 1-5% faster per launch at Cin 64 and 128 (56x56 and 112x112,
// Cout 64 and 128) and within 0.5% at Cin 32.
static bool rows_tall(int Ho, int Cout) { return Cout % 64 != 0 || Ho >= 8; }

template <int CIN>
static int launch_rows(miaie_ctx* ctx, const int8_t* X, const int8_t* W, const uint8_t* shifts, int8_t* Y, int N,
                       int H, int Wd, int Cout, int pad, int Ho, int Wo) {
  const hipError_t e =
      rows_tall(Ho, Cout)
          ? conv::launch_rows_as<CIN, 4, 32, false>(ctx->device, ctx->stream, X, W, shifts, Y, N, H, Wd, Cout, pad, Ho, Wo)
          : conv::launch_rows_as<CIN, 2, 64, false>(ctx->device, ctx->stream, X, W, shifts, Y, N, H, Wd, Cout, pad, Ho, Wo);
  return check_launch(ctx, e, "conv2d_i8_rows");
}

// Workgroups per tile of the implicit-GEMM kernels (1: no split).  Split
// when at least 3 workgroups per tile fit on the CUs (a 2-way split measured
// no faster: the reduce kernel's launch costs what the halved k-chain
// saves), into at most 8 and at most cus / tiles parts, each keeping at least
// min_per_split k-steps, with the partial sums inside the context's
// workspace of work_bytes.
static int conv_ksplit(size_t tiles, int T, int min_per_split, size_t elems, int cus, size_t work_bytes) {
  if (tiles * 3 > (size_t)cus) return 1;
  int ks = (int)std::min<size_t>((size_t)cus / tiles, 8);
  ks = std::min(ks, T / min_per_split);
  while (ks > 1 && (size_t)ks * elems * sizeof(int32_t) > work_bytes) --ks;
  return ks > 1 ? ks : 1;
}

// Estimated time of a launch (microseconds), for choosing between the
// chunked row-block kernel and the taps kernel: rounds of one workgroup per
// CU times a per-workgroup time fitted to back-to-back launches on MI355X
// (8x{56,28,14,7}^2 layers, Cin and Cout 256 and 512, 1x224^2x256 and
// 32x{28,14}^2 layers): a fixed start and end cost plus a cost per 64-channel
// chunk or per taps stage.
static double launch_rounds(size_t wgs, int cus) { return (double)((wgs + cus - 1) / cus); }

// conv2d_i8_rowsk<rows, 32*nj, nj, bw>: blocks of bw columns (64, or 32 for
// narrow layers) x rows = 256/bw rows, 8 waves of 32 pixels x 32*nj channels
struct RowsDeepTile {
  int nj, bw;
};
static double rows_deep_us(int N, int Ho, int Wo, int Cin, int Cout, RowsDeepTile t, int cus) {
  const int rows = 256 / t.bw;
  const size_t wgs = (size_t)N * ((Ho + rows - 1) / rows) * ((Wo + t.bw - 1) / t.bw) * (size_t)(Cout / (32 * t.nj));
  const int nk = Cin / 64;
  return launch_rounds(wgs, cus) * (t.nj == 2 ? 3.5 + 1.68 * nk : 2.8 + 1.0 * nk);
}

// Tile of the chunked row-block kernel with the lowest estimate: 32 x 64
// waves (two MFMAs per pixel fragment, 3/4 of the LDS reads per MAC) unless
// they leave so few workgroups that 32 x 32 finishes first; 32-column blocks
// where 64 would leave most columns empty (Wo <= 32, or just above 64).
static RowsDeepTile rows_deep_tile(int N, int Ho, int Wo, int Cin, int Cout, int cus) {
  RowsDeepTile best{1, 64};
  double best_us = rows_deep_us(N, Ho, Wo, Cin, Cout, best, cus);
  for (RowsDeepTile t : {RowsDeepTile{2, 64}, RowsDeepTile{2, 32}, RowsDeepTile{1, 32}}) {
    if (t.nj == 2 && Cout % 64) continue;
    const double us = rows_deep_us(N, Ho, Wo, Cin, Cout, t, cus);
    if (us < best_us) best = t, best_us = us;
  }
  return best;
}

// conv2d_i8_rows<3,3,128,...> (98 KiB of LDS at 4 rows x 32 channels, 116 KiB
// at 2 x 64: one workgroup per CU), 3.5-3.6 us per workgroup (8x112x112x128
// in 7 rounds, 24.4-25.1 us)
static double rows128_us(int N, int Ho, int Wo, int Cout, int cus) {
  const int rows = rows_tall(Ho, Cout) ? 4 : 2, wco = rows_tall(Ho, Cout) ? 32 : 64;
  const size_t wgs = (size_t)N * ((Ho + rows - 1) / rows) * ((Wo + conv::PB - 1) / conv::PB) * (size_t)(Cout / wco);
  return launch_rounds(wgs, cus) * 3.57;
}

// conv2d_i8_taps as its launcher runs it: 128 x 128 tiles when they fill a
// round of CUs, else 64 x 64 split over k; a stage is one tap x 128 channels.
static double taps_us(size_t P, int Cin, int Cout, int R, int S, int cus, size_t work_bytes) {
  const int stages = R * S * (Cin / 128);
  const size_t t128 = ((P + 127) / 128) * (size_t)(Cout / 128);
  if (Cout % 128 == 0 && t128 >= (size_t)cus) return launch_rounds(t128, cus) * (4.0 + 0.69 * stages);
  const size_t t64 = ((P + 63) / 64) * (size_t)(Cout / 64);
  const int ks = conv_ksplit(t64, stages, 4, P * Cout, cus, work_bytes);
  return launch_rounds(t64 * ks, cus) * (2.5 + 0.41 * stages / ks) + (ks > 1 ? 3.0 : 0.0);
}

// The kernel choice weighs estimated times on `cus` compute units: the
// context's count at launch (miaie_plan_set_cus or the device's), and an
// MI355X's 256 for miaie_plan_conv2d_i8, which has no context.
int conv2d_kernel_for(int N, int H, int Wd, int Cin, int Cout, int R, int S, int stride, int pad, bool aligned16,
                      bool shifts_aligned4, int cus) {
  const int Ho = (H + 2 * pad - R) / stride + 1;
  const int Wo = (Wd + 2 * pad - S) / stride + 1;
  const size_t P = (size_t)N * Ho * Wo;
  // Row-block kernel (3x3, stride 1, Cin 32, 64 or 128; rows wider than 64
  // output columns in blocks of 64).  Its offsets are 32-bit: X, Y and W
  // (co0 * R*S*Cin) must each stay below 2^31 bytes, and the channel blocks
  // (>= 32 channels each) fit grid.y.
  const bool rows_ok = stride == 1 && R == 3 && S == 3 && (Cin == 32 || Cin == 64 || Cin == 128) && Cout % 32 == 0 &&
                       aligned16 && shifts_aligned4 && N <= 65535 &&
                       (size_t)N * H * Wd * Cin < ((size_t)1 << 31) && (size_t)N * Ho * Wo * Cout < ((size_t)1 << 31) &&
                       (size_t)Cout * R * S * Cin < ((size_t)1 << 31) && Cout / 32 <= 65535;
  // The same kernel over 64-channel chunks of a deeper Cin (the rounding
  // term in the accumulator start needs 9 * Cin * 2^14 < 2^30).
  const bool deep_ok = stride == 1 && R == 3 && S == 3 && Cin % 64 == 0 && Cin <= 4096 && Cout % 32 == 0 &&
                       aligned16 && shifts_aligned4 && N <= 65535 &&
                       (size_t)N * H * Wd * Cin < ((size_t)1 << 31) && (size_t)N * Ho * Wo * Cout < ((size_t)1 << 31) &&
                       (size_t)Cout * R * S * Cin < ((size_t)1 << 31) && Cout / 32 <= 65535;
  if (rows_ok) {
    // At Cin = 128 both apply: the chunked kernel's 32-column blocks leave
    // fewer empty columns on narrow layers, which pays where the row-block
    // kernel's grid takes more than one round of CUs
    if (Cin == 128 && deep_ok) {
      const RowsDeepTile t = rows_deep_tile(N, Ho, Wo, Cin, Cout, cus);
      if (rows_deep_us(N, Ho, Wo, Cin, Cout, t, cus) < rows128_us(N, Ho, Wo, Cout, cus))
        return MIAIE_CONV_ROWS_DEEP;
    }
    return MIAIE_CONV_ROWS;
  }
  // LDS-staged taps kernel (Cin a multiple of 128, Cout of 64): 32-bit copy
  // offsets, so X and W each stay below 2^31 bytes; 4-byte shift loads.
  const bool taps_ok = Cin % 128 == 0 && Cout % 64 == 0 && aligned16 && shifts_aligned4 &&
                       (size_t)N * H * Wd * Cin < ((size_t)1 << 31) && (size_t)Cout * R * S * Cin < ((size_t)1 << 31) &&
                       P < ((size_t)1 << 31) && Cout / 64 <= 65535;
  if (deep_ok && taps_ok) {
    const RowsDeepTile t = rows_deep_tile(N, Ho, Wo, Cin, Cout, cus);
    return rows_deep_us(N, Ho, Wo, Cin, Cout, t, cus) <=
                   taps_us(P, Cin, Cout, R, S, cus, MIAIE_CTX_WORK_BYTES)
               ? MIAIE_CONV_ROWS_DEEP
               : MIAIE_CONV_TAPS;
  }
  if (deep_ok) return MIAIE_CONV_ROWS_DEEP;
  if (taps_ok) return MIAIE_CONV_TAPS;
  const bool fast = Cin % 32 == 0 && Cout % COB == 0 && aligned16 && P < ((size_t)1 << 31) &&
                    (P + PIX - 1) / PIX < ((size_t)1 << 31) && Cout / COB <= 65535;
  if (fast) return MIAIE_CONV_IGEMM;
  return MIAIE_CONV_DIRECT;
}

int launch_conv2d_i8(miaie_ctx* ctx, const int8_t* X, const int8_t* W, const uint8_t* shifts, int8_t* Y,
                     int N, int H, int Wd, int Cin, int Cout, int R, int S, int stride, int pad) {
  const int Ho = (H + 2 * pad - R) / stride + 1;
  const int Wo = (Wd + 2 * pad - S) / stride + 1;
  const size_t P = (size_t)N * Ho * Wo;
  const int kernel = conv2d_kernel_for(N, H, Wd, Cin, Cout, R, S, stride, pad,
                                       aligned(X, 16) && aligned(W, 16) && aligned(Y, 16), aligned(shifts, 4),
                                       ctx->cus);
  if (kernel == MIAIE_CONV_ROWS) {
    if (Cin == 128) return launch_rows<128>(ctx, X, W, shifts, Y, N, H, Wd, Cout, pad, Ho, Wo);
    if (Cin == 64) return launch_rows<64>(ctx, X, W, shifts, Y, N, H, Wd, Cout, pad, Ho, Wo);
    return launch_rows<32>(ctx, X, W, shifts, Y, N, H, Wd, Cout, pad, Ho, Wo);
  }
  if (kernel == MIAIE_CONV_ROWS_DEEP) {
    const RowsDeepTile t = rows_deep_tile(N, Ho, Wo, Cin, Cout, ctx->cus);
    const int dev = ctx->device;
    hipError_t e;
    if (t.bw == 64 && t.nj == 2)
      e = conv::launch_rowsk_as<4, 64, 2, 64>(dev, ctx->stream, X, W, shifts, Y, N, H, Wd, Cin, Cout, pad, Ho, Wo);
    else if (t.bw == 64)
      e = conv::launch_rowsk_as<4, 32, 1, 64>(dev, ctx->stream, X, W, shifts, Y, N, H, Wd, Cin, Cout, pad, Ho, Wo);
    else if (t.nj == 2)
      e = conv::launch_rowsk_as<8, 64, 2, 32>(dev, ctx->stream, X, W, shifts, Y, N, H, Wd, Cin, Cout, pad, Ho, Wo);
    else
      e = conv::launch_rowsk_as<8, 32, 1, 32>(dev, ctx->stream, X, W, shifts, Y, N, H, Wd, Cin, Cout, pad, Ho, Wo);
    return check_launch(ctx, e, "conv2d_i8_rowsk");
  }
  if (kernel == MIAIE_CONV_TAPS) {
    // 128 x 128 tiles when they fill at least one round of CUs, else 64 x 64
    // (split over k when even those leave most CUs idle)
    const bool big = Cout % 128 == 0 && ((P + 127) / 128) * (size_t)(Cout / 128) >= (size_t)ctx->cus;
    const int tp = big ? 128 : 64;
    const unsigned pxb = (unsigned)((P + tp - 1) / tp), chb = (unsigned)(Cout / tp);
    const int ks = big ? 1 : conv_ksplit((size_t)pxb * chb, R * S * (Cin / 128), 4, P * Cout, ctx->cus,
                                             ctx->work_bytes);
    const int dev = ctx->device;
    if (big) {
      const hipError_t e = launch<conv2d_i8_taps<128, 128, false>>(dev, dim3(pxb, chb, 1), dim3(256), 0, ctx->stream,
                                                                   X, W, shifts, Y, nullptr, N, H, Wd, Cin, Cout, R,
                                                                   S, stride, pad, Ho, Wo, 1);
      return check_launch(ctx, e, "conv2d_i8_taps (128 x 128)");
    }
    if (ks > 1) {
      int32_t* const psum = static_cast<int32_t*>(ctx->work);
      hipError_t e = launch<conv2d_i8_taps<64, 64, true>>(dev, dim3(pxb, chb, (unsigned)ks), dim3(256), 0,
                                                          ctx->stream, X, W, shifts, Y, psum, N, H, Wd, Cin, Cout, R,
                                                          S, stride, pad, Ho, Wo, ks);
      if (int rc = check_launch(ctx, e, "conv2d_i8_taps (split K)")) return rc;
      const long long PC = (long long)(P * Cout);
      e = launch<conv2d_i8_splitk_reduce>(dev, dim3((unsigned)((PC / 16 + 255) / 256)), dim3(256), 0, ctx->stream,
                                          psum, shifts, Y, PC, Cout, ks);
      return check_launch(ctx, e, "conv2d_i8_splitk_reduce");
    }
    const hipError_t e = launch<conv2d_i8_taps<64, 64, false>>(dev, dim3(pxb, chb, 1), dim3(256), 0, ctx->stream, X,
                                                               W, shifts, Y, nullptr, N, H, Wd, Cin, Cout, R, S,
                                                               stride, pad, Ho, Wo, 1);
    return check_launch(ctx, e, "conv2d_i8_taps");
  }
  if (kernel == MIAIE_CONV_IGEMM) {
    const unsigned pxb = (unsigned)((P + PIX - 1) / PIX), chb = (unsigned)(Cout / COB);
    const int ks = conv_ksplit((size_t)pxb * chb, R * S * (Cin / 32), 4 * BATCH, P * Cout, ctx->cus, ctx->work_bytes);
    if (ks > 1) {
      int32_t* const part = static_cast<int32_t*>(ctx->work);
      hipError_t e = launch<conv2d_i8_igemm<true>>(ctx->device, dim3(pxb, chb, (unsigned)ks), dim3(256), 0,
                                                   ctx->stream, X, W, shifts, Y, part, N, H, Wd, Cin, Cout, R, S,
                                                   stride, pad, Ho, Wo, ks);
      if (int rc = check_launch(ctx, e, "conv2d_i8_igemm (split K)")) return rc;
      const long long PC = (long long)(P * Cout);
      e = launch<conv2d_i8_splitk_reduce>(ctx->device, dim3((unsigned)((PC / 16 + 255) / 256)), dim3(256), 0,
                                          ctx->stream, part, shifts, Y, PC, Cout, ks);
      return check_launch(ctx, e, "conv2d_i8_splitk_reduce");
    }
    const hipError_t e = launch<conv2d_i8_igemm<false>>(ctx->device, dim3(pxb, chb), dim3(256), 0, ctx->stream, X, W,
                                                        shifts, Y, nullptr, N, H, Wd, Cin, Cout, R, S, stride, pad,
                                                        Ho, Wo, 1);
    return check_launch(ctx, e, "conv2d_i8_igemm");
  }
  const size_t total = P * Cout;
  const size_t blocks = (total + 255) / 256;
  if (blocks >= ((size_t)1 << 31)) return fail(ctx, MIAIE_EINVAL, "conv2d: output too large for the direct kernel");
  const hipError_t e = launch<conv2d_i8_direct>(ctx->device, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, X, W,
                                                shifts, Y, N, H, Wd, Cin, Cout, R, S, stride, pad, Ho, Wo);
  return check_launch(ctx, e, "conv2d_i8_direct");
}

}  // namespace miaie
