// miaie_examples — the reference's example harness flows on one MI355X.
//
// Each subcommand follows one example program of the reference: allocate
// device memory, move the input in, launch the kernel through the aiehlc
// launch surface (miaie.hpp), wait for it with a deadline, move the output
// back, compute the CPU golden the way the example does and count
// mismatches.  Exit status 0 means the device result matched.
//
//   mm [n] [base]   example/matrixmultiply/aieml_mm.cc:108-249 (n=16, inputs i),
//                   example/other/aieoob.c:80-147 (n=8)
//   perf            example/perf/aieml_perf.cc:105-254 (uint32, inputs i+1)
//   nokernelload    example/nokernelload/aie_nokernelload.cc:106-187 (the
//                   perf<1,1,4,4,256,16,64>(phy, phy_out) launch)
//   multi_tile      example/multi/multi_tile.cpp:65-181 (k1 -> k2, expects 26)
//   seq_full_col    example/multi/seq_full_col.cpp:65-181 (8 stages, expects 23)
//   vek385          example/multi/vek385_verification.cpp:104-157 (3x3 A.A per tile)
//   gemm M N K s    int8 GEMM + requant (benchmark configs), golden on sampled rows
//   conv [reps] [streams]
//                   int8 3x3 conv2d, benchmark config 4, golden on one image;
//                   with reps, then times reps back-to-back calls; with
//                   streams > 1, also reps independent calls dealt round-robin
//                   over that many contexts (one stream and one set of
//                   buffers each), every context's output checked against
//                   the first's
//   mlp M K F N     chained int8 MLP, golden on sampled rows
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "miaie.hpp"

namespace {

using clk = std::chrono::steady_clock;
constexpr int kDeadlineMs = 60000;

double us_since(clk::time_point t0) {
  return std::chrono::duration<double, std::micro>(clk::now() - t0).count();
}

int report(int mismatches, const char* what) {
  if (mismatches == 0)
    printf("%s: CPU result matches the device output.\n", what);
  else
    printf("%s: there were %d mismatches.\n", what, mismatches);
  return mismatches == 0 ? 0 : 1;
}

// SplitMix64 streams used for the benchmark's synthetic tensors
// (state0 = mix(0x5EED0000 + id + gamma); draw i = mix(state0 + (i+1)*gamma)).
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;
uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
std::vector<int8_t> seeded_i8(size_t n, uint64_t id) {
  std::vector<int8_t> v(n);
  const uint64_t s0 = mix(0x5EED0000ull + id + kGamma);
  for (size_t i = 0; i < n; ++i) v[i] = (int8_t)(uint8_t)(mix(s0 + (i + 1) * kGamma) >> 56);
  return v;
}
std::vector<uint8_t> seeded_shifts(size_t n, uint64_t id) {
  std::vector<uint8_t> v(n);
  const uint64_t s0 = mix(0x5EED0000ull + id + kGamma);
  for (size_t i = 0; i < n; ++i) v[i] = (uint8_t)(8 + (mix(s0 + (i + 1) * kGamma) >> 32) % 5);
  return v;
}
int8_t rq(int64_t acc, int s, bool relu) {
  int64_t q = s ? (acc + ((int64_t)1 << (s - 1))) >> s : acc;
  if (relu && q < 0) q = 0;
  return (int8_t)(q > 127 ? 127 : q < -128 ? -128 : q);
}

// ---------------------------------------------------------------- mm / perf
template <int NN, typename T>
int run_window(miaie::Context& ctx, int base, const char* what) {
  constexpr int MAT = NN * NN;
  std::vector<T> vmem(2 * MAT), vmem_out(MAT, 0);
  for (int i = 0; i < 2 * MAT; ++i) vmem[i] = (T)(i + base);
  miaie::Buffer<T> in(ctx, 2 * MAT), out(ctx, MAT);
  out.move_in(vmem_out);
  const auto t0 = clk::now();
  in.move_in(vmem);
  if constexpr (sizeof(T) == 4 && T(-1) < T(0))
    miaie::mm<1, 1, 4, 4, NN, NN, NN>(in.data(), out.data());
  else
    miaie::perf<1, 1, 4, 4, NN, NN, NN>(in.data(), out.data());
  if (!ctx.wait(kDeadlineMs)) {
    printf("%s: kernel did not finish within %d ms\n", what, kDeadlineMs);
    return 2;
  }
  out.move_out(vmem_out.data(), MAT);
  printf("Output took %.2f us.\n", us_since(t0));
  // golden: A row major, B stored [N][K], C[i][j] += A[i][k] * B[j][k]
  int mismatches = 0;
  for (int i = 0; i < NN; ++i)
    for (int j = 0; j < NN; ++j) {
      uint32_t acc = 0;
      for (int k = 0; k < NN; ++k) acc += (uint32_t)vmem[i * NN + k] * (uint32_t)vmem[MAT + j * NN + k];
      if ((uint32_t)vmem_out[i * NN + j] != acc) {
        if (mismatches < 10)
          printf("Mismatch at index %d: CPU=%d, device=%d\n", i * NN + j, (int)acc, (int)vmem_out[i * NN + j]);
        ++mismatches;
      }
    }
  return report(mismatches, what);
}

// ---------------------------------------------------------------- nokernelload
int run_nokernelload(miaie::Context& ctx) {
  std::vector<uint32_t> vmem(512);
  for (int i = 0; i < 512; ++i) vmem[i] = i;
  vmem[0] = 1024 * 1024;  // param_nn
  miaie::Buffer<uint32_t> in(ctx, 512), out(ctx, 512);
  std::vector<uint32_t> zeros(512, 0);
  out.move_in(zeros);
  in.move_in(vmem);
  const auto t0 = clk::now();
  miaie::dot_probe<1, 1, 4, 4, 256, 16, 64>(in.data(), out.data());
  if (!ctx.wait(kDeadlineMs)) return 2;
  const double us = us_since(t0);
  const std::vector<uint32_t> o = out.move_out();
  // The kernel's own contract (aie_nokernelload.cc:62-82): with the operator
  // precedence of :67-68, vec1[i] = (i + (p&1)) ? 1 : 2, vec2[i] = (p&1) ? 1 : 2.
  const uint32_t p = vmem[0];
  uint32_t dot = 0;
  for (uint32_t i = 0; i < 128; ++i) dot += ((i + (p & 1)) ? 1u : 2u) * ((p & 1) ? 1u : 2u);
  const uint64_t reps = 3ull * p;
  const uint32_t want[5] = {(uint32_t)reps, 4567u, (uint32_t)(dot * reps), 3u, (p & 1) ? 1u : 2u};
  int mismatches = 0;
  for (int i = 0; i < 5; ++i)
    if (o[i] != want[i]) {
      printf("Mismatch at index %d: CPU=%u, device=%u\n", i, want[i], o[i]);
      ++mismatches;
    }
  printf("uint8 MAC probe: %.3e MACs in %.1f us (%.1f TMAC/s incl. launch)\n", (double)reps * 128, us,
         (double)reps * 128 / us / 1e6);
  return report(mismatches, "nokernelload");
}

// ---------------------------------------------------------------- chains
int run_chain(miaie::Context& ctx, const std::vector<int32_t>& addends, int32_t expect, const char* what) {
  std::vector<int32_t> vmem(20, 15), vmem_out(20, 0);
  miaie::Buffer<int32_t> in(ctx, 20), out(ctx, 20);
  in.move_in(vmem);
  out.move_in(vmem_out);
  ctx.check(miaie_chain_add_i32(ctx.get(), in.data(), out.data(), 20, addends.data(), (int)addends.size()));
  if (!ctx.wait(kDeadlineMs)) return 2;
  out.move_out(vmem_out.data(), 20);
  int mismatches = 0;
  for (int i = 0; i < 20; ++i) mismatches += vmem_out[i] != expect;
  printf("%s: out[0] = %d (expected %d)\n", what, vmem_out[0], expect);
  return report(mismatches, what);
}

// ---------------------------------------------------------------- vek385
int run_vek385(miaie::Context& ctx) {
  const int n = 3, tiles = 4;
  const uint64_t iters = 1000;
  std::vector<uint64_t> in(tiles * n * n);
  for (int t = 0; t < tiles; ++t)
    for (int e = 0; e < n * n; ++e) in[t * n * n + e] = (uint64_t)(t + 3);
  miaie::Buffer<uint64_t> din(ctx, in.size()), dout(ctx, tiles * (n * n + 1));
  din.move_in(in);
  ctx.check(miaie_mm_square_u64(ctx.get(), din.data(), dout.data(), n, tiles, iters));
  if (!ctx.wait(kDeadlineMs)) return 2;
  const std::vector<uint64_t> o = dout.move_out();
  int mismatches = 0;
  for (int t = 0; t < tiles; ++t) {
    const uint64_t v = t + 3, want = 3 * v * v;  // {27, 48, 75, 108}
    for (int e = 0; e < n * n; ++e) mismatches += o[t * (n * n + 1) + e] != want;
    mismatches += o[t * (n * n + 1) + n * n] != iters;
    printf("tile %d: out[0] = %llu, count = %llu\n", t, (unsigned long long)o[t * (n * n + 1)],
           (unsigned long long)o[t * (n * n + 1) + n * n]);
  }
  return report(mismatches, "vek385");
}

// ---------------------------------------------------------------- benchmark shapes
int run_gemm(miaie::Context& ctx, int M, int N, int K, int shift) {
  const std::vector<int8_t> A = seeded_i8((size_t)M * K, 1), B = seeded_i8((size_t)K * N, 2);
  miaie::Buffer<int8_t> dA(ctx, A.size()), dB(ctx, B.size()), dY(ctx, (size_t)M * N);
  dA.move_in(A);
  dB.move_in(B);
  const auto t0 = clk::now();
  ctx.check(miaie_gemm_i8_rq(ctx.get(), dA.data(), dB.data(), dY.data(), M, N, K, shift, 0, nullptr, MIAIE_B_NN));
  if (!ctx.wait(kDeadlineMs)) return 2;
  const double us = us_since(t0);
  const std::vector<int8_t> Y = dY.move_out();
  int mismatches = 0;
  const int rows[] = {0, 1, M / 3, M / 2, M - 2, M - 1};
  for (int i : rows)
    for (int j = 0; j < N; ++j) {
      int64_t acc = 0;
      for (int k = 0; k < K; ++k) acc += (int64_t)A[(size_t)i * K + k] * B[(size_t)k * N + j];
      mismatches += Y[(size_t)i * N + j] != rq(acc, shift, false);
    }
  printf("int8 GEMM %dx%dx%d shift %d: %.1f us incl. launch and wait (%.1f TOP/s)\n", M, N, K, shift, us,
         2.0 * M * N * K / us / 1e6);
  const miaie_gemm_plan plan = ctx.plan_gemm_i8(M, N, K);
  printf("plan: kernel %d, tile %dx%d, %d workgroups of %d threads\n", plan.kernel, plan.tile_m, plan.tile_n,
         plan.workgroups, plan.threads);
  return report(mismatches, "gemm");
}

int run_conv(miaie::Context& ctx, int reps, int streams) {
  const int Nb = 8, H = 56, Wd = 56, C = 64, Co = 64;
  const std::vector<int8_t> X = seeded_i8((size_t)Nb * H * Wd * C, 3), W = seeded_i8((size_t)Co * 9 * C, 4);
  const std::vector<uint8_t> sh = seeded_shifts(Co, 7);
  miaie::Buffer<int8_t> dX(ctx, X.size()), dW(ctx, W.size()), dY(ctx, X.size());
  miaie::Buffer<uint8_t> dS(ctx, Co);
  dX.move_in(X);
  dW.move_in(W);
  dS.move_in(sh);
  miaie::conv2d_i8(dX, dW, dS, dY, miaie::ConvShape{Nb, H, Wd, C, Co}, ctx);
  if (!ctx.wait(kDeadlineMs)) return 2;
  const std::vector<int8_t> Y = dY.move_out();
  int mismatches = 0;
  const int n = Nb - 1;  // golden on the last image
  for (int h = 0; h < H; ++h)
    for (int w = 0; w < Wd; ++w)
      for (int co = 0; co < Co; ++co) {
        int64_t acc = 0;
        for (int r = 0; r < 3; ++r)
          for (int s = 0; s < 3; ++s) {
            const int hi = h + r - 1, wi = w + s - 1;
            if (hi < 0 || hi >= H || wi < 0 || wi >= Wd) continue;
            for (int ci = 0; ci < C; ++ci)
              acc += (int64_t)X[(((size_t)n * H + hi) * Wd + wi) * C + ci] * W[((size_t)co * 9 + r * 3 + s) * C + ci];
          }
        mismatches += Y[(((size_t)n * H + h) * Wd + w) * Co + co] != rq(acc, sh[co], false);
      }
  if (reps > 0) {
    // back-to-back calls of the C entry point from C++, after as many
    // untimed ones: host launch work and device time overlap, so this is the
    // device's time per convolution unless the host is slower
    for (int i = 0; i < reps; ++i) miaie::conv2d_i8(dX, dW, dS, dY, miaie::ConvShape{Nb, H, Wd, C, Co}, ctx);
    if (!ctx.wait(kDeadlineMs)) return 2;
    const auto t0 = clk::now();
    for (int i = 0; i < reps; ++i) miaie::conv2d_i8(dX, dW, dS, dY, miaie::ConvShape{Nb, H, Wd, C, Co}, ctx);
    const double issue_us = us_since(t0) / reps;  // the host's time per call alone
    if (!ctx.wait(kDeadlineMs)) return 2;
    printf("conv2d back-to-back: %.3f us per call over %d calls (host issue %.3f us per call)\n", us_since(t0) / reps,
           reps, issue_us);
  }
  if (reps > 0 && streams > 1) {
    // independent convolutions (a batch each) on `streams` contexts: the
    // command processor's per-launch work of one stream overlaps another's
    struct Set {
      std::unique_ptr<miaie::Context> ctx;
      miaie::Buffer<int8_t> X, W, Y;
      miaie::Buffer<uint8_t> S;
    };
    std::vector<Set> sets;
    for (int s = 0; s < streams; ++s) {
      auto c = std::make_unique<miaie::Context>(0);
      miaie::Context& cr = *c;
      sets.push_back(Set{std::move(c), miaie::Buffer<int8_t>(cr, X.size()), miaie::Buffer<int8_t>(cr, W.size()),
                         miaie::Buffer<int8_t>(cr, X.size()), miaie::Buffer<uint8_t>(cr, Co)});
      sets.back().X.move_in(X);
      sets.back().W.move_in(W);
      sets.back().S.move_in(sh);
    }
    auto issue = [&]() {
      for (int i = 0; i < reps; ++i) {
        Set& st = sets[i % streams];
        miaie::conv2d_i8(st.X, st.W, st.S, st.Y, miaie::ConvShape{Nb, H, Wd, C, Co}, *st.ctx);
      }
      for (Set& st : sets)
        if (!st.ctx->wait(kDeadlineMs)) return false;
      return true;
    };
    // the same calls issued by one host thread per stream (each thread uses
    // only its own context): the device's rate with `streams` convolutions
    // in flight, no longer bounded by one thread's issue time
    auto issue_threaded = [&]() {
      std::atomic<int> failed{0};
      std::vector<std::thread> th;
      for (int s = 0; s < streams; ++s)
        th.emplace_back([&, s]() {
          try {
            Set& st = sets[s];
            for (int i = s; i < reps; i += streams)
              miaie::conv2d_i8(st.X, st.W, st.S, st.Y, miaie::ConvShape{Nb, H, Wd, C, Co}, *st.ctx);
            if (!st.ctx->wait(kDeadlineMs)) failed = 1;
          } catch (const miaie::Error& e) {
            fprintf(stderr, "conv2d thread %d: miaie error %d: %s\n", s, e.code(), e.what());
            failed = 1;
          }
        });
      for (std::thread& t : th) t.join();
      return failed.load() == 0;
    };
    if (!issue()) return 2;
    auto t0 = clk::now();
    if (!issue()) return 2;
    printf("conv2d on %d streams: %.3f us per call over %d calls\n", streams, us_since(t0) / reps, reps);
    if (!issue_threaded()) return 2;
    t0 = clk::now();
    if (!issue_threaded()) return 2;
    printf("conv2d on %d streams from %d threads: %.3f us per call over %d calls\n", streams, streams,
           us_since(t0) / reps, reps);
    const std::vector<int8_t> Y0 = dY.move_out();
    for (Set& st : sets) mismatches += st.Y.move_out() != Y0;
    // last constructed first, so each context hands "current" back to the
    // one constructed before it
    while (!sets.empty()) sets.pop_back();
  }
  return report(mismatches, "conv2d");
}

int run_mlp(miaie::Context& ctx, int M, int K, int F, int Nout) {
  const std::vector<int8_t> X = seeded_i8((size_t)M * K, 3), W1 = seeded_i8((size_t)K * F, 5),
                            W2 = seeded_i8((size_t)F * Nout, 6);
  miaie::Buffer<int8_t> dX(ctx, X.size()), d1(ctx, W1.size()), d2(ctx, W2.size()), dH(ctx, (size_t)M * F),
      dY(ctx, (size_t)M * Nout);
  dX.move_in(X);
  d1.move_in(W1);
  d2.move_in(W2);
  miaie::mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, 11, 12, ctx);
  if (!ctx.wait(kDeadlineMs)) return 2;
  const std::vector<int8_t> Y = dY.move_out();
  int mismatches = 0;
  std::vector<int8_t> h(F);
  for (int i : {0, M / 2, M - 1}) {
    for (int f = 0; f < F; ++f) {
      int64_t acc = 0;
      for (int k = 0; k < K; ++k) acc += (int64_t)X[(size_t)i * K + k] * W1[(size_t)k * F + f];
      h[f] = rq(acc, 11, true);
    }
    for (int j = 0; j < Nout; ++j) {
      int64_t acc = 0;
      for (int f = 0; f < F; ++f) acc += (int64_t)h[f] * W2[(size_t)f * Nout + j];
      mismatches += Y[(size_t)i * Nout + j] != rq(acc, 12, false);
    }
  }
  return report(mismatches, "mlp");
}

int usage() {
  fprintf(stderr,
          "usage: miaie_examples mm [n 8|16] [base] | perf | nokernelload | multi_tile | seq_full_col | vek385 |\n"
          "                      gemm M N K shift | conv [reps] [streams] | mlp M K F N\n");
  return 64;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return usage();
  const std::string cmd = argv[1];
  auto arg = [&](int i, int dflt) { return argc > i ? atoi(argv[i]) : dflt; };
  try {
    miaie::Context ctx(0);
    if (cmd == "mm") {
      const int n = arg(2, 16), base = arg(3, 0);
      if (n == 16) return run_window<16, int32_t>(ctx, base, "mm");
      if (n == 8) return run_window<8, int32_t>(ctx, base, "mm");
      return usage();
    }
    if (cmd == "perf") return run_window<16, uint32_t>(ctx, 1, "perf");
    if (cmd == "nokernelload") return run_nokernelload(ctx);
    if (cmd == "multi_tile") return run_chain(ctx, {1, 10}, 26, "multi_tile");
    if (cmd == "seq_full_col") return run_chain(ctx, std::vector<int32_t>(8, 1), 23, "seq_full_col");
    if (cmd == "vek385") return run_vek385(ctx);
    if (cmd == "gemm") return run_gemm(ctx, arg(2, 4096), arg(3, 4096), arg(4, 4096), arg(5, 10));
    if (cmd == "conv") return run_conv(ctx, arg(2, 0), arg(3, 1));
    if (cmd == "mlp") return run_mlp(ctx, arg(2, 256), arg(3, 4096), arg(4, 11008), arg(5, 4096));
    return usage();
  } catch (const miaie::Error& e) {
    fprintf(stderr, "miaie error %d: %s\n", e.code(), e.what());
    return 3;
  }
}
