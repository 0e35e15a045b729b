// qmv1_timeline -- time line of the M = 1 decode GEMV (qmv1_slice_kernel, int4
// group 64) inside a HIP graph of back-to-back launches over distinct weight
// copies, as the bench runs it.  A diagnostic, not part of the library: build.py
// --diag compiles it with fmxq_qmv.hip under FMXQ_QMV1_TIMELINE, which makes
// every wave of the kernel store s_memrealtime stamps (100 MHz) at five points:
//   start      the wave's first instruction;
//   issued     its weight loads issued (x, scales and biases before them);
//   row0 done  its first row's arithmetic done, so its weight bytes arrived;
//   rows done  its last row's arithmetic done;
//   end        its output stored (after the block's slice reduction).
// Six launches in the middle of the graph carry a stamp buffer; the program
// prints, per launch, the percentiles of each stamp over all waves (relative to
// the launch's first wave start), the gap after the previous launch's last wave,
// per-wave intervals, and the first start and last end on each XCD.
//
// usage: qmv1_timeline [N [K]]   (defaults 4096 14336, the north-star shape)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "fmxq_internal.hpp"

#ifndef FMXQ_QMV1_TIMELINE
#error "build with -DFMXQ_QMV1_TIMELINE (python -m fastmlx_amd.build --diag)"
#endif

#define CK(x)                                                                          \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);       \
      std::exit(1);                                                                    \
    }                                                                                  \
  } while (0)

int main(int argc, char** argv) {
  const int64_t N = argc > 1 ? std::atol(argv[1]) : 4096, K = argc > 2 ? std::atol(argv[2]) : 14336;
  // qmv1_slice_kernel<16, 7, 1>: 16 rows x 7 slices of 2048 values per block (K = 14336);
  // the launcher picks it for these shapes, and the stamp buffer is sized for it.
  constexpr int RW = 16, KS = 7;
  if (K != 2048 * KS || N < 1 || N > (int64_t(1) << 20)) {
    std::printf("K must be %d and N in 1..2^20\n", 2048 * KS);
    return 1;
  }
  const int copies = 32, launches = 128, NI = 6, first = 60;
  const int64_t blocks = (N + RW - 1) / RW, waves = blocks * KS;
  const size_t wb = (size_t)N * K / 2, sb = (size_t)N * (K / 64) * 2;
  std::vector<uint32_t> hw(wb / 4);
  std::vector<uint16_t> hs(N * (K / 64)), hb(N * (K / 64)), hx(K);
  uint32_t seed = 7;
  auto rnd = [&]() { return seed = seed * 1664525u + 1013904223u; };
  for (auto& v : hw) v = rnd();
  for (auto& v : hs) v = 0x3c00 + (rnd() & 0xff);  // bf16 scales in [2^-7, 2^-6)
  for (auto& v : hb) v = 0xbc00 + (rnd() & 0xff);
  for (auto& v : hx) v = 0x3f00 + (rnd() & 0x7f) + ((rnd() & 1) << 15);
  std::vector<uint32_t*> dw(copies);
  std::vector<uint16_t*> ds(copies), db(copies);
  for (int c = 0; c < copies; ++c) {
    CK(hipMalloc(&dw[c], wb));
    CK(hipMemcpy(dw[c], hw.data(), wb, hipMemcpyHostToDevice));
    CK(hipMalloc(&ds[c], sb));
    CK(hipMemcpy(ds[c], hs.data(), sb, hipMemcpyHostToDevice));
    CK(hipMalloc(&db[c], sb));
    CK(hipMemcpy(db[c], hb.data(), sb, hipMemcpyHostToDevice));
  }
  uint16_t *dx, *dy;
  CK(hipMalloc(&dx, K * 2));
  CK(hipMemcpy(dx, hx.data(), K * 2, hipMemcpyHostToDevice));
  CK(hipMalloc(&dy, N * 2));
  uint64_t* st;
  const size_t words = (size_t)NI * waves * 6;
  CK(hipMalloc(&st, words * 8));
  CK(hipMemset(st, 0, words * 8));
  hipStream_t stream;
  CK(hipStreamCreate(&stream));
  hipGraph_t g;
  hipGraphExec_t ge;
  CK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
  for (int i = 0; i < launches; ++i) {
    fmxq::QmmArgs a{dx, dw[i % copies], ds[i % copies], db[i % copies], nullptr, dy, 1, N, K, K, N,
                    64, 4};
    a.tl_stamps = (i >= first && i < first + NI) ? st + (size_t)(i - first) * waves * 6 : nullptr;
    CK(fmxq::launch_qmv(a, stream));
  }
  CK(hipStreamEndCapture(stream, &g));
  CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  for (int w = 0; w < 5; ++w) CK(hipGraphLaunch(ge, stream));
  const int reps = 10;
  CK(hipEventRecord(e0, stream));
  for (int w = 0; w < reps; ++w) CK(hipGraphLaunch(ge, stream));
  CK(hipEventRecord(e1, stream));
  CK(hipEventSynchronize(e1));
  float ms = 0.f;
  CK(hipEventElapsedTime(&ms, e0, e1));
  const double us = ms * 1000.0 / (reps * launches);
  const double bytes = (double)wb + 2.0 * sb + K * 2 + N * 2;
  std::printf("N=%lld K=%lld: %.3f us per launch (graph of %d launches over %d copies), %.0f GB/s\n",
              (long long)N, (long long)K, us, launches, copies, bytes / us * 1e-3);
  std::vector<uint64_t> h(words);
  CK(hipMemcpy(h.data(), st, words * 8, hipMemcpyDeviceToHost));
  auto pct = [](std::vector<double> v, double p) {
    std::sort(v.begin(), v.end());
    return v[(size_t)std::min<double>((double)v.size() - 1, p * v.size())];
  };
  const char* names[5] = {"start", "issued", "row0 done", "rows done", "end"};
  double prev_end = 0;
  for (int l = 0; l < NI; ++l) {
    const uint64_t* o = h.data() + (size_t)l * waves * 6;
    uint64_t t0 = ~0ull, t4 = 0;
    for (int64_t w = 0; w < waves; ++w) {
      t0 = std::min(t0, o[w * 6]);
      t4 = std::max(t4, o[w * 6 + 4]);
    }
    std::vector<double> d[5];
    for (int64_t w = 0; w < waves; ++w)
      for (int k = 0; k < 5; ++k) d[k].push_back((o[w * 6 + k] - t0) * 0.01);
    std::printf("launch %d: span %.2f us", first + l, (t4 - t0) * 0.01);
    if (l) std::printf(", gap after the previous launch's last wave %.2f us", t0 * 0.01 - prev_end);
    std::printf("\n");
    prev_end = t4 * 0.01;
    for (int k = 0; k < 5; ++k)
      std::printf("  %-10s p0 %5.2f  p10 %5.2f  p50 %5.2f  p90 %5.2f  p99 %5.2f  max %5.2f us\n",
                  names[k], pct(d[k], 0), pct(d[k], 0.1), pct(d[k], 0.5), pct(d[k], 0.9),
                  pct(d[k], 0.99), pct(d[k], 1.0));
    std::vector<double> arrive, rows, tail;
    for (int64_t w = 0; w < waves; ++w) {
      arrive.push_back((o[w * 6 + 2] - o[w * 6 + 1]) * 0.01);
      rows.push_back((o[w * 6 + 3] - o[w * 6 + 2]) * 0.01);
      tail.push_back((o[w * 6 + 4] - o[w * 6 + 3]) * 0.01);
    }
    std::printf("  per wave: issued->row0 p50 %.2f p90 %.2f; row0->rows p50 %.2f p90 %.2f; "
                "rows->end p50 %.2f p90 %.2f us\n",
                pct(arrive, .5), pct(arrive, .9), pct(rows, .5), pct(rows, .9), pct(tail, .5),
                pct(tail, .9));
    std::vector<double> xs(8, 1e9), xe(8, 0);
    for (int64_t w = 0; w < waves; ++w) {
      const int x = (int)(o[w * 6 + 5] >> 32) & 7;
      xs[x] = std::min(xs[x], d[0][w]);
      xe[x] = std::max(xe[x], d[4][w]);
    }
    std::printf("  per XCD first start / last end:");
    for (int x = 0; x < 8; ++x) std::printf(" [%.2f %.2f]", xs[x], xe[x]);
    std::printf("\n");
  }
  return 0;
}
