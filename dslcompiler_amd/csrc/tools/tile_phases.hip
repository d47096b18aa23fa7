// llk-tile-phases -- per-workgroup phase timing of the prefill / GEMM tile
// kernel (kernels/mfma_tile.hip built with LLK_TILE_PHASES): every
// workgroup records the 100 MHz real-time counter at entry, when its first
// pipeline stage has landed, after the K loop and after the epilogue, and
// the tool prints the spread of each phase and the K loop's time per 32-k
// stage.  Inputs are bf16 with a normal distribution (X ~ N(0,1), weights
// ~ N(0, 1/sqrt(K))), because the operand values set the board's power draw
// and so its clock.
//
//   llk-tile-phases                       # config 3, GEMM 4096^3, SwiGLU M=255
//   llk-tile-phases swiglu 2048 11008 4096 [S] gemm 4096 4096 4096 ...
#define LLK_TILE_PHASES 1
#include "kernels/mfma_tile.hip"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "tools/fill_normal.h"

namespace {

bool check(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

struct Shape {
  int mode;  // 1 SwiGLU, 0 GEMM
  int M, N, K, S;
};

struct Stat {
  double min, mean, max;
};

Stat stat(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  double s = 0;
  for (double x : v) s += x;
  return {v.front(), s / v.size(), v.back()};
}

bool run(const Shape& sh) {
  const int KB = sh.K / 64, NB = (sh.N + 127) / 128;
  const size_t wbytes = (size_t)NB * KB * 16384;
  const int tiles = (sh.M + 255) / 256 * (sh.mode == 1 ? NB : (NB + 1) / 2);
  const int wgs = tiles * sh.S;
  const size_t part_bytes = llk_tile_split_bytes(sh.mode, sh.M, NB, sh.S);
  uint16_t *x = nullptr, *w0 = nullptr, *w1 = nullptr;
  void *y = nullptr, *part = nullptr;
  unsigned long long* ph = nullptr;
  bool ok = check(hipMalloc(&x, (size_t)sh.M * sh.K * 2), "hipMalloc x") &&
            check(hipMalloc(&w0, wbytes), "hipMalloc w0") &&
            (sh.mode == 0 || check(hipMalloc(&w1, wbytes), "hipMalloc w1")) &&
            check(hipMalloc(&y, (size_t)sh.M * sh.N * 2), "hipMalloc y") &&
            (part_bytes == 0 || check(hipMalloc(&part, part_bytes), "hipMalloc part")) &&
            check(hipMalloc(&ph, (size_t)wgs * 4 * sizeof(unsigned long long)), "hipMalloc ph");
  if (ok) {
    hipLaunchKernelGGL(llk_tools::fill_normal_kernel, dim3(4096), dim3(256), 0, 0, x, (size_t)sh.M * sh.K, 1ull, 1.0f);
    const float ws = 1.0f / std::sqrt((float)sh.K);
    hipLaunchKernelGGL(llk_tools::fill_normal_kernel, dim3(4096), dim3(256), 0, 0, w0, wbytes / 2, 2ull, ws);
    if (w1) hipLaunchKernelGGL(llk_tools::fill_normal_kernel, dim3(4096), dim3(256), 0, 0, w1, wbytes / 2, 3ull, ws);
    ok = check(hipDeviceSynchronize(), "fill");
  }
  auto launch = [&]() {
    return llk_launch_tile(sh.mode, x, sh.K, w0, w1, y, sh.N, sh.M, sh.N, KB, NB, sh.S, part,
                           llk_gfx950::kOutBF16, sh.N % 4 == 0, nullptr);
  };
  if (ok) {
    llk_tile_phases_buffer = ph;
    for (int i = 0; i < 300 && ok; ++i) ok = check(launch(), "launch");  // reach the steady clock
    ok = ok && check(hipDeviceSynchronize(), "warm-up");
  }
  float ms = 0.0f;
  if (ok) {
    hipEvent_t e0, e1;
    ok = check(hipEventCreate(&e0), "event") && check(hipEventCreate(&e1), "event");
    if (ok) {
      (void)hipEventRecord(e0, nullptr);
      for (int i = 0; i < 50 && ok; ++i) ok = check(launch(), "launch");
      (void)hipEventRecord(e1, nullptr);
      ok = ok && check(hipEventSynchronize(e1), "timed launches");
      if (ok) (void)hipEventElapsedTime(&ms, e0, e1);
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
    }
  }
  std::vector<unsigned long long> h((size_t)wgs * 4);
  if (ok) {
    ok = check(launch(), "launch") && check(hipDeviceSynchronize(), "instrumented launch") &&
         check(hipMemcpy(h.data(), ph, h.size() * 8, hipMemcpyDeviceToHost), "copy");
  }
  if (ok) {
    unsigned long long t0 = ~0ull, t1 = 0;
    std::vector<double> pro, loop, epi;
    for (int i = 0; i < wgs; ++i) {
      const unsigned long long* r = &h[(size_t)i * 4];
      t0 = std::min(t0, r[0]);
      t1 = std::max(t1, r[3]);
      pro.push_back((r[1] - r[0]) / 100.0);
      loop.push_back((r[2] - r[1]) / 100.0);
      epi.push_back((r[3] - r[2]) / 100.0);
    }
    const Stat p = stat(pro), l = stat(loop), e = stat(epi);
    const int stages = (KB + sh.S - 1) / sh.S * 2;
    std::printf("%s M=%d N=%d K=%d S=%d: %d workgroups, %.1f us per launch (HIP events, "
                "incl. the split reduce), kernel span %.1f us\n",
                sh.mode == 1 ? "swiglu" : "gemm", sh.M, sh.N, sh.K, sh.S, wgs, ms * 1000.0 / 50,
                (t1 - t0) / 100.0);
    std::printf("  prologue (entry -> first stage landed)  min %6.2f  mean %6.2f  max %6.2f us\n",
                p.min, p.mean, p.max);
    std::printf("  K loop (%3d stages of 32 k)             min %6.2f  mean %6.2f  max %6.2f us"
                "  (%.3f us per stage)\n",
                stages, l.min, l.mean, l.max, l.mean / stages);
    std::printf("  epilogue                                min %6.2f  mean %6.2f  max %6.2f us\n",
                e.min, e.mean, e.max);
    std::fflush(stdout);
  }
  llk_tile_phases_buffer = nullptr;
  (void)hipFree(x);
  (void)hipFree(w0);
  (void)hipFree(w1);
  (void)hipFree(y);
  (void)hipFree(part);
  (void)hipFree(ph);
  return ok;
}

}  // namespace

int main(int argc, char** argv) {
  std::vector<Shape> shapes;
  for (int i = 1; i < argc;) {
    const std::string op = argv[i];
    if ((op != "swiglu" && op != "gemm") || i + 3 >= argc) {
      std::fprintf(stderr, "usage: %s [swiglu|gemm M N K [S]]...\n", argv[0]);
      return 2;
    }
    Shape s{op == "swiglu" ? 1 : 0, std::atoi(argv[i + 1]), std::atoi(argv[i + 2]),
            std::atoi(argv[i + 3]), 1};
    i += 4;
    if (i < argc && std::isdigit(static_cast<unsigned char>(argv[i][0]))) s.S = std::atoi(argv[i++]);
    shapes.push_back(s);
  }
  if (shapes.empty())
    shapes = {{1, 2048, 11008, 4096, 1}, {0, 4096, 4096, 4096, 1}, {1, 255, 13824, 5120, 2}};
  for (const Shape& s : shapes) {
    const int KB = s.K / 64;
    const int kbs = s.S > 0 ? (KB + s.S - 1) / s.S : 0;
    if (s.M < 1 || s.N < 1 || s.K < 64 || s.K % 64 != 0 || s.S < 1 || (s.S - 1) * kbs >= KB ||
        !llk_tile_x_fits(s.M, s.K)) {
      std::fprintf(stderr, "shape M=%d N=%d K=%d S=%d: need M, N >= 1, K a multiple of 64, "
                   "every split non-empty, X within the kernel's 32-bit offsets\n",
                   s.M, s.N, s.K, s.S);
      return 2;
    }
    if (!run(s)) return 1;
  }
  return 0;
}
