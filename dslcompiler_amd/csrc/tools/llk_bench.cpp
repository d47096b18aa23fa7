// llk-bench -- GPU benchmark of the gfx950 kernels, the counterpart of the
// reference's benchmarking harness (tools/llk-bench/llk-bench.cpp:21-121):
// same options and method (warm up for --warmup-ms, then --reps windows of
// at least --measure-ms each, report the best), timing the real fused
// SwiGLU / matmul launches with HIP events instead of a CPU stand-in.
//
//   llk-bench [--op=fused_swiglu|matmul] [--M=128] [--N=4096] [--K=4096]
//             [--threads=8] [--out=bf16|f32] [--warmup-ms=500]
//             [--measure-ms=2000] [--reps=5] [--copies=1] [--seed=42]
//             [--kernel-fn] [--dry-run]
//
// --kernel-fn times llk_swiglu_kernel_fn -- the reference's KernelFn shape,
// five MemRef2D, synchronous, row-major weights read at every call -- by
// wall clock around each call, as the reference's harness times its
// function, on device-resident X, Y and row-major weights (SwiGLU, bf16
// result only).  Without it the asynchronous llk_swiglu_bf16 / llk_gemm_bf16
// launches on packed weights are timed with HIP events.
// --dry-run prints the parsed shape and the launch the dispatcher would make
// (llk_describe_launch), and times nothing (no GPU needed).
//
// Options take llvm::cl's forms (-M 2048, --M=2048, -M=2048; cl_opts.h);
// an unknown option exits 1.  --threads is the reference's CPU thread
// count: accepted so that its scripts run unchanged, and reported as not
// used (the GPU launch takes its parallelism from the grid).
//
// Inputs: X ~ N(0,1), weights ~ N(0, 1/sqrt(K)) in bf16 (llk_fill_normal_bf16),
// resident in HBM before timing.  --copies rotates that many weight sets so
// small-M runs stream from HBM rather than the 256 MB MALL.
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "cl_opts.h"
#include "llk/llk_abi.h"

namespace {

[[noreturn]] void die(const char* what, const char* msg) {
  std::fprintf(stderr, "llk-bench: %s: %s\n", what, msg);
  std::exit(1);
}

void check_llk(int rc, const char* what) {
  if (rc != LLK_OK) die(what, llk_last_error());
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) die(what, hipGetErrorString(e));
}

double now_ms() {
  return std::chrono::duration<double, std::milli>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

}  // namespace

int main(int argc, char** argv) {
  std::string op = "fused_swiglu", out = "bf16";
  int64_t M = 128, N = 4096, K = 4096, threads = 8, warmup_ms = 500, measure_ms = 2000, reps = 5,
          copies = 1, seed_opt = 42;
  llk_tools::Options cl("llk-bench", "LLK kernel benchmark (gfx950)");
  cl.add_str("op", &op, "Operation: fused_swiglu or matmul");
  cl.add_int("M", &M, "M dimension (rows)");
  cl.add_int("N", &N, "N dimension (hidden)");
  cl.add_int("K", &K, "K dimension (input)");
  cl.add_int("threads", &threads, "Thread count (CPU; not used by the GPU launch)");
  cl.add_str("out", &out, "Output type: bf16 or f32");
  cl.add_int("warmup-ms", &warmup_ms, "Warmup milliseconds");
  cl.add_int("measure-ms", &measure_ms, "Measurement milliseconds");
  cl.add_int("reps", &reps, "Measurement repetitions");
  cl.add_int("copies", &copies, "Weight sets rotated between launches");
  cl.add_int("seed", &seed_opt, "Input generator seed");
  bool dry = false, kfn = false;
  cl.add_flag("dry-run", &dry, "Print the shape and launch plan; time nothing");
  cl.add_flag("kernel-fn", &kfn,
              "Time llk_swiglu_kernel_fn (synchronous, row-major device weights) per call");
  if (!cl.parse(argc, argv)) return 1;
  copies = std::max<int64_t>(1, copies);
  const uint64_t seed = (uint64_t)seed_opt;
  const bool swiglu = op == "fused_swiglu";
  if (!swiglu && op != "matmul") die("--op", "fused_swiglu or matmul");
  if (out != "bf16" && out != "f32") die("--out", "bf16 or f32");
  if (M < 1 || N < 1 || K < 1 || reps < 1) die("shape", "M, N, K and reps must be positive");
  if (threads < 1) die("--threads", "must be positive");
  if (kfn && (!swiglu || out != "bf16"))
    die("--kernel-fn", "llk_swiglu_kernel_fn computes --op=fused_swiglu with --out=bf16");
  const int y_dtype = out == "bf16" ? LLK_BF16 : LLK_FP32;
  if (dry) {
    llk_launch_plan plan;
    check_llk(llk_describe_launch(swiglu ? 0 : 3, M, N, K, LLK_PLAN_X_ALIGNED, &plan), "plan");
    std::printf("LLK Bench (dry run) — op=%s M=%lld N=%lld K=%lld threads=%lld out=%s "
                "warmup-ms=%lld measure-ms=%lld reps=%lld copies=%lld%s\n",
                op.c_str(), (long long)M, (long long)N, (long long)K, (long long)threads,
                out.c_str(), (long long)warmup_ms, (long long)measure_ms, (long long)reps,
                (long long)copies, kfn ? " kernel-fn" : "");
    std::printf("plan: kernel=%s splits=%d group_width=%d workgroups=%lld launches=%lld "
                "workspace=%zu\n",
                llk_tools::kernel_name(plan.kernel), plan.splits, plan.group_width,
                (long long)plan.workgroups, (long long)plan.launches, plan.workspace_bytes);
    return 0;
  }

  char arch[64] = {0};
  int cus = 0, lds = 0, clk = 0;
  check_llk(llk_device_info(arch, sizeof arch, &cus, &lds, &clk), "device");
  std::printf("LLK Bench — op=%s M=%lld N=%lld K=%lld threads=%lld out=%s device=%s CUs=%d "
              "copies=%lld\n",
              op.c_str(), (long long)M, (long long)N, (long long)K, (long long)threads,
              out.c_str(), arch, cus, (long long)copies);
  std::printf("note: --threads is not used on the GPU (the launch grid covers %d CUs)\n", cus);

  // Host inputs (generator streams: X 0, Wg 1, Wu 2), packed once per copy
  // (--kernel-fn: copied to the device row-major instead).
  std::vector<uint16_t> x((size_t)M * K), w((size_t)K * N);
  check_llk(llk_fill_normal_bf16(seed, 0, 1.0f, x.data(), (int64_t)x.size(), 0), "fill X");
  const int nmat = swiglu ? 2 : 1;
  std::vector<llk_packed_weights*> packed;
  std::vector<void*> rowmajor;
  for (int c = 0; c < copies; ++c)
    for (int p = 0; p < nmat; ++p) {
      check_llk(llk_fill_normal_bf16(seed + 1000 * c, 1 + p, 1.0f / std::sqrt((float)K), w.data(),
                                     (int64_t)w.size(), 0),
                "fill W");
      if (kfn) {
        void* dw = nullptr;
        check_hip(hipMalloc(&dw, w.size() * 2), "hipMalloc W");
        check_hip(hipMemcpy(dw, w.data(), w.size() * 2, hipMemcpyHostToDevice), "copy W");
        rowmajor.push_back(dw);
        continue;
      }
      llk_tensor2d wt{w.data(), K, N, N, 1};
      llk_packed_weights* pw = nullptr;
      check_llk(llk_pack_weights(&wt, 64, 0, &pw), "pack");
      packed.push_back(pw);
    }
  void *dx = nullptr, *dy = nullptr;
  check_hip(hipMalloc(&dx, x.size() * 2), "hipMalloc X");
  check_hip(hipMalloc(&dy, (size_t)M * N * (y_dtype == LLK_BF16 ? 2 : 4)), "hipMalloc Y");
  check_hip(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice), "copy X");
  hipStream_t stream;
  check_hip(hipStreamCreate(&stream), "stream");
  llk_tensor2d xt{dx, M, K, K, 1}, yt{dy, M, N, N, 1};
  llk_kernel_context ctx{nullptr, 0, stream};
  int64_t it = 0;
  auto launch = [&]() {
    const int c = (int)(it++ % copies);
    const int rc = swiglu ? llk_swiglu_bf16(&xt, packed[2 * c], packed[2 * c + 1], &yt, y_dtype, &ctx)
                          : llk_gemm_bf16(&xt, packed[c], &yt, y_dtype, &ctx);
    check_llk(rc, "launch");
  };
  llk_memref2d mx{dx, dx, 0, M, K, K, 1}, my{dy, dy, 0, M, N, N, 1};
  auto call = [&]() {  // one synchronous KernelFn call: Y = SwiGLU(X; Wg, Wu)
    const int c = (int)(it++ % copies);
    llk_memref2d mg{rowmajor[2 * c], rowmajor[2 * c], 0, K, N, N, 1};
    llk_memref2d mu{rowmajor[2 * c + 1], rowmajor[2 * c + 1], 0, K, N, N, 1};
    llk_swiglu_kernel_fn(&mx, &mg, &mu, &my, &my);
    check_llk(llk_kernel_fn_status(), "KernelFn");
  };

  // Warm-up: the GPU reaches its steady clock after ~35 ms of load.
  const double t0 = now_ms();
  do {
    for (int i = 0; i < 10; ++i) kfn ? call() : launch();
    check_hip(hipStreamSynchronize(stream), "sync");
  } while (now_ms() - t0 < (double)warmup_ms);

  hipEvent_t e0, e1;
  check_hip(hipEventCreate(&e0), "event");
  check_hip(hipEventCreate(&e1), "event");
  double best_ms = 0.0;
  for (int r = 0; r < reps; ++r) {
    int64_t iters = 0;
    const double w0 = now_ms();
    double per = 0.0;
    if (kfn) {  // synchronous calls: wall clock around them
      do {
        for (int i = 0; i < 10; ++i) call();
        iters += 10;
      } while (now_ms() - w0 < (double)measure_ms);
      per = (now_ms() - w0) / (double)iters;
    } else {
      check_hip(hipEventRecord(e0, stream), "record");
      do {
        for (int i = 0; i < 10; ++i) launch();
        iters += 10;
        check_hip(hipEventRecord(e1, stream), "record");
        check_hip(hipEventSynchronize(e1), "sync");
      } while (now_ms() - w0 < (double)measure_ms);
      float ms = 0.f;
      check_hip(hipEventElapsedTime(&ms, e0, e1), "elapsed");
      per = ms / (double)iters;
    }
    if (best_ms == 0.0 || per < best_ms) best_ms = per;
  }
  const double flops = 2.0 * nmat * (double)M * N * K;
  const double bytes = 2.0 * nmat * (double)K * N + 2.0 * M * K +
                       (double)M * N * (y_dtype == LLK_BF16 ? 2 : 4);
  std::printf("Best: %.1f GFLOPS (%.6f ms/iter, %lld reps)\n", flops / (best_ms * 1e-3) / 1e9,
              best_ms, (long long)reps);
  std::printf("      %.1f TFLOP/s, %.1f GB/s of algorithmic bytes (%.0f B/launch)\n",
              flops / (best_ms * 1e-3) / 1e12, bytes / (best_ms * 1e-3) / 1e9, bytes);
  if (kfn) std::printf("      llk_swiglu_kernel_fn: synchronous calls, wall clock per call\n");
  for (auto* pw : packed) llk_packed_weights_free(pw);
  for (void* dw : rowmajor) (void)hipFree(dw);
  (void)hipFree(dx);
  (void)hipFree(dy);
  (void)hipStreamDestroy(stream);
  return 0;
}
