// llk-tune -- measured schedule search for the gfx950 kernels, the
// counterpart of the reference's grid-search driver
// (tools/llk-tune/llk-tune.cpp:65-232), which generates candidates and
// writes schedule_db.json records but measures nothing.  Here every
// candidate is launched and timed on the GPU.
//
//   llk-tune [--op=fused_swiglu|matmul] [--M=128] [--N=4096] [--K=4096]
//            [-o tune_result.json] [--top=3] [--measure-ms=200]
//            [--copies=0] [--dry-run]
//
// Options take llvm::cl's forms (-M 2048, --M=2048, -o out.json;
// cl_opts.h); an unknown option exits 1.
//
// Candidates are the dispatcher's launch knobs for the shape's kernel:
// M <= 64: the dispatcher's own choice (the decode tile kernel where it
// applies, else the small-M kernel's width, and splits from the cost
// models), the same kernel at k splits S in {1, 2, 3, 4, 6, 8}, then the
// small-M kernel at 32-column groups per workgroup G in {1, 2, 4} x S in
// {auto, 1, 2, 3, 4, 6, 8}; mid M (M > 64 where the dispatcher takes the
// decode tile kernel's 128- or 256-row form): that kernel at S in {auto, 1,
// 2, 3, 4, 6, 8}; tile kernels: S in {auto, 1, 2, 3, 4, 6, 8, 12, 16} (at
// least 4 k-steps of 64 per split).  Each is timed with HIP events
// (best of 3 windows of --measure-ms after a warm-up); the --top fastest
// are written as schedule_db.json records in the reference schema with this
// target's field meaning (BN = 32 G for the small-M kernel, 0 for the
// decode tile kernel, the tile's columns for the tile kernels; grain_size =
// S; 0 = the dispatcher chooses), best first, so that
// the loader's first-match rule picks the best.  --copies rotates weight sets (default:
// enough to exceed the 256 MB MALL for small M, 1 otherwise).
#include <hip/hip_runtime_api.h>

#include <algorithm>
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
  std::fprintf(stderr, "llk-tune: %s: %s\n", what, msg);
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

struct Candidate {
  int G = 0;  // small-M workgroup width; 0: chosen by the dispatcher (or tile kernel)
  int S = 0;  // 0: auto
  llk_launch_plan plan{};
  double us = 0.0;
};

}  // namespace

int main(int argc, char** argv) {
  std::string op = "fused_swiglu", outp = "tune_result.json";
  int64_t M = 128, N = 4096, K = 4096, top_opt = 3, measure_ms = 200, copies_opt = 0;
  bool dry = false;
  llk_tools::Options cl("llk-tune", "LLK autotuning search (gfx950, measured)");
  cl.add_str("op", &op, "Operation: fused_swiglu or matmul");
  cl.add_int("M", &M, "M dimension (rows)");
  cl.add_int("N", &N, "N dimension (hidden)");
  cl.add_int("K", &K, "K dimension (input)");
  cl.add_str("o", &outp, "Output JSON file");
  cl.add_int("top", &top_opt, "Records written, best first");
  cl.add_int("measure-ms", &measure_ms, "Measurement milliseconds per window");
  cl.add_int("copies", &copies_opt, "Weight sets rotated between launches (0: automatic)");
  cl.add_flag("dry-run", &dry, "Generate configs without measuring");
  if (!cl.parse(argc, argv)) return 1;
  const int top = (int)std::max<int64_t>(1, top_opt);
  const bool swiglu = op == "fused_swiglu";
  if (!swiglu && op != "matmul") die("--op", "fused_swiglu or matmul");
  if (M < 1 || N < 1 || K < 1) die("shape", "M, N, K must be positive");
  const int opcode = swiglu ? 0 : 3;
  const int nmat = swiglu ? 2 : 1;
  const int bucket = llk_classify_m(M);
  const bool small = M <= 64;
  const int64_t KB = (K + 63) / 64;
  // Mid M: the dispatcher's own plan for this shape (aligned X) is the
  // decode tile kernel; its k splits follow decode_splits.
  llk_launch_plan own{};
  check_llk(llk_describe_launch(swiglu ? 0 : 3, M, N, K, 1, &own), "describe");
  const bool midm = !small && own.kernel == 3;
  const bool dsplits = small || midm;  // candidates set decode_splits, not tile_splits
  int copies = (int)copies_opt;
  if (copies <= 0) {
    const double wbytes = 2.0 * nmat * (double)K * N;
    copies = small ? (int)std::min(8.0, std::ceil(3.0 * 256e6 / wbytes)) : 1;
    copies = std::max(1, copies);
  }

  // Candidate list (knob settings), each with the plan it produces.
  std::vector<Candidate> cands;
  const int gs[] = {1, 2, 4};
  const int small_s[] = {0, 1, 2, 3, 4, 6, 8};
  const int tile_s[] = {0, 1, 2, 3, 4, 6, 8, 12, 16};
  int64_t saved_g = 0, saved_ds = 0, saved_ts = 0;
  check_llk(llk_get_tunable("decode_group_width", &saved_g), "tunable");
  check_llk(llk_get_tunable("decode_splits", &saved_ds), "tunable");
  check_llk(llk_get_tunable("tile_splits", &saved_ts), "tunable");
  auto apply = [&](const Candidate& c) {
    check_llk(llk_set_tunable("decode_group_width", small ? c.G : saved_g), "tunable");
    check_llk(llk_set_tunable(dsplits ? "decode_splits" : "tile_splits", c.S), "tunable");
  };
  auto restore = [&]() {
    (void)llk_set_tunable("decode_group_width", saved_g);
    (void)llk_set_tunable("decode_splits", saved_ds);
    (void)llk_set_tunable("tile_splits", saved_ts);
  };
  if (small) {
    cands.push_back({0, 0});  // the dispatcher's own choice (kernel, width and splits)
    for (int s : small_s)     // its kernel (the decode tile kernel where it applies) at S
      if (s > 0 && s <= KB) cands.push_back({0, s});
    for (int g : gs)
      for (int s : small_s)
        if (s <= KB) cands.push_back({g, s});
  } else if (midm) {
    for (int s : small_s)
      if (s <= KB) cands.push_back({0, s});
  } else {
    for (int s : tile_s)
      if (s == 0 || s == 1 || KB / s >= 4) cands.push_back({0, s});
  }
  for (auto& c : cands) {
    apply(c);
    check_llk(llk_describe_launch(opcode, M, N, K, 1, &c.plan), "describe");
  }
  restore();
  // Drop candidates that produce the same launch as an earlier one.
  std::vector<Candidate> uniq;
  for (const auto& c : cands) {
    bool dup = false;
    for (const auto& u : uniq)
      dup |= u.plan.kernel == c.plan.kernel && u.plan.splits == c.plan.splits &&
             u.plan.group_width == c.plan.group_width && (u.S == 0) == (c.S == 0) &&
             (u.G == 0) == (c.G == 0);
    if (!dup) uniq.push_back(c);
  }
  cands.swap(uniq);
  std::printf("M=%lld (bucket %d) N=%lld K=%lld op=%s kernel=%s\n", (long long)M, bucket,
              (long long)N, (long long)K, op.c_str(),
              small ? "small_m" : midm ? "decode_tile (mid M)" : "mfma_tile");
  std::printf("Generated %zu candidate launches\n", cands.size());

  if (!dry) {
    char arch[64] = {0};
    int cus = 0, lds = 0, clk = 0;
    check_llk(llk_device_info(arch, sizeof arch, &cus, &lds, &clk), "device");
    std::vector<uint16_t> x((size_t)M * K), w((size_t)K * N);
    check_llk(llk_fill_normal_bf16(42, 0, 1.0f, x.data(), (int64_t)x.size(), 0), "fill");
    std::vector<llk_packed_weights*> packed;
    for (int c = 0; c < copies; ++c)
      for (int p = 0; p < nmat; ++p) {
        check_llk(llk_fill_normal_bf16(42 + 1000 * c, 1 + p, 1.0f / std::sqrt((float)K), w.data(),
                                       (int64_t)w.size(), 0),
                  "fill");
        llk_tensor2d wt{w.data(), K, N, N, 1};
        llk_packed_weights* pw = nullptr;
        check_llk(llk_pack_weights(&wt, 64, 0, &pw), "pack");
        packed.push_back(pw);
      }
    void *dx = nullptr, *dy = nullptr;
    check_hip(hipMalloc(&dx, x.size() * 2), "hipMalloc");
    check_hip(hipMalloc(&dy, (size_t)M * N * 2), "hipMalloc");
    check_hip(hipMemcpy(dx, x.data(), x.size() * 2, hipMemcpyHostToDevice), "copy");
    hipStream_t stream;
    check_hip(hipStreamCreate(&stream), "stream");
    llk_tensor2d xt{dx, M, K, K, 1}, yt{dy, M, N, N, 1};
    llk_kernel_context ctx{nullptr, 0, stream};
    int64_t it = 0;
    auto launch = [&]() {
      const int c = (int)(it++ % copies);
      check_llk(swiglu ? llk_swiglu_bf16(&xt, packed[2 * c], packed[2 * c + 1], &yt, LLK_BF16, &ctx)
                       : llk_gemm_bf16(&xt, packed[c], &yt, LLK_BF16, &ctx),
                "launch");
    };
    hipEvent_t e0, e1;
    check_hip(hipEventCreate(&e0), "event");
    check_hip(hipEventCreate(&e1), "event");
    // Bring the GPU to its steady clock once (~35 ms of load needed).
    apply(cands.front());
    const double t0 = now_ms();
    do {
      for (int i = 0; i < 10; ++i) launch();
      check_hip(hipStreamSynchronize(stream), "sync");
    } while (now_ms() - t0 < 200.0);
    for (auto& c : cands) {
      apply(c);
      for (int i = 0; i < 10; ++i) launch();  // allocate workspace, settle
      check_hip(hipStreamSynchronize(stream), "sync");
      double best = 0.0;
      for (int r = 0; r < 3; ++r) {
        int64_t iters = 0;
        const double w0 = now_ms();
        check_hip(hipEventRecord(e0, stream), "record");
        do {
          for (int i = 0; i < 10; ++i) launch();
          iters += 10;
          check_hip(hipEventRecord(e1, stream), "record");
          check_hip(hipEventSynchronize(e1), "sync");
        } while (now_ms() - w0 < (double)measure_ms);
        float ms = 0.f;
        check_hip(hipEventElapsedTime(&ms, e0, e1), "elapsed");
        const double us = 1000.0 * ms / (double)iters;
        if (best == 0.0 || us < best) best = us;
      }
      c.us = best;
    }
    restore();
    for (auto* pw : packed) llk_packed_weights_free(pw);
    (void)hipFree(dx);
    (void)hipFree(dy);
    (void)hipStreamDestroy(stream);
    std::stable_sort(cands.begin(), cands.end(),
                     [](const Candidate& a, const Candidate& b) { return a.us < b.us; });
  }

  const double flops = 2.0 * nmat * (double)M * N * K;
  const double bytes = 2.0 * nmat * (double)K * N + 2.0 * M * K + 2.0 * M * N;
  std::printf("\n%s candidates:\n", dry ? "Generated" : "Measured");
  for (size_t i = 0; i < cands.size(); ++i) {
    const auto& c = cands[i];
    std::printf("  [%zu] G=%s S=%s -> splits=%d group_width=%d workgroups=%lld", i,
                c.G ? std::to_string(c.G).c_str() : "auto",
                c.S ? std::to_string(c.S).c_str() : "auto", c.plan.splits, c.plan.group_width,
                (long long)c.plan.workgroups);
    if (!dry)
      std::printf("  %.2f us  %.1f TFLOP/s  %.1f GB/s", c.us, flops / c.us / 1e6, bytes / c.us / 1e3);
    std::printf("\n");
  }

  FILE* f = std::fopen(outp.c_str(), "w");
  if (!f) die("output", outp.c_str());
  std::fprintf(f, "{\n  \"version\": 1,\n  \"comment\": \"llk-tune %s M=%lld N=%lld K=%lld on "
                  "gfx950; best first\",\n  \"entries\": [\n",
               op.c_str(), (long long)M, (long long)N, (long long)K);
  const int count = std::min<int>(top, (int)cands.size());
  for (int i = 0; i < count; ++i) {
    const auto& c = cands[i];
    const bool sm = c.plan.kernel == 0 || c.plan.kernel == 3;  // small-M or decode tile
    // BM: rows per workgroup (the decode tile kernel: 64, or 128 / 256 at mid M)
    const int64_t BM = c.plan.kernel == 0   ? (M <= 32 ? 32 : 64)
                       : c.plan.kernel == 3 ? (M <= 64 ? 64 : M <= 128 ? 128 : 256)
                                            : 256;
    // BN 0 / grain_size 0: the dispatcher chooses for each shape (for M <= 64
    // the decode tile kernel where it applies, else the small-M kernel's
    // width); VM x VN is the MFMA tile (small-M and decode tile kernels
    // 32x32x16, tile kernels 16x16x32)
    const int64_t BN = c.plan.kernel == 0 ? (c.G ? 32 * c.plan.group_width : 0)
                                          : sm ? 0 : c.plan.tile_columns;
    std::fprintf(f,
                 "    {\"operation\": \"%s\", \"target\": \"gfx950\", \"shape\": {\"M_bucket\": %d, "
                 "\"N\": %lld, \"K\": %lld}, \"dtype\": \"bf16\", \"math_mode\": \"strict\",\n"
                 "     \"schedule\": {\"BM\": %lld, \"BN\": %lld, \"BK\": %d, \"VM\": %d, \"VN\": %d, "
                 "\"vector_width\": 8, \"num_threads\": %lld, \"parallel_axis\": \"%s\", "
                 "\"grain_size\": %d},\n     \"source\": \"llk-tune\", \"measured_us\": %.3f}%s\n",
                 op.c_str(), bucket, (long long)N, (long long)K, (long long)BM, (long long)BN,
                 sm ? 64 : 32, sm ? 32 : 16, sm ? 32 : 16, (long long)c.plan.threads_per_workgroup, sm ? "n" : "mn", c.S, c.us,
                 i + 1 < count ? "," : "");
  }
  std::fprintf(f, "  ]\n}\n");
  if (std::fclose(f) != 0) die("output", "write failed");
  std::printf("Wrote top-%d configs to %s\n", count, outp.c_str());
  return 0;
}
