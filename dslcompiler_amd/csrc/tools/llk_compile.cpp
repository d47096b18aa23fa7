// llk-compile -- the gfx950 counterpart of the reference's compiler driver
// (tools/llk-compile/llk-compile.cpp:209-319).
//
//   llk-compile <input.mlir> [--M=<dim>] [--N=<dim>] [--K=<dim>]
//               [--schedule-db=<path>] [--quiet]
//
// Options take llvm::cl's forms (-M 2048, --M=2048; cl_opts.h); an unknown
// option or a missing input exits 1.
// Reads an MLIR module with llk.fused_swiglu / llk.matmul ops in the
// reference's textual form, checks every op with the reference verifier's
// rules (llk_verify_fused_swiglu / llk_verify_matmul), resolves dynamic
// dimensions from --M/--N/--K, and for each op reports what the reference
// pipeline would decide and what this backend launches: the M bucket
// (ShapeSpecialization), the schedule DB entry (ScheduleSelection), the
// KernelKey and its hash, and the gfx950 entry point and launch plan
// obtained through the kernel cache (JitCache::lookupOrCompile).  Kernels
// are compiled ahead of time, so nothing is generated here.  Prints
// "Compilation successful" and exits 0, or reports the first error and
// exits 1, as the reference tool does.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

#include "cl_opts.h"
#include "llk/llk_abi.h"
#include "runtime/mlir_scan.h"

namespace {

using llk::mlir_scan::OpInfo;
using llk::mlir_scan::scan;

std::string default_db(const char* argv0) {
  std::string exe = argv0;
  const size_t slash = exe.rfind('/');
  const std::string dir = slash == std::string::npos ? "." : exe.substr(0, slash);
  return dir + "/../schedules/gfx950/schedule_db.json";
}

int fail(const std::string& msg) {
  std::fprintf(stderr, "%s\n", msg.c_str());
  return 1;
}

}  // namespace

int main(int argc, char** argv) {
  std::string input, db = default_db(argv[0]);
  int64_t optM = 0, optN = 0, optK = 0;
  bool quiet = false;
  llk_tools::Options cl("llk-compile", "LLK compiler driver (gfx950)");
  cl.add_positional(&input, "<input .mlir>", true);
  cl.add_int("M", &optM, "M dimension (rows)");
  cl.add_int("N", &optN, "N dimension (cols)");
  cl.add_int("K", &optK, "K dimension (hidden)");
  cl.add_str("schedule-db", &db, "Schedule database (schedule_db.json)");
  cl.add_flag("quiet", &quiet, "Print only the final line");
  if (!cl.parse(argc, argv)) return 1;

  std::ifstream f(input);
  if (!f) return fail("Failed to parse " + input);
  std::stringstream buf;
  buf << f.rdbuf();
  std::string err;
  const std::vector<OpInfo> ops = scan(buf.str(), &err);
  if (!err.empty()) return fail("Failed to parse " + input + ": " + err);
  if (ops.empty()) return fail("Failed to parse " + input + ": no llk.fused_swiglu or llk.matmul op");

  llk_jit_cache* cache = nullptr;
  if (llk_cache_create(&cache) != LLK_OK) return fail(llk_last_error());
  int rc = 0;
  for (const OpInfo& o : ops) {
    const std::string where = input + ":" + std::to_string(o.line) + ": '" + "llk." + o.kind + "' op ";
    const size_t want_ins = o.kind == "fused_swiglu" ? 3 : 2;
    if (o.ins.size() != want_ins || o.outs.size() != 1) {
      rc = fail(where + "expects " + std::to_string(want_ins) + " inputs and 1 init");
      break;
    }
    bool rank_ok = true;
    for (const auto& t : o.ins) rank_ok &= t.dims.size() == 2;
    rank_ok &= o.outs[0].dims.size() == 2;
    if (!rank_ok) {
      rc = fail(where + (o.kind == "fused_swiglu" ? "X, Wg, Wu and init must be 2D tensors"
                                                  : "requires rank-2 inputs"));
      break;
    }
    bool bf16 = true;
    for (const auto& t : o.ins) bf16 &= t.elem == "bf16";
    if (!bf16) {
      rc = fail(where + "inputs must be bf16 tensors");
      break;
    }
    int64_t M, N, K;
    int vr;
    int out_dtype = LLK_BF16;
    if (o.kind == "fused_swiglu") {
      const auto &x = o.ins[0].dims, &wg = o.ins[1].dims, &wu = o.ins[2].dims, &in = o.outs[0].dims;
      vr = llk_verify_fused_swiglu(x[0], x[1], wg[0], wg[1], wu[0], wu[1], in[0], in[1]);
      M = x[0] >= 0 ? x[0] : in[0];
      K = x[1] >= 0 ? x[1] : (wg[0] >= 0 ? wg[0] : wu[0]);
      N = wg[1] >= 0 ? wg[1] : (wu[1] >= 0 ? wu[1] : in[1]);
      if (o.outs[0].elem != "bf16") {
        rc = fail(where + "result must be a bf16 tensor");
        break;
      }
    } else {
      const auto &a = o.ins[0].dims, &b = o.ins[1].dims, &in = o.outs[0].dims;
      vr = llk_verify_matmul(a[1], b[0]);
      M = a[0] >= 0 ? a[0] : in[0];
      K = a[1] >= 0 ? a[1] : b[0];
      N = b[1] >= 0 ? b[1] : in[1];
      const std::string& e = o.outs[0].elem;
      if (e == "f32") out_dtype = LLK_FP32;
      else if (e != "bf16") {
        rc = fail(where + "result type " + e + " has no gfx950 kernel (bf16 or f32)");
        break;
      }
    }
    if (vr != LLK_OK) {
      rc = fail(where + llk_last_error());
      break;
    }
    if (M < 0) M = optM;
    if (N < 0) N = optN;
    if (K < 0) K = optK;
    if (M <= 0 || N <= 0 || K <= 0) {
      rc = fail(where + "dynamic dimension: pass --M/--N/--K");
      break;
    }
    const int bucket = llk_classify_m(M);
    llk_schedule_entry se;
    int nmatch = 0;
    const char* db_op = o.kind == "fused_swiglu" ? "fused_swiglu" : "matmul";
    const int dbrc = llk_select_schedule(db.c_str(), db_op, bucket, &se, &nmatch);
    llk_kernel_key key{};
    key.operation = o.kind == "fused_swiglu" ? 0 : 3;
    key.input_type = LLK_BF16;
    key.output_type = (uint8_t)out_dtype;
    key.M_bucket = bucket;
    key.N = N;
    key.K = K;
    key.weight_layout = 2;
    key.isa = 7;
    key.math_mode = o.math_mode == "strict" ? 0 : o.math_mode == "unsafe_fast" ? 2 : 1;
    key.thread_count = 1;
    key.compiler_version = 1;
    key.schedule_version = 1;
    llk_kernel_fn fn = nullptr;  // the key's entry (also checks the op has a gfx950 kernel)
    if (llk_cache_lookup_or_compile_packed(cache, &key, &fn) != LLK_OK) {
      rc = fail(where + llk_last_error());
      break;
    }
    llk_launch_plan plan;
    if (llk_describe_launch(key.operation, M, N, K, 1, &plan) != LLK_OK) {
      rc = fail(where + llk_last_error());
      break;
    }
    const uint64_t h = llk_kernel_key_hash(key.operation, key.input_type, key.output_type,
                                           key.M_bucket, key.N, key.K, key.weight_layout, key.isa,
                                           key.math_mode, key.thread_count,
                                           key.compiler_version, key.schedule_version);
    if (!quiet) {
      std::printf("%s: llk.%s M=%lld N=%lld K=%lld -> bucket %d\n", o.func.c_str(), o.kind.c_str(),
                  (long long)M, (long long)N, (long long)K, bucket);
      std::printf("  schedule%s: BM=%lld BN=%lld BK=%lld VM=%lld VN=%lld vector_width=%lld "
                  "num_threads=%lld grain_size=%lld parallel_axis=%s\n",
                  dbrc == LLK_OK ? (nmatch ? "" : " (default)") : " (default: DB unreadable)",
                  (long long)se.BM, (long long)se.BN, (long long)se.BK, (long long)se.VM,
                  (long long)se.VN, (long long)se.vector_width, (long long)se.num_threads,
                  (long long)se.grain_size, se.parallel_axis);
      std::printf("  key=0x%016llx math_mode=%s\n", (unsigned long long)h, o.math_mode.c_str());
      std::printf("  kernel=%s splits=%d group_width=%d pad_x=%d workgroups=%lld threads=%lld "
                  "launches=%lld workspace=%zu\n",
                  llk_tools::kernel_name(plan.kernel), plan.splits, plan.group_width, plan.pad_x,
                  (long long)plan.workgroups, (long long)plan.threads_per_workgroup,
                  (long long)plan.launches, plan.workspace_bytes);
    }
  }
  if (!rc) {
    // The module's KernelFn under the key the reference's driver derives
    // (llk-compile.cpp:298-310): "llk_" + hash of the module text + the
    // --M/--N/--K values.  (The reference hashes the module as printed after
    // its pipeline; here the input text is hashed.)
    const std::string text = buf.str();
    const std::string cacheKey = "llk_" + std::to_string(std::hash<std::string>{}(text)) + "_M" +
                                 std::to_string(optM) + "_N" + std::to_string(optN) + "_K" +
                                 std::to_string(optK);
    llk_memref_kernel_fn fn = nullptr;
    if (llk_cache_lookup_or_compile_str(cache, cacheKey.c_str(), text.data(), text.size(), &fn) !=
        LLK_OK) {
      rc = fail(std::string("JIT compilation failed: ") + llk_last_error());
    } else if (!quiet) {
      std::printf("entry: %s\n", cacheKey.c_str());
    }
  }
  llk_cache_destroy(cache);
  if (rc) return rc;
  std::printf("Compilation successful\n");
  return 0;
}
