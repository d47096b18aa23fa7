// llk-compile -- the gfx950 counterpart of the reference's compiler driver
// (tools/llk-compile/llk-compile.cpp:209-319).
//
//   llk-compile <input.mlir> [--M=<dim>] [--N=<dim>] [--K=<dim>]
//               [--schedule-db=<path>] [--quiet]
//
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
#include <sstream>
#include <string>
#include <vector>

#include "llk/llk_abi.h"

namespace {

struct TensorType {
  std::vector<int64_t> dims;  // -1 = dynamic
  std::string elem;
};

struct OpInfo {
  std::string func, kind;  // kind: fused_swiglu | matmul
  std::vector<TensorType> ins, outs;
  std::string math_mode = "bounded_fast";
  int line = 0;
};

bool parse_tensor(const std::string& s, size_t pos, TensorType* t, size_t* end) {
  // tensor<AxBx...xELEM>
  const size_t open = s.find('<', pos), close = s.find('>', pos);
  if (open == std::string::npos || close == std::string::npos || close < open) return false;
  const std::string body = s.substr(open + 1, close - open - 1);
  std::vector<std::string> parts;
  std::stringstream ss(body);
  std::string p;
  while (std::getline(ss, p, 'x')) parts.push_back(p);
  if (parts.empty()) return false;
  t->elem = parts.back();
  t->dims.clear();
  for (size_t i = 0; i + 1 < parts.size(); ++i) {
    if (parts[i] == "?") {
      t->dims.push_back(-1);
    } else {
      char* e = nullptr;
      const long long v = std::strtoll(parts[i].c_str(), &e, 10);
      if (!e || *e) return false;
      t->dims.push_back(v);
    }
  }
  *end = close + 1;
  return true;
}

// Tensor types after the ':' of an ins(...) / outs(...) group.
bool parse_group(const std::string& s, size_t start, const char* tag, std::vector<TensorType>* out,
                 size_t* end) {
  const size_t g = s.find(tag, start);
  if (g == std::string::npos) return false;
  const size_t close = s.find(')', g);
  const size_t colon = s.find(':', g);
  if (close == std::string::npos || colon == std::string::npos || colon > close) return false;
  size_t pos = colon;
  while (true) {
    const size_t t = s.find("tensor<", pos);
    if (t == std::string::npos || t > close) break;
    TensorType tt;
    size_t e;
    if (!parse_tensor(s, t, &tt, &e)) return false;
    out->push_back(tt);
    pos = e;
  }
  *end = close + 1;
  return true;
}

std::vector<OpInfo> scan(const std::string& text, std::string* err) {
  std::vector<OpInfo> ops;
  std::string func = "<module>";
  size_t pos = 0;
  while (pos < text.size()) {
    const size_t f = text.find("func.func @", pos);
    const size_t a = text.find("llk.fused_swiglu", pos);
    const size_t b = text.find("llk.matmul", pos);
    const size_t op = std::min(a, b);
    if (op == std::string::npos) break;
    if (f != std::string::npos && f < op) {
      const size_t n0 = f + 11, n1 = text.find_first_of("( ", n0);
      func = "@" + text.substr(n0, n1 - n0);
      pos = n1;
      continue;
    }
    OpInfo o;
    o.func = func;
    o.kind = (op == a) ? "fused_swiglu" : "matmul";
    o.line = 1 + (int)std::count(text.begin(), text.begin() + op, '\n');
    size_t e1, e2;
    if (!parse_group(text, op, "ins(", &o.ins, &e1) ||
        !parse_group(text, e1, "outs(", &o.outs, &e2)) {
      *err = "line " + std::to_string(o.line) + ": cannot parse operands of llk." + o.kind;
      return {};
    }
    const size_t attr = text.find('{', e2), arrow = text.find("->", e2);
    if (attr != std::string::npos && (arrow == std::string::npos || attr < arrow)) {
      const size_t close = text.find('}', attr);
      const std::string dict = text.substr(attr, close - attr);
      const size_t mm = dict.find("#llk.math_mode<");
      if (mm != std::string::npos) {
        const size_t s0 = mm + 15, s1 = dict.find('>', s0);
        o.math_mode = dict.substr(s0, s1 - s0);
      }
    }
    ops.push_back(o);
    pos = e2;
  }
  return ops;
}

int64_t arg_value(int argc, char** argv, const char* name, int64_t dflt, bool* ok) {
  const size_t n = std::strlen(name);
  for (int i = 1; i < argc; ++i) {
    if (std::strncmp(argv[i], name, n) != 0) continue;
    const char* v = nullptr;
    if (argv[i][n] == '=') v = argv[i] + n + 1;
    else if (argv[i][n] == '\0' && i + 1 < argc) v = argv[i + 1];
    if (!v) continue;
    char* e = nullptr;
    const long long x = std::strtoll(v, &e, 10);
    if (!e || *e) *ok = false;
    return x;
  }
  return dflt;
}

std::string arg_string(int argc, char** argv, const char* name, const std::string& dflt) {
  const size_t n = std::strlen(name);
  for (int i = 1; i < argc; ++i)
    if (std::strncmp(argv[i], name, n) == 0 && argv[i][n] == '=') return argv[i] + n + 1;
  return dflt;
}

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
  std::string input;
  for (int i = 1; i < argc; ++i) {
    if (argv[i][0] != '-') {
      // a bare value following "--M" etc. is not the input
      if (i > 1 && argv[i - 1][0] == '-' && std::strchr(argv[i - 1], '=') == nullptr &&
          std::strcmp(argv[i - 1], "--quiet") != 0)
        continue;
      input = argv[i];
      break;
    }
  }
  if (input.empty())
    return fail("usage: llk-compile <input.mlir> [--M=<dim>] [--N=<dim>] [--K=<dim>] "
                "[--schedule-db=<path>] [--quiet]");
  bool ok = true;
  const int64_t optM = arg_value(argc, argv, "--M", 0, &ok);
  const int64_t optN = arg_value(argc, argv, "--N", 0, &ok);
  const int64_t optK = arg_value(argc, argv, "--K", 0, &ok);
  if (!ok) return fail("--M/--N/--K take integers");
  const std::string db = arg_string(argc, argv, "--schedule-db", default_db(argv[0]));
  bool quiet = false;
  for (int i = 1; i < argc; ++i) quiet |= std::strcmp(argv[i], "--quiet") == 0;

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
    llk_kernel_fn fn = nullptr;
    if (llk_cache_lookup_or_compile(cache, &key, &fn) != LLK_OK) {
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
                  plan.kernel ? "mfma_tile" : "small_m", plan.splits, plan.group_width, plan.pad_x,
                  (long long)plan.workgroups, (long long)plan.threads_per_workgroup,
                  (long long)plan.launches, plan.workspace_bytes);
    }
  }
  llk_cache_destroy(cache);
  if (rc) return rc;
  std::printf("Compilation successful\n");
  return 0;
}
