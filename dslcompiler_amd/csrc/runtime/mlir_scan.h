// mlir_scan.h -- a scanner for the llk.fused_swiglu / llk.matmul ops of a
// module in the reference's MLIR text form (the syntax of
// test/Dialect/LLK/*.mlir and the ops of LLKOps.td:13-67, 210-255): for
// each op, the enclosing function, its ins/outs tensor types (dims, -1 for
// '?', and element type), its math_mode attribute and its line.  Shared by
// llk-compile and the kernel cache's string-keyed lookup; header-only, no
// MLIR dependency.  Not a parser of MLIR in general: it reads exactly the
// op forms the reference's pipeline feeds the JIT.
#pragma once

#include <algorithm>
#include <cstdlib>
#include <sstream>
#include <string>
#include <vector>

namespace llk {
namespace mlir_scan {

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

inline bool parse_tensor(const std::string& s, size_t pos, TensorType* t, size_t* end) {
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
inline bool parse_group(const std::string& s, size_t start, const char* tag, std::vector<TensorType>* out,
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

inline std::vector<OpInfo> scan(const std::string& text, std::string* err) {
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

}  // namespace mlir_scan
}  // namespace llk
