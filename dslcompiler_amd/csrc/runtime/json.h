// json.h -- minimal JSON reader for schedule databases (objects, arrays,
// strings, numbers, true/false/null).  Enough for the schedule_db.json
// record format; not a general-purpose library.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace llk {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  bool is_integer = false;  // the literal had no fraction or exponent
  int64_t integer = 0;
  std::string str;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;  // insertion order

  const Value* get(const std::string& key) const {
    if (kind != Object) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  // llvm::json::Object::getInteger semantics: present and an integer.
  bool getInteger(const std::string& key, int64_t* out) const {
    const Value* v = get(key);
    if (!v || v->kind != Number || !v->is_integer) return false;
    *out = v->integer;
    return true;
  }
  const std::string* getString(const std::string& key) const {
    const Value* v = get(key);
    return (v && v->kind == String) ? &v->str : nullptr;
  }
  const Value* getObject(const std::string& key) const {
    const Value* v = get(key);
    return (v && v->kind == Object) ? v : nullptr;
  }
  const Value* getArray(const std::string& key) const {
    const Value* v = get(key);
    return (v && v->kind == Array) ? v : nullptr;
  }
};

// Returns false (and leaves *out unspecified) on malformed input.
bool parse(const std::string& text, Value* out);

}  // namespace json
}  // namespace llk
