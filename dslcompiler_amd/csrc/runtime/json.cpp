// json.cpp -- recursive-descent reader for json.h.
#include "json.h"

#include <cctype>
#include <cmath>
#include <cstdlib>

namespace llk {
namespace json {
namespace {

struct Parser {
  const std::string& s;
  size_t i = 0;
  int depth = 0;

  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
  }
  bool lit(const char* w) {
    size_t n = 0;
    while (w[n]) ++n;
    if (s.compare(i, n, w) != 0) return false;
    i += n;
    return true;
  }
  static void put_utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
      o += static_cast<char>(cp);
    } else if (cp < 0x800) {
      o += static_cast<char>(0xc0 | (cp >> 6));
      o += static_cast<char>(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      o += static_cast<char>(0xe0 | (cp >> 12));
      o += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      o += static_cast<char>(0x80 | (cp & 0x3f));
    } else {
      o += static_cast<char>(0xf0 | (cp >> 18));
      o += static_cast<char>(0x80 | ((cp >> 12) & 0x3f));
      o += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      o += static_cast<char>(0x80 | (cp & 0x3f));
    }
  }
  bool hex4(uint32_t* cp) {
    if (i + 4 > s.size()) return false;
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      char c = s[i++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else return false;
    }
    *cp = v;
    return true;
  }
  bool string(std::string* out) {
    if (i >= s.size() || s[i] != '"') return false;
    ++i;
    out->clear();
    while (i < s.size()) {
      char c = s[i++];
      if (c == '"') return true;
      if (static_cast<unsigned char>(c) < 0x20) return false;
      if (c != '\\') {
        *out += c;
        continue;
      }
      if (i >= s.size()) return false;
      char e = s[i++];
      switch (e) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xd800 && cp < 0xdc00) {  // surrogate pair
            uint32_t lo;
            if (!lit("\\u") || !hex4(&lo) || lo < 0xdc00 || lo >= 0xe000) return false;
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          put_utf8(*out, cp);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  bool number(Value* v) {
    size_t st = i;
    if (i < s.size() && s[i] == '-') ++i;
    if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) return false;
    if (s[i] == '0') ++i;
    else while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
    bool integral = true;
    if (i < s.size() && s[i] == '.') {
      integral = false;
      ++i;
      if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) return false;
      while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
    }
    if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
      integral = false;
      ++i;
      if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
      if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) return false;
      while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
    }
    std::string tok = s.substr(st, i - st);
    v->kind = Value::Number;
    v->num = std::strtod(tok.c_str(), nullptr);
    v->is_integer = integral;
    if (integral) v->integer = std::strtoll(tok.c_str(), nullptr, 10);
    return true;
  }
  bool value(Value* v) {
    if (++depth > 256) return false;
    ws();
    if (i >= s.size()) return false;
    char c = s[i];
    bool ok = false;
    if (c == '{') {
      ++i;
      v->kind = Value::Object;
      ws();
      if (i < s.size() && s[i] == '}') {
        ++i;
        ok = true;
      } else {
        for (;;) {
          ws();
          std::string key;
          if (!string(&key)) break;
          ws();
          if (i >= s.size() || s[i] != ':') break;
          ++i;
          Value child;
          if (!value(&child)) break;
          v->obj.emplace_back(std::move(key), std::move(child));
          ws();
          if (i < s.size() && s[i] == ',') {
            ++i;
            continue;
          }
          if (i < s.size() && s[i] == '}') {
            ++i;
            ok = true;
          }
          break;
        }
      }
    } else if (c == '[') {
      ++i;
      v->kind = Value::Array;
      ws();
      if (i < s.size() && s[i] == ']') {
        ++i;
        ok = true;
      } else {
        for (;;) {
          Value child;
          if (!value(&child)) break;
          v->arr.push_back(std::move(child));
          ws();
          if (i < s.size() && s[i] == ',') {
            ++i;
            continue;
          }
          if (i < s.size() && s[i] == ']') {
            ++i;
            ok = true;
          }
          break;
        }
      }
    } else if (c == '"') {
      v->kind = Value::String;
      ok = string(&v->str);
    } else if (c == 't') {
      v->kind = Value::Bool;
      v->b = true;
      ok = lit("true");
    } else if (c == 'f') {
      v->kind = Value::Bool;
      ok = lit("false");
    } else if (c == 'n') {
      v->kind = Value::Null;
      ok = lit("null");
    } else {
      ok = number(v);
    }
    --depth;
    return ok;
  }
};

}  // namespace

bool parse(const std::string& text, Value* out) {
  Parser p{text};
  *out = Value();
  if (!p.value(out)) return false;
  p.ws();
  return p.i == text.size();
}

}  // namespace json
}  // namespace llk
