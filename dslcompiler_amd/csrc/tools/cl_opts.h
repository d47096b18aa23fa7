// cl_opts.h -- command-line options for the tools in the forms the
// reference's tools accept through llvm::cl (tools/llk-bench/llk-bench.cpp:
// 21-35, tools/llk-tune/llk-tune.cpp:21-31, tools/llk-compile/
// llk-compile.cpp:76-82):
//
//   -name=value  --name=value  -name value  --name value   (value options)
//   -name  --name  -name=true|false|1|0                      (flags)
//   positional arguments, and "--" to end the options
//   -help / --help prints the options and exits 0
//
// An unknown option, a missing or malformed value, or a missing or extra
// positional argument is reported on stderr and the tool exits 1, as
// llvm::cl::ParseCommandLineOptions does (the messages follow its wording).
#pragma once

#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace llk_tools {

// Name of llk_launch_plan::kernel.
inline const char* kernel_name(int kernel) {
  return kernel == 0 ? "small_m" : kernel == 1 ? "mfma_tile" : kernel == 2 ? "swiglu_wide"
                                                                          : "decode_tile";
}

class Options {
 public:
  Options(const char* tool, const char* overview) : tool_(tool), overview_(overview) {}

  void add_int(const char* name, int64_t* v, const char* desc) {
    opts_.push_back({name, desc, kInt, v, nullptr, nullptr});
  }
  void add_str(const char* name, std::string* v, const char* desc) {
    opts_.push_back({name, desc, kStr, nullptr, v, nullptr});
  }
  void add_flag(const char* name, bool* v, const char* desc) {
    opts_.push_back({name, desc, kFlag, nullptr, nullptr, v});
  }
  // Positional arguments, in order; `required` of them must be given.
  void add_positional(std::string* v, const char* desc, bool required) {
    pos_.push_back({v, desc, required});
  }

  // Parses argv into the registered variables (defaults are what they hold
  // before the call).  Exits 0 after printing help; returns false after
  // reporting an error (the caller exits 1).
  bool parse(int argc, char** argv) {
    size_t npos = 0;
    bool only_positional = false;
    for (int i = 1; i < argc; ++i) {
      const char* a = argv[i];
      if (only_positional || a[0] != '-' || a[1] == '\0') {
        if (npos >= pos_.size()) return error("Too many positional arguments specified!");
        *pos_[npos++].value = a;
        continue;
      }
      if (std::strcmp(a, "--") == 0) {
        only_positional = true;
        continue;
      }
      const char* body = a + (a[1] == '-' ? 2 : 1);
      const char* eq = std::strchr(body, '=');
      const std::string name = eq ? std::string(body, eq - body) : std::string(body);
      if (name == "help") {
        print_help();
        std::exit(0);
      }
      Opt* o = find(name);
      if (!o)
        return error(std::string("Unknown command line argument '") + a + "'.  Try: '" + tool_ +
                     " --help'");
      if (o->kind == kFlag) {
        if (!eq) {
          *o->flag = true;
        } else if (!std::strcmp(eq + 1, "true") || !std::strcmp(eq + 1, "1")) {
          *o->flag = true;
        } else if (!std::strcmp(eq + 1, "false") || !std::strcmp(eq + 1, "0")) {
          *o->flag = false;
        } else {
          return error(std::string("for the -") + name + " option: '" + (eq + 1) +
                       "' is invalid value for boolean argument! Try 0 or 1");
        }
        continue;
      }
      std::string value;
      if (eq) {
        value = eq + 1;
      } else if (i + 1 < argc) {
        value = argv[++i];
      } else {
        return error(std::string("for the -") + name + " option: requires a value!");
      }
      if (o->kind == kStr) {
        *o->str = value;
        continue;
      }
      errno = 0;
      char* end = nullptr;
      const long long v = std::strtoll(value.c_str(), &end, 0);
      if (value.empty() || !end || *end || errno == ERANGE)
        return error(std::string("for the -") + name + " option: '" + value +
                     "' value invalid for integer argument!");
      *o->num = v;
    }
    for (size_t k = npos; k < pos_.size(); ++k)
      if (pos_[k].required)
        return error("Not enough positional command line arguments specified!\nMust specify at "
                     "least 1 positional argument: See: " + tool_ + " --help");
    return true;
  }

 private:
  enum Kind { kInt, kStr, kFlag };
  struct Opt {
    const char* name;
    const char* desc;
    Kind kind;
    int64_t* num;
    std::string* str;
    bool* flag;
  };
  struct Pos {
    std::string* value;
    const char* desc;
    bool required;
  };

  Opt* find(const std::string& name) {
    for (Opt& o : opts_)
      if (name == o.name) return &o;
    return nullptr;
  }

  bool error(const std::string& msg) {
    std::fprintf(stderr, "%s: %s\n", tool_.c_str(), msg.c_str());
    return false;
  }

  void print_help() const {
    std::printf("OVERVIEW: %s\n\nUSAGE: %s [options]", overview_.c_str(), tool_.c_str());
    for (const Pos& p : pos_) std::printf(" %s", p.desc);
    std::printf("\n\nOPTIONS:\n");
    for (const Opt& o : opts_) {
      const char* arg = o.kind == kInt ? "=<int>" : o.kind == kStr ? "=<string>" : "";
      std::string left = std::string("--") + o.name + arg;
      std::printf("  %-24s - %s\n", left.c_str(), o.desc);
    }
  }

  std::string tool_, overview_;
  std::vector<Opt> opts_;
  std::vector<Pos> pos_;
};

}  // namespace llk_tools
