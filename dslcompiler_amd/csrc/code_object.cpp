// code_object.cpp -- the gfx950 code objects behind the object-code level
// (L3) of the kernel cache: one per operation, llk_fused_swiglu_gfx950.hsaco
// and llk_matmul_gfx950.hsaco, built ahead of time from the kernel sources
// (dslcompiler_amd/build.py) into the library's objects/ directory.  A
// kernel key's object is read and checked (a 64-bit AMDGPU ELF for gfx950
// that defines kernels), loaded per device with hipModuleLoadData, and its
// kernels resolved with hipModuleGetFunction; the entry point handed back
// runs the operation with that object's kernels.  This is the counterpart
// of the reference's per-key compile-and-lookup (JitCache.cpp:182-245: the
// module is lowered and added to the JIT, its exported entry symbol looked
// up and cached by key), with the compile moved ahead of time: the
// kernels take N and K at run time, so the object is per operation, and
// the key's output type is bound into the entry.
#include <dlfcn.h>
#include <elf.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>

#include <array>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "llk/llk_abi.h"

#ifndef EM_AMDGPU
#define EM_AMDGPU 224
#endif

namespace llk {
// A code object loaded on one device: its module and every kernel by name.
struct ModuleFns {
  hipModule_t module = nullptr;
  std::unordered_map<std::string, hipFunction_t> fns;
};

int setError(int code, const char* msg);  // llk_abi.cpp
int swiglu_with_module(const llk_tensor2d* x, const llk_packed_weights* wg,
                       const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                       llk_kernel_context* ctx, const ModuleFns* mod);
int gemm_with_module(const llk_tensor2d* a, const llk_packed_weights* b, llk_tensor2d* c,
                     int c_dtype, llk_kernel_context* ctx, const ModuleFns* mod,
                     bool accumulate);
// The KernelFn-shaped call (kernel_fn.cpp) and its thread's status.
int memref_call(int op, int out_dtype, const ModuleFns* mod, llk_memref2d* x, llk_memref2d* wg,
                llk_memref2d* wu, llk_memref2d* init, llk_memref2d* result);
void set_kernel_fn_status(int rc);

hipFunction_t module_function(const ModuleFns* m, const char* symbol) {
  auto it = m->fns.find(symbol);
  return it == m->fns.end() ? nullptr : it->second;
}
}  // namespace llk

namespace {

constexpr int kMaxDevices = 64;
constexpr uint32_t kMachGfx950 = 0x4f;  // EF_AMDGPU_MACH_AMDGCN_GFX950
constexpr int kOpSwiglu = 0, kOpMatmul = 3;  // OperationKind (KernelKey.h:22-27)

int err(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int err(int code, const char* fmt, ...) {
  char buf[768];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return llk::setError(code, buf);
}

// Checks that `b` is a 64-bit little-endian AMDGPU ELF for gfx950 and lists
// its kernels: the symbols with a kernel descriptor, "<name>.kd".
int inspect(const std::vector<uint8_t>& b, const std::string& path,
            std::vector<std::string>* kernels) {
  kernels->clear();
  Elf64_Ehdr eh;
  if (b.size() < sizeof(eh))
    return err(LLK_ERR_INVALID_ARGUMENT, "%s: not a code object (%zu bytes)", path.c_str(),
               b.size());
  std::memcpy(&eh, b.data(), sizeof(eh));
  if (std::memcmp(eh.e_ident, ELFMAG, SELFMAG) != 0 || eh.e_ident[EI_CLASS] != ELFCLASS64 ||
      eh.e_ident[EI_DATA] != ELFDATA2LSB)
    return err(LLK_ERR_INVALID_ARGUMENT, "%s: not a 64-bit little-endian ELF code object",
               path.c_str());
  if (eh.e_machine != EM_AMDGPU)
    return err(LLK_ERR_UNSUPPORTED_ARCH, "%s: ELF machine %u is not AMDGPU (%u)", path.c_str(),
               (unsigned)eh.e_machine, (unsigned)EM_AMDGPU);
  if ((eh.e_flags & 0xffu) != kMachGfx950)
    return err(LLK_ERR_UNSUPPORTED_ARCH, "%s: code object is for AMDGPU mach 0x%x, not gfx950 (0x%x)",
               path.c_str(), eh.e_flags & 0xffu, kMachGfx950);
  const size_t shnum = eh.e_shnum;
  if (eh.e_shentsize != sizeof(Elf64_Shdr) || eh.e_shoff > b.size() ||
      shnum > (b.size() - eh.e_shoff) / sizeof(Elf64_Shdr))
    return err(LLK_ERR_INVALID_ARGUMENT, "%s: malformed section headers", path.c_str());
  std::vector<Elf64_Shdr> sh(shnum);
  if (shnum) std::memcpy(sh.data(), b.data() + eh.e_shoff, shnum * sizeof(Elf64_Shdr));
  auto in_file = [&](const Elf64_Shdr& s) { return s.sh_offset <= b.size() && s.sh_size <= b.size() - s.sh_offset; };
  for (const Elf64_Shdr& s : sh) {
    if (s.sh_type != SHT_DYNSYM && s.sh_type != SHT_SYMTAB) continue;
    if (!in_file(s) || s.sh_entsize != sizeof(Elf64_Sym) || s.sh_link >= shnum ||
        !in_file(sh[s.sh_link]))
      return err(LLK_ERR_INVALID_ARGUMENT, "%s: malformed symbol table", path.c_str());
    const Elf64_Shdr& str = sh[s.sh_link];
    const char* strtab = reinterpret_cast<const char*>(b.data() + str.sh_offset);
    for (size_t i = 0; i < s.sh_size / sizeof(Elf64_Sym); ++i) {
      Elf64_Sym sym;
      std::memcpy(&sym, b.data() + s.sh_offset + i * sizeof(Elf64_Sym), sizeof(sym));
      if (sym.st_name >= str.sh_size) continue;
      const size_t len = strnlen(strtab + sym.st_name, str.sh_size - sym.st_name);
      const std::string name(strtab + sym.st_name, len);
      if (len > 3 && name.compare(len - 3, 3, ".kd") == 0) kernels->push_back(name.substr(0, len - 3));
    }
    if (s.sh_type == SHT_DYNSYM && !kernels->empty()) break;  // the dynamic table suffices
  }
  if (kernels->empty())
    return err(LLK_ERR_INVALID_ARGUMENT, "%s: code object defines no kernels", path.c_str());
  return LLK_OK;
}

int read_file(const std::string& path, std::vector<uint8_t>* out) {
  struct stat st;
  if (::stat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode))
    return err(LLK_ERR_NOT_FOUND, "no gfx950 code object at %s", path.c_str());
  std::ifstream f(path, std::ios::binary);
  if (!f) return err(LLK_ERR_NOT_FOUND, "cannot open code object %s", path.c_str());
  try {
    out->assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  } catch (const std::bad_alloc&) {
    return err(LLK_ERR_OUT_OF_MEMORY, "reading %s", path.c_str());
  }
  return LLK_OK;
}

// One operation's code object: read and checked once per process (by
// path), loaded on each device at first use there; modules stay loaded
// until the process ends, so an entry point handed out stays valid.
struct CodeObject {
  std::string path;
  int operation = 0;
  std::vector<uint8_t> image;
  std::vector<std::string> kernels;
  std::mutex mu;
  std::array<std::unique_ptr<llk::ModuleFns>, kMaxDevices> dev;
};

std::mutex g_mu;
std::map<std::string, std::unique_ptr<CodeObject>> g_objects;

int open_object(const std::string& path, int operation, CodeObject** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_objects.find(path);
  if (it != g_objects.end()) {
    *out = it->second.get();
    return LLK_OK;
  }
  auto obj = std::make_unique<CodeObject>();
  obj->path = path;
  obj->operation = operation;
  int rc = read_file(path, &obj->image);
  if (!rc) rc = inspect(obj->image, path, &obj->kernels);
  if (rc) return rc;
  *out = obj.get();
  g_objects.emplace(path, std::move(obj));
  return LLK_OK;
}

// The object's functions on the current device, loading it there first.
int module_on_current_device(CodeObject* obj, const llk::ModuleFns** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0) return err(LLK_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (dev >= kMaxDevices) return err(LLK_ERR_NO_DEVICE, "device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(obj->mu);
  if (!obj->dev[dev]) {
    auto m = std::make_unique<llk::ModuleFns>();
    e = hipModuleLoadData(&m->module, obj->image.data());
    if (e != hipSuccess)
      return err(LLK_ERR_HIP, "hipModuleLoadData(%s) on device %d: %s", obj->path.c_str(), dev,
                 hipGetErrorString(e));
    for (const std::string& k : obj->kernels) {
      hipFunction_t f = nullptr;
      e = hipModuleGetFunction(&f, m->module, k.c_str());
      if (e != hipSuccess) {
        (void)hipModuleUnload(m->module);
        return err(LLK_ERR_HIP, "hipModuleGetFunction(%s) in %s: %s", k.c_str(),
                   obj->path.c_str(), hipGetErrorString(e));
      }
      m->fns.emplace(k, f);
    }
    obj->dev[dev] = std::move(m);
  }
  *out = obj->dev[dev].get();
  return LLK_OK;
}

// Entry points: a fixed pool of functions, each bound to one (object,
// output type) pair when first handed out; slot i has an entry of each
// shape, kEntries[i] (llk_kernel_fn: packed handles, a context) and
// kMemrefEntries[i] (the reference's KernelFn: five MemRef2D).
struct Slot {
  CodeObject* obj = nullptr;
  int out_dtype = 0;
};
constexpr int kSlots = 64;
std::array<Slot, kSlots> g_slots;
int g_nslots = 0;

Slot slot_of(int i) {
  std::lock_guard<std::mutex> lk(g_mu);
  return g_slots[i];
}

int run_slot(int i, const llk_tensor2d* x, const llk_packed_weights* w0,
             const llk_packed_weights* w1, llk_tensor2d* y, int y_dtype,
             llk_kernel_context* ctx) {
  const Slot sl = slot_of(i);
  if (!sl.obj) return err(LLK_ERR_INVALID_ARGUMENT, "unbound code-object entry %d", i);
  if (y_dtype != sl.out_dtype)
    return err(LLK_ERR_DTYPE, "entry of a key with output type %d called with output type %d",
               sl.out_dtype, y_dtype);
  const llk::ModuleFns* m = nullptr;
  int rc = module_on_current_device(sl.obj, &m);
  if (rc) return rc;
  if (sl.obj->operation == kOpSwiglu) return llk::swiglu_with_module(x, w0, w1, y, y_dtype, ctx, m);
  return llk::gemm_with_module(x, w0, y, y_dtype, ctx, m, false);
}

// The KernelFn shape: no return value; the status is the thread's
// llk_kernel_fn_status().
void run_memref_slot(int i, llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu,
                     llk_memref2d* init, llk_memref2d* result) {
  const Slot sl = slot_of(i);
  if (!sl.obj) {
    llk::set_kernel_fn_status(err(LLK_ERR_INVALID_ARGUMENT, "unbound code-object entry %d", i));
    return;
  }
  const llk::ModuleFns* m = nullptr;
  const int rc = module_on_current_device(sl.obj, &m);
  if (rc) {
    llk::set_kernel_fn_status(rc);
    return;
  }
  (void)llk::memref_call(sl.obj->operation, sl.out_dtype, m, x, wg, wu, init, result);
}

template <int I>
int slot_entry(const llk_tensor2d* x, const llk_packed_weights* w0, const llk_packed_weights* w1,
               llk_tensor2d* y, int y_dtype, llk_kernel_context* ctx) {
  return run_slot(I, x, w0, w1, y, y_dtype, ctx);
}

template <int I>
void memref_slot_entry(llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu, llk_memref2d* init,
                       llk_memref2d* result) {
  run_memref_slot(I, x, wg, wu, init, result);
}

template <int... I>
constexpr std::array<llk_kernel_fn, sizeof...(I)> slot_entries(std::integer_sequence<int, I...>) {
  return {&slot_entry<I>...};
}
template <int... I>
constexpr std::array<llk_memref_kernel_fn, sizeof...(I)> memref_slot_entries(
    std::integer_sequence<int, I...>) {
  return {&memref_slot_entry<I>...};
}
constexpr std::array<llk_kernel_fn, kSlots> kEntries =
    slot_entries(std::make_integer_sequence<int, kSlots>{});
constexpr std::array<llk_memref_kernel_fn, kSlots> kMemrefEntries =
    memref_slot_entries(std::make_integer_sequence<int, kSlots>{});

const char* object_file(int operation) {
  return operation == kOpSwiglu ? "llk_fused_swiglu_gfx950.hsaco"
                                : operation == kOpMatmul ? "llk_matmul_gfx950.hsaco" : nullptr;
}

std::string default_dir() {
  const char* env = std::getenv("LLK_CODE_OBJECT_DIR");
  if (env && *env) return env;
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&default_dir), &info) && info.dli_fname) {
    std::string lib = info.dli_fname;
    const size_t slash = lib.rfind('/');
    return (slash == std::string::npos ? std::string(".") : lib.substr(0, slash)) + "/objects";
  }
  return "objects";
}

std::string object_path(int operation, const char* dir) {
  const std::string d = (dir && *dir) ? std::string(dir) : default_dir();
  return d + "/" + object_file(operation);
}

}  // namespace

namespace llk {

// The entry points of (operation, out_dtype) from the operation's code
// object in `dir` (empty: the default directory), in both shapes.  The
// caller has checked the key.  The object is read and checked here; with a
// device present it is also loaded on the current device, so that a bad
// object is reported now.
int code_object_entry(int operation, int out_dtype, const std::string& dir, llk_kernel_fn* packed,
                      llk_memref_kernel_fn* memref) {
  if (!object_file(operation))
    return err(LLK_ERR_INVALID_ARGUMENT, "operation %d has no gfx950 code object", operation);
  CodeObject* obj = nullptr;
  int rc = open_object(object_path(operation, dir.c_str()), operation, &obj);
  if (rc) return rc;
  int count = 0;
  if (hipGetDeviceCount(&count) == hipSuccess && count > 0) {
    const ModuleFns* m = nullptr;
    if ((rc = module_on_current_device(obj, &m))) return rc;
  } else {
    (void)hipGetLastError();
  }
  std::lock_guard<std::mutex> lk(g_mu);
  int i = 0;
  while (i < g_nslots && !(g_slots[i].obj == obj && g_slots[i].out_dtype == out_dtype)) ++i;
  if (i == g_nslots) {
    if (g_nslots == kSlots)
      return err(LLK_ERR_OUT_OF_MEMORY, "more than %d (code object, output type) entry points",
                 kSlots);
    g_slots[g_nslots++] = Slot{obj, out_dtype};
  }
  *packed = kEntries[i];
  *memref = kMemrefEntries[i];
  return LLK_OK;
}

}  // namespace llk

extern "C" {

int llk_code_object_path(int operation, const char* dir, char* buf, size_t cap) {
  if (!object_file(operation))
    return err(LLK_ERR_INVALID_ARGUMENT, "operation %d has no gfx950 code object", operation);
  const std::string p = object_path(operation, dir);
  if (buf && cap) std::snprintf(buf, cap, "%s", p.c_str());
  return (int)p.size();
}

int llk_code_object_info(const char* path, int* kernel_count, char* names, size_t cap,
                         size_t* len) {
  if (!path) return err(LLK_ERR_INVALID_ARGUMENT, "path is NULL");
  std::vector<uint8_t> image;
  std::vector<std::string> kernels;
  int rc = read_file(path, &image);
  if (!rc) rc = inspect(image, path, &kernels);
  if (rc) return rc;
  if (kernel_count) *kernel_count = (int)kernels.size();
  std::string all;
  for (const std::string& k : kernels) all += k + "\n";
  if (len) *len = all.size();
  if (names && cap) {
    const size_t n = all.size() < cap - 1 ? all.size() : cap - 1;
    std::memcpy(names, all.data(), n);
    names[n] = '\0';
  }
  return LLK_OK;
}

}  // extern "C"
