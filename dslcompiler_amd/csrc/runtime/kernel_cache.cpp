// kernel_cache.cpp -- C ABI of the four-level cache (llk_cache_* in
// include/llk/llk_abi.h), built on LruLevel and the library's public entry
// points only.
#include "kernel_cache.h"

#include <condition_variable>
#include <memory>
#include <new>
#include <set>
#include <string>
#include <unordered_map>

#include "kernel_key.h"
#include "llk/llk_abi.h"
#include "mlir_scan.h"

namespace llk {
int setError(int code, const char* msg);  // llk_abi.cpp
// The entry points of an operation's gfx950 code object (code_object.cpp):
// the packed-handle shape and the KernelFn (MemRef2D) shape.
int code_object_entry(int operation, int out_dtype, const std::string& dir, llk_kernel_fn* packed,
                      llk_memref_kernel_fn* memref);

// An object-code (L3) entry: both shapes of one (code object, output type).
struct L3Entry {
  llk_kernel_fn packed = nullptr;
  llk_memref_kernel_fn memref = nullptr;
};
}  // namespace llk

struct llk_jit_cache {
  llk::LruLevel<std::string> ir;         // L1
  llk::LruLevel<std::string> optimized;  // L2
  llk::LruLevel<llk::L3Entry> object;    // L3
  llk::LruLevel<std::shared_ptr<llk_packed_weights>> weights;  // L4
  std::string object_dir;  // where the code objects are read (empty: the default)
  // L4 get-or-pack runs one pack per key at a time: keys being packed, and
  // the waiters for them.
  std::mutex pack_mu;
  std::condition_variable pack_cv;
  std::set<std::string> packing;
  // Counted references handed out by llk_cache_acquire_packed_weights.
  std::mutex held_mu;
  std::unordered_map<const llk_packed_weights*,
                     std::pair<std::shared_ptr<llk_packed_weights>, size_t>>
      held;
};

namespace {

llk::KernelKey to_key(const llk_kernel_key& k) {
  llk::KernelKey key;
  key.operation = static_cast<llk::OperationKind>(k.operation);
  key.input_type = static_cast<llk::DType>(k.input_type);
  key.output_type = static_cast<llk::DType>(k.output_type);
  key.M_bucket = k.M_bucket;
  key.N = k.N;
  key.K = k.K;
  key.weight_layout = static_cast<llk::Layout>(k.weight_layout);
  key.isa = static_cast<llk::Isa>(k.isa);
  key.math_mode = static_cast<llk::MathMode>(k.math_mode);
  key.thread_count = k.thread_count;
  key.compiler_version = k.compiler_version;
  key.schedule_version = k.schedule_version;
  return key;
}

std::string weight_key_string(const llk_weight_key& k) {
  llk::WeightKey w;
  w.weight_ptr = k.weight_ptr;
  w.shape_hash = k.shape_hash;
  w.BK = k.BK;
  w.BN = k.BN;
  return w.serialize();
}

// Checks a key against what this backend builds: gfx950, bf16 input, an
// output type the operation has (SwiGLU bf16 or f32 -- the op's bf16 result
// and its pre-truncf value; matmul bf16, f16 or f32 as llk.matmul allows),
// and an operation with a gfx950 kernel.
int check_key(const llk_kernel_key& k) {
  if (k.isa != static_cast<uint8_t>(llk::Isa::GFX950))
    return llk::setError(LLK_ERR_UNSUPPORTED_ARCH, "kernel key isa is not gfx950 (7)");
  if (k.input_type != LLK_BF16)
    return llk::setError(LLK_ERR_DTYPE, "kernel key input type must be bf16");
  const auto op = static_cast<llk::OperationKind>(k.operation);
  if (op != llk::OperationKind::FusedSwiGLU && op != llk::OperationKind::Matmul)
    return llk::setError(LLK_ERR_INVALID_ARGUMENT,
                         "kernel key operation has no gfx950 kernel (RoPE and attention are "
                         "outside this backend)");
  const bool out_ok = k.output_type == LLK_BF16 || k.output_type == LLK_FP32 ||
                      (op == llk::OperationKind::Matmul && k.output_type == LLK_FP16);
  if (!out_ok)
    return llk::setError(LLK_ERR_DTYPE, op == llk::OperationKind::Matmul
                                            ? "kernel key output type must be bf16, f16 or f32"
                                            : "kernel key output type must be bf16 or f32");
  if (k.N < 1 || k.K < 1) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "kernel key N, K < 1");
  return LLK_OK;
}

// The L3 entry under `skey`: a hit, or on a miss the entry points of the
// operation's gfx950 code object (read, checked and loaded by
// code_object_entry) with the output type bound in, inserted under skey.
// This backend builds no code at run time.  Nothing is inserted on an error.
int l3_get(llk_jit_cache* c, const std::string& skey, int operation, int out_dtype,
           llk::L3Entry* out) {
  if (c->object.lookup(skey, out) && out->packed && out->memref) return LLK_OK;
  llk::L3Entry e;
  const int rc = llk::code_object_entry(operation, out_dtype, c->object_dir, &e.packed, &e.memref);
  if (rc) return rc;
  c->object.insert(skey, e);
  *out = e;
  return LLK_OK;
}

}  // namespace

namespace llk {

// L4 get-or-pack as a counted reference: the handle stays valid while `out`
// (or a copy) lives, whatever the level does meanwhile.  One pack per key:
// a caller that finds the key being packed waits for that pack.
int cache_get_shared(llk_jit_cache* c, const llk_tensor2d* w, int64_t bk, int on_device,
                     unsigned flags, std::shared_ptr<llk_packed_weights>* out) {
  if (!c || !w || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  out->reset();
  llk_weight_key key;
  key.weight_ptr = w->data;
  key.shape_hash = llk::key_mix(llk::key_mix(llk::key_mix(0x9ae16a3b2f90404fULL ^
                                                          (uint64_t)w->dim0) ^
                                             (uint64_t)w->dim1) ^
                                (uint64_t)w->stride0);
  key.BK = bk;
  key.BN = 128;
  const std::string sk = weight_key_string(key);
  {
    std::unique_lock<std::mutex> lk(c->pack_mu);
    for (;;) {
      if (c->weights.lookup(sk, out)) return LLK_OK;
      if (c->packing.count(sk) == 0) break;
      c->pack_cv.wait(lk);
    }
    try {
      c->packing.insert(sk);
    } catch (const std::bad_alloc&) {
      return llk::setError(LLK_ERR_OUT_OF_MEMORY, "cache bookkeeping");
    }
  }
  // Whatever happens below, the key stops being "in flight" and the
  // waiters look again.
  struct Done {
    llk_jit_cache* c;
    const std::string& sk;
    ~Done() {
      {
        std::lock_guard<std::mutex> lk(c->pack_mu);
        c->packing.erase(sk);
      }
      c->pack_cv.notify_all();
    }
  } done{c, sk};
  llk_packed_weights* pw = nullptr;
  int rc = on_device ? llk_pack_weights_device(w, bk, nullptr, &pw)
                     : llk_pack_weights(w, bk, flags, &pw);
  if (rc) return rc;
  try {
    std::shared_ptr<llk_packed_weights> h(pw, &llk_packed_weights_free);
    c->weights.insert(sk, h);
    *out = std::move(h);
  } catch (const std::bad_alloc&) {
    return llk::setError(LLK_ERR_OUT_OF_MEMORY, "cache insertion");  // pw freed by h
  }
  return LLK_OK;
}

}  // namespace llk

extern "C" {

int llk_cache_create(llk_jit_cache** out) {
  if (!out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = new (std::nothrow) llk_jit_cache();
  return *out ? LLK_OK : llk::setError(LLK_ERR_OUT_OF_MEMORY, "cache allocation");
}

void llk_cache_destroy(llk_jit_cache* c) { delete c; }

int llk_cache_lookup_or_compile(llk_jit_cache* c, const llk_kernel_key* key,
                                llk_memref_kernel_fn* out) {
  if (!c || !key || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  int rc = check_key(*key);
  if (rc) return rc;
  llk::L3Entry e;
  if ((rc = l3_get(c, to_key(*key).serialize(), key->operation, key->output_type, &e))) return rc;
  *out = e.memref;
  return LLK_OK;
}

int llk_cache_lookup_or_compile_packed(llk_jit_cache* c, const llk_kernel_key* key,
                                       llk_kernel_fn* out) {
  if (!c || !key || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  int rc = check_key(*key);
  if (rc) return rc;
  llk::L3Entry e;
  if ((rc = l3_get(c, to_key(*key).serialize(), key->operation, key->output_type, &e))) return rc;
  *out = e.packed;
  return LLK_OK;
}

int llk_cache_lookup_or_compile_str(llk_jit_cache* c, const char* cache_key, const char* module,
                                    size_t module_len, llk_memref_kernel_fn* out) {
  if (!c || !cache_key || !module || !out)
    return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  const std::string skey(cache_key);
  llk::L3Entry e;
  if (c->object.lookup(skey, &e) && e.memref) {
    *out = e.memref;
    return LLK_OK;
  }
  std::string err;
  const auto ops = llk::mlir_scan::scan(std::string(module, module_len), &err);
  if (!err.empty()) return llk::setError(LLK_ERR_INVALID_ARGUMENT, ("Lowering passes failed: " + err).c_str());
  if (ops.empty())
    return llk::setError(LLK_ERR_INVALID_ARGUMENT, "No exported kernel entry point found in module");
  // The module's entry is its first op (the reference takes the first
  // external function: JitCache.cpp:214-220).
  const auto& o = ops.front();
  llk_kernel_key k{};
  k.operation = o.kind == "fused_swiglu" ? 0 : 3;
  k.input_type = LLK_BF16;
  for (const auto& t : o.ins)
    if (t.elem != "bf16") return llk::setError(LLK_ERR_DTYPE, "module inputs must be bf16 tensors");
  const std::string res = o.outs.empty() ? "" : o.outs[0].elem;
  k.output_type = res == "bf16" ? LLK_BF16 : res == "f32" ? LLK_FP32 : res == "f16" ? LLK_FP16 : 255;
  k.isa = static_cast<uint8_t>(llk::Isa::GFX950);
  k.N = k.K = 1;  // the entry takes N and K at run time
  int rc = check_key(k);
  if (rc) return rc;
  if ((rc = l3_get(c, skey, k.operation, k.output_type, &e))) return rc;
  *out = e.memref;
  return LLK_OK;
}

int llk_cache_set_object_dir(llk_jit_cache* c, const char* dir) {
  if (!c) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  c->object_dir = dir ? dir : "";
  return LLK_OK;
}

int llk_cache_lookup_object_code(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn* out) {
  if (!c || !key) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  llk::L3Entry e;
  if (!c->object.lookup(to_key(*key).serialize(), &e)) return 0;
  if (out) *out = e.packed;
  return 1;
}

int llk_cache_insert_object_code(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn fn) {
  if (!c || !key) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  llk::L3Entry e;
  e.packed = fn;  // no KernelFn-shaped entry: a later lookup_or_compile makes one
  c->object.insert(to_key(*key).serialize(), e);
  return LLK_OK;
}

static llk::LruLevel<std::string>* string_level(llk_jit_cache* c, int level) {
  return level == 1 ? &c->ir : level == 2 ? &c->optimized : nullptr;
}

int llk_cache_insert_blob(llk_jit_cache* c, int level, const char* key, size_t key_len,
                          const void* value, size_t value_len) {
  if (!c || (!key && key_len) || (!value && value_len))
    return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  auto* lv = string_level(c, level);
  if (!lv) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "blob levels are 1 and 2");
  lv->insert(std::string(key ? key : "", key_len),
             std::string(static_cast<const char*>(value ? value : ""), value_len));
  return LLK_OK;
}

int llk_cache_lookup_blob(llk_jit_cache* c, int level, const char* key, size_t key_len, void* out,
                          size_t cap, size_t* len) {
  if (!c || (!key && key_len)) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  auto* lv = string_level(c, level);
  if (!lv) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "blob levels are 1 and 2");
  std::string v;
  if (!lv->lookup(std::string(key ? key : "", key_len), &v)) return 0;
  if (len) *len = v.size();
  if (out && cap) v.copy(static_cast<char*>(out), cap < v.size() ? cap : v.size());
  return 1;
}

int llk_cache_insert_packed_weights(llk_jit_cache* c, const llk_weight_key* key,
                                    llk_packed_weights* pw) {
  if (!c || !key || !pw) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  // Re-inserting the handle a key already holds only refreshes the entry
  // (a second owner of the same handle would free it twice).
  try {
    c->weights.insert_with(
        weight_key_string(*key),
        [pw](const std::shared_ptr<llk_packed_weights>& h) { return h.get() == pw; },
        [pw] { return std::shared_ptr<llk_packed_weights>(pw, &llk_packed_weights_free); });
  } catch (const std::bad_alloc&) {
    // The owning shared_ptr (made or being made) has freed pw.
    return llk::setError(LLK_ERR_OUT_OF_MEMORY, "cache insertion");
  }
  return LLK_OK;
}

int llk_cache_lookup_packed_weights(llk_jit_cache* c, const llk_weight_key* key,
                                    llk_packed_weights** out) {
  if (!c || !key) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  std::shared_ptr<llk_packed_weights> h;
  if (!c->weights.lookup(weight_key_string(*key), &h)) return 0;
  if (out) *out = h.get();
  return 1;
}

int llk_cache_get_packed_weights(llk_jit_cache* c, const llk_tensor2d* w, int64_t bk,
                                 int on_device, unsigned flags, llk_packed_weights** out) {
  if (!c || !w || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  std::shared_ptr<llk_packed_weights> h;
  const int rc = llk::cache_get_shared(c, w, bk, on_device, flags, &h);
  if (rc) return rc;
  *out = h.get();  // borrowed: the level keeps it
  return LLK_OK;
}

int llk_cache_acquire_packed_weights(llk_jit_cache* c, const llk_tensor2d* w, int64_t bk,
                                     int on_device, unsigned flags, llk_packed_weights** out) {
  if (!c || !w || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  std::shared_ptr<llk_packed_weights> h;
  const int rc = llk::cache_get_shared(c, w, bk, on_device, flags, &h);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(c->held_mu);
  try {
    auto& slot = c->held[h.get()];
    if (!slot.first) slot.first = h;
    ++slot.second;
  } catch (const std::bad_alloc&) {
    return llk::setError(LLK_ERR_OUT_OF_MEMORY, "cache bookkeeping");
  }
  *out = h.get();
  return LLK_OK;
}

int llk_cache_release_packed_weights(llk_jit_cache* c, llk_packed_weights* pw) {
  if (!c || !pw) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  std::shared_ptr<llk_packed_weights> last;  // freed after the lock, if it was the last owner
  std::lock_guard<std::mutex> lk(c->held_mu);
  auto it = c->held.find(pw);
  if (it == c->held.end())
    return llk::setError(LLK_ERR_INVALID_ARGUMENT, "handle holds no reference acquired from this cache");
  if (--it->second.second == 0) {
    last = std::move(it->second.first);
    c->held.erase(it);
  }
  return LLK_OK;
}

int llk_cache_evict_lru(llk_jit_cache* c, int level, size_t max_entries) {
  if (!c) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  switch (level) {
    case 1: c->ir.evict(max_entries); return LLK_OK;
    case 2: c->optimized.evict(max_entries); return LLK_OK;
    case 3: c->object.evict(max_entries); return LLK_OK;
    case 4: c->weights.evict(max_entries); return LLK_OK;
    default: return llk::setError(LLK_ERR_INVALID_ARGUMENT, "cache levels are 1..4");
  }
}

int llk_cache_set_max_entries(llk_jit_cache* c, int level, size_t max_entries) {
  return llk_cache_evict_lru(c, level, max_entries);
}

int llk_cache_get_stats(const llk_jit_cache* c, llk_cache_stats* out) {
  if (!c || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  c->ir.stats(&out->hits[0], &out->misses[0], &out->evictions[0]);
  c->optimized.stats(&out->hits[1], &out->misses[1], &out->evictions[1]);
  c->object.stats(&out->hits[2], &out->misses[2], &out->evictions[2]);
  c->weights.stats(&out->hits[3], &out->misses[3], &out->evictions[3]);
  return LLK_OK;
}

void llk_cache_clear(llk_jit_cache* c) {
  if (!c) return;
  c->ir.clear();
  c->optimized.clear();
  c->object.clear();
  c->weights.clear();
}

size_t llk_cache_size(const llk_jit_cache* c) {
  if (!c) return 0;
  return c->ir.size() + c->optimized.size() + c->object.size() + c->weights.size();
}

}  // extern "C"
