// kernel_cache.cpp -- C ABI of the four-level cache (llk_cache_* in
// include/llk/llk_abi.h), built on LruLevel and the library's public entry
// points only.
#include "kernel_cache.h"

#include <memory>
#include <new>
#include <string>

#include "kernel_key.h"
#include "llk/llk_abi.h"

namespace llk {
int setError(int code, const char* msg);  // llk_abi.cpp
// The entry point of an operation's gfx950 code object (code_object.cpp).
int code_object_entry(int operation, int out_dtype, const std::string& dir, llk_kernel_fn* out);
}

struct llk_jit_cache {
  llk::LruLevel<std::string> ir;         // L1
  llk::LruLevel<std::string> optimized;  // L2
  llk::LruLevel<llk_kernel_fn> object;   // L3
  llk::LruLevel<std::shared_ptr<llk_packed_weights>> weights;  // L4
  std::string object_dir;  // where the code objects are read (empty: the default)
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

// The entry point a key selects: the operation's gfx950 code object (read,
// checked and loaded by code_object_entry) with the key's output type bound
// in.  Keys of other targets, dtypes or operations are errors: this backend
// builds no code at run time.
int select_entry(const llk_jit_cache* c, const llk_kernel_key& k, llk_kernel_fn* out) {
  if (k.isa != static_cast<uint8_t>(llk::Isa::GFX950))
    return llk::setError(LLK_ERR_UNSUPPORTED_ARCH, "kernel key isa is not gfx950 (7)");
  if (k.input_type != LLK_BF16)
    return llk::setError(LLK_ERR_DTYPE, "kernel key input type must be bf16");
  if (k.output_type != LLK_BF16 && k.output_type != LLK_FP32)
    return llk::setError(LLK_ERR_DTYPE, "kernel key output type must be bf16 or f32");
  if (k.N < 1 || k.K < 1) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "kernel key N, K < 1");
  switch (static_cast<llk::OperationKind>(k.operation)) {
    case llk::OperationKind::FusedSwiGLU:
    case llk::OperationKind::Matmul:
      return llk::code_object_entry(k.operation, k.output_type, c->object_dir, out);
    default:
      return llk::setError(LLK_ERR_INVALID_ARGUMENT,
                           "kernel key operation has no gfx950 kernel (RoPE and attention are "
                           "outside this backend)");
  }
}

}  // namespace

extern "C" {

int llk_cache_create(llk_jit_cache** out) {
  if (!out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = new (std::nothrow) llk_jit_cache();
  return *out ? LLK_OK : llk::setError(LLK_ERR_OUT_OF_MEMORY, "cache allocation");
}

void llk_cache_destroy(llk_jit_cache* c) { delete c; }

int llk_cache_lookup_or_compile(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn* out) {
  if (!c || !key || !out) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  const std::string skey = to_key(*key).serialize();
  if (c->object.lookup(skey, out)) return LLK_OK;
  llk_kernel_fn fn = nullptr;
  int rc = select_entry(c, *key, &fn);
  if (rc) return rc;
  c->object.insert(skey, fn);
  *out = fn;
  return LLK_OK;
}

int llk_cache_set_object_dir(llk_jit_cache* c, const char* dir) {
  if (!c) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  c->object_dir = dir ? dir : "";
  return LLK_OK;
}

int llk_cache_lookup_object_code(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn* out) {
  if (!c || !key) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  return c->object.lookup(to_key(*key).serialize(), out) ? 1 : 0;
}

int llk_cache_insert_object_code(llk_jit_cache* c, const llk_kernel_key* key, llk_kernel_fn fn) {
  if (!c || !key) return llk::setError(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  c->object.insert(to_key(*key).serialize(), fn);
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
  llk_weight_key key;
  key.weight_ptr = w->data;
  key.shape_hash = llk::key_mix(llk::key_mix(llk::key_mix(0x9ae16a3b2f90404fULL ^
                                                          (uint64_t)w->dim0) ^
                                             (uint64_t)w->dim1) ^
                                (uint64_t)w->stride0);
  key.BK = bk;
  key.BN = 128;
  if (llk_cache_lookup_packed_weights(c, &key, out) == 1) return LLK_OK;
  llk_packed_weights* pw = nullptr;
  int rc = on_device ? llk_pack_weights_device(w, bk, nullptr, &pw)
                     : llk_pack_weights(w, bk, flags, &pw);
  if (rc) return rc;
  if ((rc = llk_cache_insert_packed_weights(c, &key, pw))) return rc;  // pw freed on failure
  *out = pw;
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
