// kernel_fn.cpp -- the reference's KernelFn calling convention
// (include/LLK/Runtime/JitCache.h:79-81): five MemRef2D* (x, wg, wu, init,
// result), no stream, no context, no return value, raw row-major weights.
//
// The reference's JIT'd function reads wg and wu on every call
// (swiglu_vector_avx2.cpp:278-285 passes the caller's buffers straight
// through), so by default so does this one.  Device-resident weights with
// 16-byte aligned rows go straight to a row-major form of the kernels --
// the decode tile kernel's at most 128 rows of X (the same launch and bits
// as the packed path), the tile kernel's above (the SwiGLU's 128-column
// plan, the matmul's accumulating plan, and their bits; K a multiple of 64,
// N of 8); otherwise each call packs wg
// and wu into the MFMA operand layout on the device (one pack launch per
// matrix, into a per-device buffer the library owns) and then runs the same
// kernels as llk_swiglu_bf16.  A caller whose weight buffers never change may opt into
// reusing packed handles across calls (llk_kernel_fn_assume_immutable_
// weights): they are then resolved through the L4 weight level of a
// per-device cache (WeightKey = address, shape, BK: JitCache.h:143-146,
// KernelKey.h:114-124) as counted references, so a concurrent eviction or
// clear cannot free a handle a call is using.
//
// Calls are synchronous, like the reference's CPU function: everything runs
// on the null stream and the call returns when the result is written.
// Operands may be device memory or host memory (the reference's callers
// pass host buffers); host operands are staged through device buffers.
// KernelFn calls on one device run one at a time (they share its staging
// buffers), from any number of threads.
//
// The same call serves the library's llk_swiglu_kernel_fn and the
// MemRef2D-shaped entry points the object-code level hands out
// (code_object.cpp), which pass the kernels of their loaded code object.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <memory>
#include <mutex>

#include "llk/llk_abi.h"
#include "packed_weights.h"

namespace llk {
int setError(int code, const char* msg);  // llk_abi.cpp
int swiglu_with_module(const llk_tensor2d* x, const llk_packed_weights* wg,
                       const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                       llk_kernel_context* ctx, const ModuleFns* mod);
int gemm_with_module(const llk_tensor2d* a, const llk_packed_weights* b, llk_tensor2d* c,
                     int c_dtype, llk_kernel_context* ctx, const ModuleFns* mod,
                     bool accumulate);
int rowmajor_with_module(int mode, const llk_tensor2d* x, const llk_tensor2d* wg,
                         const llk_tensor2d* wu, llk_tensor2d* y, int out_dtype,
                         llk_kernel_context* ctx, const ModuleFns* mod, bool accumulate,
                         bool* taken);
// L4 get-or-pack as a counted reference (kernel_cache.cpp).
int cache_get_shared(llk_jit_cache* c, const llk_tensor2d* w, int64_t bk, int on_device,
                     unsigned flags, std::shared_ptr<llk_packed_weights>* out);
}  // namespace llk

namespace {

constexpr int kMaxDevices = 64;
constexpr int64_t kBK = 64;  // PackWeights' kDefaultBK (PackWeights.cpp:36)
constexpr int kOpSwiglu = 0, kOpMatmul = 3;  // OperationKind (KernelKey.h:22-27)

thread_local int g_status = LLK_OK;
std::atomic<int> g_immutable{0};

struct FnDevice {
  std::mutex mu;                   // one KernelFn call at a time on the device
  llk_jit_cache* cache = nullptr;  // L4 of the calls that reuse packed weights
  void* wstage = nullptr;          // packed wg | wu of the current call
  size_t wstage_bytes = 0;
  llk_packed_weights* view[2] = {nullptr, nullptr};  // handles over wstage
  void* stage = nullptr;           // device copies of host X and result
  size_t stage_bytes = 0;
};
FnDevice g_fn[kMaxDevices];

int fail(int code, const char* msg) {
  g_status = code;
  return llk::setError(code, msg);
}
int status(int rc) {
  g_status = rc;
  return rc;
}

size_t elem_bytes(int dtype) { return dtype == LLK_FP32 ? 4 : 2; }

// Data address of a memref: aligned + offset elements.
void* memref_data(const llk_memref2d& m, size_t elem) {
  return static_cast<char*>(m.aligned) + m.offset * (int64_t)elem;
}

// True when `p` is host memory the GPU cannot address directly (pageable or
// unregistered); device, managed and pinned host memory go to the kernels.
bool is_host_only(const void* p) {
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // an unknown pointer is plain host memory
    return true;
  }
  return attr.type == hipMemoryTypeUnregistered || (attr.type == hipMemoryTypeHost &&
                                                     attr.devicePointer == nullptr);
}

int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess || *dev < 0 || *dev >= kMaxDevices)
    return fail(LLK_ERR_NO_DEVICE, "KernelFn: no current HIP device");
  return LLK_OK;
}

// Grows a device buffer to `need` bytes; its contents are not kept.  Called
// with the device's mutex held after every earlier call has synchronised,
// so no queued work still reads the old buffer.
int ensure(void** buf, size_t* bytes, size_t need, const char* what) {
  if (*bytes >= need) return LLK_OK;
  if (*buf) (void)hipFree(*buf);
  *buf = nullptr;
  *bytes = 0;
  const size_t n = std::max(need, (size_t)1 << 20);
  if (hipMalloc(buf, n) != hipSuccess) {
    *buf = nullptr;
    (void)hipGetLastError();
    return fail(LLK_ERR_OUT_OF_MEMORY, what);
  }
  *bytes = n;
  return LLK_OK;
}

int device_cache(FnDevice& d, llk_jit_cache** out) {
  if (!d.cache) {
    const int rc = llk_cache_create(&d.cache);
    if (rc) return status(rc);
  }
  *out = d.cache;
  return LLK_OK;
}

llk_tensor2d weight_tensor(const llk_memref2d& m) {
  return llk_tensor2d{memref_data(m, 2), m.size0, m.size1, m.stride0, m.stride1};
}

}  // namespace

namespace llk {

void set_kernel_fn_status(int rc) { g_status = rc; }

// A KernelFn-shaped call: operation 0 (fused SwiGLU: result =
// bf16/f32(SiLU(x wg) * (x wu)), init only shape-checked, as the
// reference's fused lowering fills its accumulators with zero:
// FuseDoubleContraction.cpp:119-135) or 3 (matmul with linalg.matmul's
// outs(init) semantics: result = init + x wg, wu unused); result elements
// of out_dtype; the kernels of `mod` (null: the library's own).
int memref_call(int op, int out_dtype, const ModuleFns* mod, llk_memref2d* x, llk_memref2d* wg,
                llk_memref2d* wu, llk_memref2d* init, llk_memref2d* result) {
  g_status = LLK_OK;
  const bool swiglu = op == kOpSwiglu;
  if (!x || !wg || (swiglu && !wu) || !init || !result)
    return fail(LLK_ERR_INVALID_ARGUMENT, "KernelFn: NULL memref");
  const int64_t M = x->size0, K = x->size1, N = wg->size1;
  int rc = swiglu ? llk_verify_fused_swiglu(M, K, wg->size0, wg->size1, wu->size0, wu->size1,
                                            init->size0, init->size1)
                  : llk_verify_matmul(K, wg->size0);
  if (rc) return status(rc);
  if (!swiglu && (init->size0 != M || init->size1 != N))
    return fail(LLK_ERR_SHAPE, "KernelFn: init shape differs from (M, N)");
  if (result->size0 != init->size0 || result->size1 != init->size1)
    return fail(LLK_ERR_SHAPE, "KernelFn: result shape differs from init");
  if (M == 0 || N == 0) return LLK_OK;
  if (x->stride1 != 1 || result->stride1 != 1 || init->stride1 != 1 || wg->stride1 != 1 ||
      (swiglu && wu->stride1 != 1))
    return fail(LLK_ERR_LAYOUT, "KernelFn: memrefs need unit inner stride");
  int dev;
  if ((rc = current_device(&dev))) return rc;
  FnDevice& d = g_fn[dev];
  std::lock_guard<std::mutex> lk(d.mu);
  const size_t ye = elem_bytes(out_dtype);
  hipStream_t s = nullptr;

  // X and the result: in place when the GPU can address them, else through
  // dense device copies.
  llk_tensor2d xt{memref_data(*x, 2), M, K, x->stride0, 1};
  llk_tensor2d yt{memref_data(*result, ye), M, N, result->stride0, 1};
  void* const init_data = memref_data(*init, ye);
  const bool x_host = K > 0 && is_host_only(xt.data);
  const bool y_host = is_host_only(yt.data);
  const size_t xbytes = x_host ? ((size_t)M * K * 2 + 255) / 256 * 256 : 0;
  const size_t ybytes = y_host ? (size_t)M * N * ye : 0;
  if (xbytes + ybytes > 0 &&
      (rc = ensure(&d.stage, &d.stage_bytes, xbytes + ybytes, "KernelFn: staging buffer")))
    return rc;
  uint8_t* const base = static_cast<uint8_t*>(d.stage);
  hipError_t e = hipSuccess;
  if (x_host) {
    e = hipMemcpy2DAsync(base, (size_t)K * 2, xt.data, (size_t)x->stride0 * 2, (size_t)K * 2,
                         (size_t)M, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return fail(LLK_ERR_HIP, hipGetErrorString(e));
    xt = llk_tensor2d{base, M, K, K, 1};
  }
  void* const y_user = yt.data;
  if (y_host) yt = llk_tensor2d{base + xbytes, M, N, N, 1};
  // matmul: result = init + x wg, computed in place in the result after
  // init has been copied there (nothing to copy when init is the result).
  if (!swiglu && (y_host || init_data != y_user)) {
    e = hipMemcpy2DAsync(yt.data, (size_t)yt.stride0 * ye, init_data, (size_t)init->stride0 * ye,
                         (size_t)N * ye, (size_t)M, hipMemcpyDefault, s);
    if (e != hipSuccess) return fail(LLK_ERR_HIP, hipGetErrorString(e));
  }
  llk_kernel_context ctx{nullptr, 0, s};  // null stream, library workspace
  auto bail = [&](int code) {
    (void)hipStreamSynchronize(s);  // nothing queued outlives the call
    return status(code);
  };
  bool direct = false;  // launched on the caller's row-major weights
  // Weights.  Read on every call (the default): device-resident weights
  // go straight to the kernels where their row-major forms take the shape
  // (rowmajor_with_module: the decode tile kernel up to 128 rows; above, the
  // tile kernel), else they are packed into the MFMA
  // operand layout first.
  const int nw = swiglu ? 2 : 1;
  llk_memref2d* wm[2] = {wg, wu};
  const llk_packed_weights* pw[2] = {nullptr, nullptr};
  std::shared_ptr<llk_packed_weights> held[2];  // references kept to the end of the call
  if (g_immutable.load(std::memory_order_relaxed)) {
    llk_jit_cache* cache = nullptr;
    if ((rc = device_cache(d, &cache))) return bail(rc);
    for (int i = 0; i < nw; ++i) {
      const llk_tensor2d t = weight_tensor(*wm[i]);
      rc = cache_get_shared(cache, &t, kBK, is_host_only(t.data) ? 0 : 1, 0, &held[i]);
      if (rc) return bail(rc);
      pw[i] = held[i].get();
    }
  } else if (!is_host_only(memref_data(*wg, 2)) &&
             (!swiglu || !is_host_only(memref_data(*wu, 2)))) {
    const llk_tensor2d wgt = weight_tensor(*wg);
    const llk_tensor2d wut = swiglu ? weight_tensor(*wu) : wgt;
    bool taken = false;
    rc = rowmajor_with_module(swiglu ? 1 : 0, &xt, &wgt, swiglu ? &wut : nullptr, &yt, out_dtype,
                              &ctx, mod, !swiglu, &taken);
    if (rc) return bail(rc);
    direct = taken;
  }
  if (!direct && pw[0] == nullptr) {
    size_t off[2] = {0, 0}, total = 0;
    for (int i = 0; i < nw; ++i) {
      off[i] = total;
      total += (llk_pack_device_bytes(wm[i]->size0, wm[i]->size1) + 255) / 256 * 256;
    }
    if ((rc = ensure(&d.wstage, &d.wstage_bytes, total, "KernelFn: packed-weight buffer")))
      return bail(rc);
    for (int i = 0; i < nw; ++i) {
      const llk_tensor2d t = weight_tensor(*wm[i]);
      rc = pack_into(&t, kBK, !is_host_only(t.data), static_cast<uint8_t*>(d.wstage) + off[i], s,
                     mod, &d.view[i]);
      if (rc) return bail(rc);
      pw[i] = d.view[i];
    }
  }

  if (!direct) {
    rc = swiglu ? swiglu_with_module(&xt, pw[0], pw[1], &yt, out_dtype, &ctx, mod)
                : gemm_with_module(&xt, pw[0], &yt, out_dtype, &ctx, mod, true);
    if (rc) return bail(rc);
  }
  if (y_host)
    e = hipMemcpy2DAsync(y_user, (size_t)result->stride0 * ye, yt.data, (size_t)N * ye,
                         (size_t)N * ye, (size_t)M, hipMemcpyDeviceToHost, s);
  const hipError_t es = hipStreamSynchronize(s);
  if (e == hipSuccess) e = es;
  if (e != hipSuccess) return fail(LLK_ERR_HIP, hipGetErrorString(e));
  return LLK_OK;
}

}  // namespace llk

extern "C" {

void llk_swiglu_kernel_fn(llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu,
                          llk_memref2d* init, llk_memref2d* result) {
  (void)llk::memref_call(kOpSwiglu, LLK_BF16, nullptr, x, wg, wu, init, result);
}

int llk_kernel_fn_status(void) { return g_status; }

int llk_kernel_fn_assume_immutable_weights(int on) {
  return g_immutable.exchange(on ? 1 : 0);
}

llk_jit_cache* llk_kernel_fn_cache(void) {
  int dev;
  if (current_device(&dev)) return nullptr;
  FnDevice& d = g_fn[dev];
  std::lock_guard<std::mutex> lk(d.mu);
  llk_jit_cache* c = nullptr;
  return device_cache(d, &c) == LLK_OK ? c : nullptr;
}

}  // extern "C"
