// kernel_fn.cpp -- the reference's KernelFn calling convention for the fused
// SwiGLU (include/LLK/Runtime/JitCache.h:79-81): five MemRef2D* (x, wg, wu,
// init, result), no stream, no context, no return value.  The raw row-major
// weights are resolved to packed device handles through the L4 weight level
// of a per-device cache (WeightKey = address, shape, BK: JitCache.h:143-146,
// KernelKey.h:114-124), packing on a miss; the call then runs the same
// kernels as llk_swiglu_bf16 on the null stream and returns when the result
// is written, as the reference's JIT'd CPU function does.  Operands may be
// in device memory or in host memory (the reference's callers pass host
// buffers); host operands are staged through device buffers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>

#include "llk/llk_abi.h"

namespace llk {
int setError(int code, const char* msg);  // llk_abi.cpp
}

namespace {

constexpr int kMaxDevices = 64;
constexpr int64_t kBK = 64;  // PackWeights' kDefaultBK (PackWeights.cpp:36)

thread_local int g_status = LLK_OK;

struct FnDevice {
  std::mutex mu;                  // guards the cache creation and the staging buffers
  llk_jit_cache* cache = nullptr;  // L4 weights of KernelFn calls on this device
  void* stage = nullptr;          // device staging for host X and result
  size_t stage_bytes = 0;
};
FnDevice g_fn[kMaxDevices];

int fail(int code, const char* msg) {
  g_status = code;
  return llk::setError(code, msg);
}

// Data address of a bf16 memref: aligned + offset elements.
void* memref_data(const llk_memref2d& m) {
  return static_cast<char*>(m.aligned) + m.offset * 2;
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

int device_cache(int dev, llk_jit_cache** out) {
  FnDevice& d = g_fn[dev];
  std::lock_guard<std::mutex> lk(d.mu);
  if (!d.cache) {
    const int rc = llk_cache_create(&d.cache);
    if (rc) {
      g_status = rc;
      return rc;
    }
  }
  *out = d.cache;
  return LLK_OK;
}

int swiglu_memref(llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu, llk_memref2d* init,
                  llk_memref2d* result) {
  if (!x || !wg || !wu || !init || !result)
    return fail(LLK_ERR_INVALID_ARGUMENT, "KernelFn: NULL memref");
  const int64_t M = x->size0, K = x->size1, N = wg->size1;
  int rc = llk_verify_fused_swiglu(M, K, wg->size0, wg->size1, wu->size0, wu->size1, init->size0,
                                   init->size1);
  if (rc) {
    g_status = rc;
    return rc;
  }
  if (result->size0 != init->size0 || result->size1 != init->size1)
    return fail(LLK_ERR_SHAPE, "KernelFn: result shape differs from init");
  if (M == 0 || N == 0) return LLK_OK;
  int dev;
  if ((rc = current_device(&dev))) return rc;
  llk_jit_cache* cache = nullptr;
  if ((rc = device_cache(dev, &cache))) return rc;

  // Weights: L4 lookup by (address, shape, BK), packed on a miss from host
  // or device memory.
  llk_packed_weights* pw[2] = {nullptr, nullptr};
  llk_memref2d* wm[2] = {wg, wu};
  for (int i = 0; i < 2; ++i) {
    llk_tensor2d t{memref_data(*wm[i]), wm[i]->size0, wm[i]->size1, wm[i]->stride0,
                   wm[i]->stride1};
    rc = llk_cache_get_packed_weights(cache, &t, kBK, is_host_only(t.data) ? 0 : 1, 0, &pw[i]);
    if (rc) {
      g_status = rc;
      return rc;
    }
  }

  llk_tensor2d xt{memref_data(*x), M, K, x->stride0, x->stride1};
  llk_tensor2d yt{memref_data(*result), M, N, result->stride0, result->stride1};
  const bool x_host = K > 0 && is_host_only(xt.data);
  const bool y_host = is_host_only(yt.data);
  llk_kernel_context ctx{nullptr, 0, nullptr};  // null stream, library workspace
  if (!x_host && !y_host) {
    rc = llk_swiglu_bf16(&xt, pw[0], pw[1], &yt, LLK_BF16, &ctx);
    if (rc) {
      g_status = rc;
      return rc;
    }
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return fail(LLK_ERR_HIP, hipGetErrorString(e));
    return LLK_OK;
  }

  // Host operands: dense device copies (X [M, K], Y [M, N]), one call at a
  // time per device (they share the device's staging buffer).
  if (x->stride1 != 1 || result->stride1 != 1)
    return fail(LLK_ERR_LAYOUT, "KernelFn: host operands need unit inner stride");
  FnDevice& d = g_fn[dev];
  std::lock_guard<std::mutex> lk(d.mu);
  const size_t xbytes = x_host ? ((size_t)M * K * 2 + 255) / 256 * 256 : 0;
  const size_t ybytes = y_host ? (size_t)M * N * 2 : 0;
  if (d.stage_bytes < xbytes + ybytes) {
    if (d.stage) (void)hipFree(d.stage);  // no launch uses it between calls
    d.stage = nullptr;
    d.stage_bytes = 0;
    const size_t bytes = std::max(xbytes + ybytes, (size_t)1 << 20);
    hipError_t e = hipMalloc(&d.stage, bytes);
    if (e != hipSuccess) {
      d.stage = nullptr;
      return fail(LLK_ERR_OUT_OF_MEMORY, "KernelFn: staging buffer");
    }
    d.stage_bytes = bytes;
  }
  uint8_t* base = static_cast<uint8_t*>(d.stage);
  hipError_t e = hipSuccess;
  if (x_host) {
    e = hipMemcpy2D(base, (size_t)K * 2, xt.data, (size_t)x->stride0 * 2, (size_t)K * 2,
                    (size_t)M, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(LLK_ERR_HIP, hipGetErrorString(e));
    xt = llk_tensor2d{base, M, K, K, 1};
  }
  void* y_user = yt.data;
  const int64_t y_ld = result->stride0;
  if (y_host) yt = llk_tensor2d{base + xbytes, M, N, N, 1};
  rc = llk_swiglu_bf16(&xt, pw[0], pw[1], &yt, LLK_BF16, &ctx);
  if (rc) {
    g_status = rc;
    return rc;
  }
  if (y_host)
    e = hipMemcpy2D(y_user, (size_t)y_ld * 2, yt.data, (size_t)N * 2, (size_t)N * 2, (size_t)M,
                    hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e != hipSuccess) return fail(LLK_ERR_HIP, hipGetErrorString(e));
  return LLK_OK;
}

}  // namespace

extern "C" {

void llk_swiglu_kernel_fn(llk_memref2d* x, llk_memref2d* wg, llk_memref2d* wu,
                          llk_memref2d* init, llk_memref2d* result) {
  g_status = LLK_OK;
  (void)swiglu_memref(x, wg, wu, init, result);
}

int llk_kernel_fn_status(void) { return g_status; }

llk_jit_cache* llk_kernel_fn_cache(void) {
  int dev;
  if (current_device(&dev)) return nullptr;
  llk_jit_cache* c = nullptr;
  return device_cache(dev, &c) == LLK_OK ? c : nullptr;
}

}  // extern "C"
