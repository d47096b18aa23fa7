// llk_abi.cpp -- C ABI of the gfx950 backend (include/llk/llk_abi.h):
// argument validation, packed-weight handles, workspace management and
// kernel dispatch.  Kernels live in kernels/*.hip.
#include "llk/llk_abi.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <tuple>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "kernels/launch.h"
#include "packed_weights.h"
#include "runtime/kernel_key.h"
#include "runtime/packed_layout.h"
#include "runtime/schedule.h"
#include "runtime/tunables.h"

namespace llk {
struct ModuleFns;  // functions of a loaded code object (code_object.cpp)
}

// Kernel launchers (kernels/*.hip).  mod: the loaded per-operation code
// object whose kernels to launch, or null for the library's own.
hipError_t llk_launch_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                           const void* w1, void* y, int64_t ldy, int M, int N, int KB, int NB,
                           int S, void* part, int out_dtype, bool yvec, bool accumulate,
                           const llk::ModuleFns* mod, hipStream_t s);
size_t llk_tile_split_bytes(int mode, int M, int NB, int S, bool accumulate);
bool llk_tile_x_fits(int M, int64_t ldx);
hipError_t llk_launch_swiglu_wide(int B, const uint16_t* x, int64_t ldx, const void* wg,
                                  const void* wu, void* y, int64_t ldy, int M, int N, int KB,
                                  int NB, int S, void* part, const llk::ModuleFns* mod,
                                  hipStream_t s);
bool llk_swiglu_wide_fits(int B, int KB);
size_t llk_swiglu_wide_split_bytes(int B, int M, int N, int S);
hipError_t llk_launch_skinny(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                             const void* w1, void* y, int64_t ldy, int M, int N, int K, int KB,
                             int NB, int S, int G, void* ws, int out_dtype, bool xvec,
                             bool yvec, bool accumulate, const llk::ModuleFns* mod,
                             hipStream_t s);
size_t llk_skinny_workspace_bytes(int nmat, int M, int N_pad, int S);
int llk_skinny_threads(int nmat, int M, int G);
bool llk_decode_tile_fits(int M, int64_t K, int64_t ldx);
hipError_t llk_launch_decode_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                                  const void* w1, void* y, int64_t ldy, int M, int N, int KB,
                                  int NB, int S, void* ws, int out, bool yvec, bool accumulate,
                                  const llk::ModuleFns* mod, hipStream_t s);
bool llk_decode_rowmajor_fits(int M, int64_t K, int64_t ldx, const void* w, int64_t ldw,
                              int64_t N);
hipError_t llk_launch_decode_rowmajor(int mode, const uint16_t* x, int64_t ldx,
                                      const uint16_t* w0, int64_t ldw0, const uint16_t* w1,
                                      int64_t ldw1, void* y, int64_t ldy, int M, int N, int K,
                                      int S, void* ws, int out, bool yvec, bool accumulate,
                                      const llk::ModuleFns* mod, hipStream_t s);
bool llk_tile_rowmajor_fits(int M, int64_t K, int64_t ldx, const void* w, int64_t ldw, int64_t N);
hipError_t llk_launch_tile_rowmajor(int mode, const uint16_t* x, int64_t ldx, const uint16_t* w0,
                                    int64_t ldw0, const uint16_t* w1, int64_t ldw1, void* y,
                                    int64_t ldy, int M, int N, int K, int S, void* part, int out,
                                    bool yvec, bool accumulate, const llk::ModuleFns* mod,
                                    hipStream_t s);
hipError_t llk_launch_pad_rows(const uint16_t* x, int64_t ldx, int M, int K, uint16_t* out,
                               int64_t ldo, const llk::ModuleFns* mod, hipStream_t s);
hipError_t llk_launch_pack(const uint16_t* w, int64_t ld, int K, int N, int KB, int NB, void* out,
                           const llk::ModuleFns* mod, hipStream_t s);
hipError_t llk_launch_zero_rows(void* y, int64_t ld_elems, int64_t M, int64_t N, int elem_bytes,
                                const llk::ModuleFns* mod, hipStream_t s);

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int fail_hip(hipError_t e, const char* what) {
  return fail(LLK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;

// A library-owned workspace: device memory, zero-filled when allocated.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  hipEvent_t done = nullptr;  // completes after the last call that used it (see bind)
  bool pinned = false;        // used under graph capture: a graph may name it, never freed
  int busy = 0;               // calls between get_workspace and release_workspace
  uint64_t tick = 0;          // last use, for LRU eviction
};

struct DeviceState {
  std::mutex mu;
  int checked = 0;  // 0 unknown, 1 gfx950, -1 other
  char arch[64] = {0};
  int cu_count = 0, lds = 0, clock_khz = 0;
  // Library-owned workspaces, one per stream (the per-thread default stream:
  // one per thread), so launches on different streams never share one; at
  // most max_workspaces of them, least recently used evicted first.
  std::map<std::pair<uintptr_t, uint64_t>, Workspace> ws;
  uint64_t tick = 0;
  std::vector<void*> retired;  // outgrown pinned workspaces, kept until process exit
  void* noalloc_scratch = nullptr;  // device address of `scratch` (below)
};
DeviceState g_dev[kMaxDevices];

// Current device, verified to be gfx950.
int current_device(int* dev) {
  int d = 0;
  hipError_t e = hipGetDevice(&d);
  if (e != hipSuccess) return fail(LLK_ERR_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (d < 0 || d >= kMaxDevices) return fail(LLK_ERR_NO_DEVICE, "device index %d out of range", d);
  DeviceState& st = g_dev[d];
  std::lock_guard<std::mutex> lk(st.mu);
  if (st.checked == 0) {
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, d);
    if (e != hipSuccess) return fail_hip(e, "hipGetDeviceProperties");
    std::snprintf(st.arch, sizeof(st.arch), "%s", p.gcnArchName);
    st.cu_count = p.multiProcessorCount;
    st.lds = static_cast<int>(p.sharedMemPerBlock);
    st.clock_khz = p.clockRate;
    st.checked = std::strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
  }
  *dev = d;
  if (st.checked != 1)
    return fail(LLK_ERR_UNSUPPORTED_ARCH, "device %d is %s, this library is built for gfx950", d,
                st.arch);
  return LLK_OK;
}

int check_tensor(const llk_tensor2d* t, const char* name) {
  if (!t) return fail(LLK_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (t->dim0 < 0 || t->dim1 < 0)
    return fail(LLK_ERR_SHAPE, "%s has negative dimension (%lld, %lld)", name,
                (long long)t->dim0, (long long)t->dim1);
  if (t->dim0 > 0 && t->dim1 > 0 && !t->data)
    return fail(LLK_ERR_INVALID_ARGUMENT, "%s.data is NULL", name);
  if (t->dim0 > 0 && t->dim1 > 0) {
    if (t->stride1 != 1)
      return fail(LLK_ERR_LAYOUT, "%s.stride1 is %lld; only unit inner stride is supported", name,
                  (long long)t->stride1);
    if (t->dim0 > 1 && t->stride0 < t->dim1)
      return fail(LLK_ERR_LAYOUT, "%s.stride0 (%lld) < dim1 (%lld)", name, (long long)t->stride0,
                  (long long)t->dim1);
  }
  return LLK_OK;
}

int check_packed(const llk_packed_weights* w, const char* name, int dev) {
  if (!w) return fail(LLK_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (!w->dev) return fail(LLK_ERR_INVALID_ARGUMENT, "%s has no device payload", name);
  if (w->device != dev)
    return fail(LLK_ERR_DEVICE_MISMATCH, "%s was packed for device %d, current device is %d",
                name, w->device, dev);
  return LLK_OK;
}

constexpr int64_t kMaxDim = (int64_t)1 << 30;

bool x_vec_ok(const llk_tensor2d* x) {
  return (reinterpret_cast<uintptr_t>(x->data) % 16 == 0) && (x->stride0 % 8 == 0) &&
         (x->dim1 % 8 == 0);
}
size_t dtype_size(int dtype) { return dtype == LLK_FP32 ? 4 : 2; }
// Rows allow a 4-element vector store.
bool y_vec_ok(const llk_tensor2d* y, int dtype) {
  const uintptr_t align = 4 * dtype_size(dtype);
  return (reinterpret_cast<uintptr_t>(y->data) % align == 0) && (y->stride0 % 4 == 0);
}

// Key of the library workspace of a stream: the stream handle, and for the
// per-thread default stream (a different stream on every thread) the thread.
std::pair<uintptr_t, uint64_t> workspace_key(hipStream_t s) {
  static std::atomic<uint64_t> next_thread{1};
  thread_local const uint64_t thread_id = next_thread.fetch_add(1);
  return {reinterpret_cast<uintptr_t>(s), s == hipStreamPerThread ? thread_id : 0};
}

// Frees a library workspace's buffer once the last call that used it has
// finished on the GPU (its `done` event; a workspace never used yet has
// none).  Called with the device mutex held, for idle, unpinned entries.
void free_workspace_buffer(Workspace* w) {
  if (w->done) (void)hipEventSynchronize(w->done);
  if (w->ptr) (void)hipFree(w->ptr);
  w->ptr = nullptr;
  w->bytes = 0;
}

// Evicts the least recently used idle, unpinned workspace of `st` other
// than `keep`; false if there is none.
bool evict_one_workspace(DeviceState& st, const Workspace* keep) {
  auto victim = st.ws.end();
  for (auto it = st.ws.begin(); it != st.ws.end(); ++it) {
    const Workspace& w = it->second;
    if (&w == keep || w.busy > 0 || w.pinned) continue;
    if (victim == st.ws.end() || w.tick < victim->second.tick) victim = it;
  }
  if (victim == st.ws.end()) return false;
  free_workspace_buffer(&victim->second);
  if (victim->second.done) (void)hipEventDestroy(victim->second.done);
  st.ws.erase(victim);
  return true;
}

// Workspace: the caller's (ctx->scratch) if given, else the library's own
// buffer for the launch stream, grown on demand.  Launches are ordered on
// their stream, so work on one stream never overlaps in its workspace, and
// two streams never share one.  (A HIP graph captured on a stream keeps
// that stream's workspace: replaying it concurrently with direct launches
// on the capture stream is the caller's race, as with any captured buffer.)
// The library keeps at most `max_workspaces` of them per device (tunable,
// default 16): a new stream (or thread, on the per-thread default stream)
// beyond that evicts the least recently used idle one.  A buffer is freed
// (on eviction, on growth, or by llk_workspace_trim) only after its event,
// which completes with the last kernel of the last call that used it, has
// completed (BindDone: the event rides on the launches themselves), so work still
// queued on a stream -- even one destroyed since -- never loses its
// buffer; a workspace that a call used while its stream was capturing a
// graph is pinned instead (the graph names it) and is never freed.  Growth
// is geometric (x1.5 at least).  *held is the library workspace handed out
// (null for a caller's scratch or when nothing is needed): the caller gives
// it back with release_workspace after enqueuing its launches.
int get_workspace(int dev, size_t need, llk_kernel_context* ctx, void** out, Workspace** held) {
  *out = nullptr;
  *held = nullptr;
  if (need == 0) return LLK_OK;
  if (ctx && ctx->scratch) {
    if (ctx->scratch_size < need)
      return fail(LLK_ERR_SCRATCH, "scratch_size %zu < required %zu bytes", ctx->scratch_size,
                  need);
    if (reinterpret_cast<uintptr_t>(ctx->scratch) % 256 != 0)
      return fail(LLK_ERR_SCRATCH, "scratch must be 256-byte aligned");
    *out = ctx->scratch;
    return LLK_OK;
  }
  DeviceState& st = g_dev[dev];
  const auto key = workspace_key(ctx ? static_cast<hipStream_t>(ctx->stream) : nullptr);
  std::lock_guard<std::mutex> lk(st.mu);
  Workspace* w = nullptr;
  const bool fresh_key = st.ws.find(key) == st.ws.end();
  if (fresh_key) {
    const size_t cap = (size_t)std::max<int64_t>(1, llk::tunable("max_workspaces"));
    while (st.ws.size() >= cap && evict_one_workspace(st, nullptr)) {
    }
  }
  try {
    w = &st.ws[key];
  } catch (const std::bad_alloc&) {
    return fail(LLK_ERR_OUT_OF_MEMORY, "workspace bookkeeping");
  }
  if (!w->done) {
    const hipError_t e = hipEventCreateWithFlags(&w->done, hipEventDisableTiming);
    if (e != hipSuccess) {
      w->done = nullptr;
      if (fresh_key) st.ws.erase(key);
      return fail_hip(e, "hipEventCreate(workspace)");
    }
  }
  if (w->bytes < need) {
    const size_t bytes = std::max({need, w->bytes + w->bytes / 2, (size_t)1 << 20});
    if (w->ptr && !w->pinned && w->busy == 0) {
      free_workspace_buffer(w);  // this stream's earlier calls have finished with it
    } else if (w->ptr) {
      try {
        st.retired.push_back(w->ptr);  // a graph or a concurrent call may still name it
      } catch (const std::bad_alloc&) {
        return fail(LLK_ERR_OUT_OF_MEMORY, "workspace bookkeeping");
      }
      w->ptr = nullptr;
      w->bytes = 0;
    }
    void* fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, bytes);
    if (e != hipSuccess && evict_one_workspace(st, w)) e = hipMalloc(&fresh, bytes);
    if (e != hipSuccess)
      return fail(LLK_ERR_OUT_OF_MEMORY, "hipMalloc(%zu) for workspace: %s", bytes,
                  hipGetErrorString(e));
    e = hipMemset(fresh, 0, bytes);
    if (e != hipSuccess) {
      (void)hipFree(fresh);
      return fail_hip(e, "hipMemset(workspace)");
    }
    w->ptr = fresh;
    w->bytes = bytes;
    w->pinned = false;
  }
  ++w->busy;
  w->tick = ++st.tick;
  *out = w->ptr;
  *held = w;
  return LLK_OK;
}

// Binds a held workspace's `done` event to the calling thread's launches
// from construction to end(): launch_kernel names it as each kernel's stop
// event, so it completes with the call's last kernel.  Not when `s` is
// capturing a graph (an event under capture would be a graph node, not a
// point the host can wait for): release_workspace then pins the workspace.
class BindDone {
 public:
  BindDone(Workspace* w, hipStream_t s) : prev_(llk_gfx950::t_launch_done) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (w && hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
      llk_gfx950::t_launch_done = w->done;
      bound_ = true;
    }
  }
  ~BindDone() { end(); }
  void end() { llk_gfx950::t_launch_done = prev_; }
  bool bound() const { return bound_; }
  BindDone(const BindDone&) = delete;
  BindDone& operator=(const BindDone&) = delete;

 private:
  hipEvent_t prev_;
  bool bound_ = false;
};

// Gives back a workspace from get_workspace once the call's launches are
// enqueued on `s`.  `bound`: its `done` event rode on those launches
// (BindDone); otherwise it is recorded on `s` now, or the workspace is
// pinned when `s` is capturing a graph.
void release_workspace(int dev, Workspace* w, hipStream_t s, bool bound = false) {
  if (!w) return;
  DeviceState& st = g_dev[dev];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  // Pinned too when the capture state or the record cannot be had: no event
  // then marks this call's end, so the buffer must outlive it.
  bool pin = !bound &&
             (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone);
  if (!bound && !pin && hipEventRecord(w->done, s) != hipSuccess) pin = true;
  if (pin) (void)hipGetLastError();  // a failed query leaves no error for the next call
  std::lock_guard<std::mutex> lk(st.mu);
  if (pin) w->pinned = true;
  --w->busy;
}

// Workspace of llk_swiglu_bf16_noalloc: a fixed device array, one copy per
// GPU (allocated when the library's code object is loaded on the device, so
// the entry point itself allocates nothing).  Its contents persist between
// calls; no kernel relies on them (every byte a launch reads from it -- k-split
// partial planes, the padded X -- was written earlier in the same call), so
// nothing is cleared.  Calls that overlap on one GPU race on it.  In host code
// `scratch` names a host-side stand-in: its device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on device `dev` (the current device), looked
// up on the first no-allocation call on that device.
int noalloc_scratch(int dev, void** out) {
  DeviceState& st = g_dev[dev];
  std::lock_guard<std::mutex> lk(st.mu);
  if (!st.noalloc_scratch) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress(scratch)");
    if (!p || reinterpret_cast<uintptr_t>(p) % 256 != 0)
      return fail(LLK_ERR_HIP, "hipGetSymbolAddress(scratch) returned an unaligned address");
    st.noalloc_scratch = p;
  }
  *out = st.noalloc_scratch;
  return LLK_OK;
}

hipStream_t stream_of(const llk_kernel_context* ctx) {
  return ctx ? static_cast<hipStream_t>(ctx->stream) : nullptr;
}

// Launch plan of one contraction (SwiGLU: nmat 2, GEMM: nmat 1).
struct Plan {
  bool skinny = false;   // small-M bandwidth kernel
  bool dtile = false;    // ... on the decode tile kernel (with skinny)
  int S = 1;             // k splits across workgroups (either kernel)
  int G = 1;             // small-M kernel: 32-column groups per workgroup
  bool pad = false;      // tile path: copy X into a padded buffer first
  int64_t chunk = 0;     // tile path: rows per launch (32-bit X offsets)
  int64_t ld = 0;        // tile path: row stride of the X the kernel reads
  size_t pad_bytes = 0;  // tile path: padded X at the start of the workspace
  size_t ws_bytes = 0;   // workspace the plan needs
  bool too_large = false;  // tile path: K beyond the kernel's 32-bit offsets
  int64_t head_nb = 0;   // tile path: leading n-blocks launched unsplit (S applies to the rest)
  int wide = 0;          // tile path, fused SwiGLU with bf16 output: the wide kernel's B
                         // (16 B columns per tile and matrix; 0 = the 128-column kernel)
};

// k splits of the tile kernel for `rows` rows: the S that minimises the
// modelled time  waves(S) * (ceil(KB / S) + 2) + partial traffic  in units
// of one 64-k step of a full wave of workgroups (about 1.6 us on MI355X:
// a 256 x 256 tile over K = 4096 takes ~102 us).  waves(S) = ceil(tiles * S /
// tile_wgs_per_wave); the "+ 2" is the per-workgroup pipeline fill and
// epilogue; the S partial planes (S * nmat * rows * N_pad fp32) are written
// and read back at ~4 TB/s, plus one step for the reduce launch.
struct SplitCost {
  int S;
  double cost;
};

SplitCost best_split(int nmat, int64_t rows, int64_t KB, int64_t NB, int64_t forced) {
  const int64_t min_kb = std::max<int64_t>(1, llk::tunable("tile_min_kb"));
  int64_t smax = std::min<int64_t>(64, std::max<int64_t>(1, KB / min_kb));
  if (forced > 0) smax = std::min(forced, KB);
  const int64_t tiles = (rows + 255) / 256 * (nmat == 2 ? NB : (NB + 1) / 2);
  const int64_t per_wave = std::max<int64_t>(1, llk::tunable("tile_wgs_per_wave"));
  SplitCost best{1, 0.0};
  for (int64_t S = forced > 0 ? smax : 1; S <= smax; ++S) {
    const int64_t kbs = (KB + S - 1) / S;
    const int64_t s_eff = (KB + kbs - 1) / kbs;  // no empty splits
    const double waves = (double)((tiles * s_eff + per_wave - 1) / per_wave);
    double cost = waves * (double)(kbs + 2);
    if (s_eff > 1) cost += 2.0 * s_eff * nmat * rows * NB * 128 * 4 / (4e12 * 1.6e-6) + 1.0;
    if (S == 1 || forced > 0 || cost < best.cost) best = SplitCost{(int)s_eff, cost};
  }
  return best;
}

// The tile kernel's launch over `rows` rows: k splits S for the columns from
// n-block head_nb on, and head_nb leading n-blocks run unsplit first (0: one
// launch over all columns).  Tail split: when the tiles fill q >= 1 whole
// waves and leave a partial one (config 5 at M = 4097: 340 GEMM tiles on 256
// CUs), the whole n-tile columns that fit q waves run unsplit and only the
// remaining columns take a k split -- one short balanced wave instead of a
// nearly empty long one, with partial planes for the tail columns only.
// Used when the model puts it 3% or more below the best single launch.
struct TilePlan {
  int S;
  int64_t head_nb;
  double cost;  // modelled time, in the units of best_split
};

TilePlan tile_plan(int nmat, int64_t rows, int64_t KB, int64_t NB, int64_t db_splits) {
  int64_t forced = llk::tunable("tile_splits");
  if (forced <= 0) forced = db_splits;
  const SplitCost all = best_split(nmat, rows, KB, NB, forced);
  if (forced > 0) return {all.S, 0, all.cost};
  const int64_t nb_per_tile = nmat == 2 ? 1 : 2;
  const int64_t tm = (rows + 255) / 256, tn = (NB + nb_per_tile - 1) / nb_per_tile;
  const int64_t per_wave = std::max<int64_t>(1, llk::tunable("tile_wgs_per_wave"));
  const int64_t head_tn = tm * tn / per_wave * per_wave / tm;  // columns of q whole waves
  TilePlan best{all.S, 0, all.cost};
  double best_cost = all.cost;
  if (llk::tunable("tile_tail_split") != 0 && head_tn > 0 && head_tn < tn) {
    const int64_t head_nb = head_tn * nb_per_tile;
    const double head = (double)((tm * head_tn + per_wave - 1) / per_wave) * (double)(KB + 2);
    const SplitCost tail = best_split(nmat, rows, KB, NB - head_nb, 0);
    if (head + tail.cost <= 0.97 * best_cost) {
      best = {tail.S, head_nb, head + tail.cost};
      best_cost = head + tail.cost;
    }
  }
  return best;
}

// Wide SwiGLU tiles (kernels/swiglu_wide.hip): B blocks of 16 columns per
// matrix instead of 8, with S k splits.  Modelled like best_split: waves of
// workgroups x (64-k steps per split + 2), each workgroup B/8 times the work
// of a 128-column tile, plus for S > 1 the register-order partials written
// and read back at ~4 TB/s and one reduce launch.  Taken when 3% or more
// below the 128-column plan's cost (config 3: 504 tiles in 2 waves x 1.375
// against 688 in 3 waves; config 5 at M = 1000: 496 tiles of B = 7 in 2 waves
// x 0.875 against 432 in 2 waves; at M = 255: 124 tiles of B = 7 x 2 splits,
// 248 workgroups, against 108 x 2 = 216).  tile_wide = 7 or 11 forces that
// width (with the forced tile_splits, if any, else the modelled S); 0 turns
// the kernel off.
struct WideChoice {
  int B = 0, S = 1;
};

WideChoice wide_choice(int64_t rows, int64_t N, int64_t KB, double std_cost, int64_t forced_s) {
  const int64_t knob = llk::tunable("tile_wide");
  if (knob == 0) return {};
  const int64_t per_wave = std::max<int64_t>(1, llk::tunable("tile_wgs_per_wave"));
  const int64_t min_kb = std::max<int64_t>(1, llk::tunable("tile_min_kb"));
  const int64_t tm = (rows + 255) / 256;
  WideChoice best;
  double best_cost = 0.97 * std_cost;
  for (int B : {11, 7}) {
    if (!llk_swiglu_wide_fits(B, (int)KB)) continue;
    if (knob != 1 && knob != B) continue;
    const int64_t tiles = tm * ((N + 16 * B - 1) / (16 * B));
    WideChoice own;
    double own_cost = 0.0;
    int64_t s_lo = 1, s_hi = std::min<int64_t>(64, std::max<int64_t>(1, KB / min_kb));
    if (forced_s > 0) s_lo = s_hi = std::min(forced_s, KB);
    for (int64_t S = s_lo; S <= s_hi; ++S) {
      const int64_t kbs = (KB + S - 1) / S;
      const int64_t s_eff = (KB + kbs - 1) / kbs;  // no empty splits
      double cost = (double)((tiles * s_eff + per_wave - 1) / per_wave) * (double)(kbs + 2) * B / 8.0;
      if (s_eff > 1)
        cost += 2.0 * (double)llk_swiglu_wide_split_bytes(B, (int)rows, (int)N, (int)s_eff) /
                    (4e12 * 1.6e-6) + 1.0;
      if (S == s_lo || cost < own_cost) {
        own = {B, (int)s_eff};
        own_cost = cost;
      }
    }
    if (knob == B) return own;
    if (own_cost < best_cost) {
      best = own;
      best_cost = own_cost;
    }
  }
  return best;
}

// Active schedule DB (llk_set_schedule_db, or the file named by the
// LLK_SCHEDULE_DB environment variable at first use): the entry the
// reference's loader + selectBest pick for (operation, M bucket), cached.
struct ActiveDb {
  std::mutex mu;
  bool env_checked = false;
  std::string path;  // empty: no DB
  std::map<std::pair<int, int>, std::pair<bool, llk::ScheduleEntry>> sel;
};
ActiveDb g_db;

bool db_entry(int nmat, int64_t M, llk::ScheduleEntry* out) {
  std::lock_guard<std::mutex> lk(g_db.mu);
  if (!g_db.env_checked) {
    g_db.env_checked = true;
    const char* env = std::getenv("LLK_SCHEDULE_DB");
    if (env && *env && g_db.path.empty()) g_db.path = env;
  }
  if (g_db.path.empty()) return false;
  const int bucket = llk::classifyM(M);
  const auto key = std::make_pair(nmat, bucket);
  auto it = g_db.sel.find(key);
  if (it == g_db.sel.end()) {
    bool ok = false;
    const auto m = llk::loadScheduleDB(g_db.path, bucket, nmat == 2 ? "fused_swiglu" : "matmul", &ok);
    it = g_db.sel.emplace(key, std::make_pair(ok && !m.empty(),
                                              m.empty() ? llk::ScheduleEntry{} : m.front())).first;
  }
  if (!it->second.first) return false;
  *out = it->second.second;
  return true;
}

// Small-M launch choice: workgroup width W (32-column groups) and k splits
// S minimising the modelled time
//   rounds x max(weight bytes / 26.5 GB/s, (weight + X bytes) / 31 GB/s)
//   + (S > 1: reduce launch ~4 us + partial planes written and read at 4 TB/s)
// per workgroup, rounds = ceil(workgroups / decode_target_wgs): on MI355X
// each CU streams its loads at ~26-31 GB/s whatever the grid, so a round's
// time is one workgroup's bytes.  X is read once per wave group (SkinnyCfg
// in kernels/swiglu_decode.hip: GW = 2 groups per wave except SwiGLU with
// M <= 32 or W = 1).  A forced width or split count (> 0) is kept; an
// automatic width is 2 unless 1 is modelled 3% faster (width 2 measured
// ahead on ties: decode M = 8 39.9 vs 41.1 us).
struct SmallMChoice {
  int width = 2, splits = 1;
};

SmallMChoice small_m_choice(int nmat, int64_t M, int64_t KB, int64_t NB, int64_t force_w,
                            int64_t force_s) {
  const int64_t target = std::max<int64_t>(1, llk::tunable("decode_target_wgs"));
  const int64_t min_kb = std::max<int64_t>(1, llk::tunable("decode_min_kb"));
  const int64_t rows = (M + 31) / 32 * 32;
  auto cost = [&](int64_t W, int64_t S, int64_t* s_out) {
    const int64_t kbs = (KB + S - 1) / S;
    const int64_t s_eff = (KB + kbs - 1) / kbs;  // no empty splits
    const int64_t per_wave = (W == 1 || (nmat == 2 && M <= 32)) ? 1 : 2;
    const int64_t wave_groups = W / per_wave;
    const int64_t wgs = NB * 4 / W * s_eff;
    const double k_bytes = (double)kbs * 64 * 2;
    const double wbytes = (double)W * 32 * nmat * k_bytes;
    const double xbytes = (double)wave_groups * M * k_bytes;
    double t = (double)((wgs + target - 1) / target) *
               std::max(wbytes / 26.5e9, (wbytes + xbytes) / 31e9);
    if (s_eff > 1) t += 4e-6 + 2.0 * s_eff * nmat * rows * NB * 128 * 4 / 4e12;
    *s_out = s_eff;
    return t;
  };
  SmallMChoice best;
  double best_t = 0.0;
  const int64_t widths[2] = {2, 1};
  const bool auto_w = !(force_w == 1 || force_w == 2 || force_w == 4);
  for (int wi = 0; wi < (auto_w ? 2 : 1); ++wi) {
    const int64_t W = auto_w ? widths[wi] : force_w;
    int64_t s_lo = 1, s_hi = std::min<int64_t>(64, std::max<int64_t>(1, KB / min_kb));
    if (force_s > 0) s_lo = s_hi = std::min(force_s, KB);
    for (int64_t S = s_lo; S <= s_hi; ++S) {
      int64_t s_eff = 1;
      double t = cost(W, S, &s_eff);
      if (W == 1 && auto_w) t /= 0.97;  // width 1 must win by 3%
      if (best_t == 0.0 || t < best_t) {
        best_t = t;
        best.width = (int)W;
        best.splits = (int)s_eff;
      }
    }
  }
  return best;
}

// Decode tile kernel k splits: the S minimising
//   rounds x per-workgroup bytes / 30 GB/s
//   + (S > 1: reduce launch ~4 us + partial planes written and read at 4 TB/s)
// with rounds = ceil(workgroups / decode_target_wgs) and per-workgroup bytes
// = the split's k steps x 24 KiB (16 KiB of weights + 8 KiB of X per 64-k
// step: 64 columns of both SwiGLU matrices, 128 of the GEMM's).  A forced
// split count (> 0) is kept.
int decode_tile_splits(int nmat, int64_t M, int64_t KB, int64_t NB, int64_t force_s) {
  const int64_t target = std::max<int64_t>(1, llk::tunable("decode_target_wgs"));
  const int64_t min_kb = std::max<int64_t>(1, llk::tunable("decode_min_kb"));
  const int64_t rows = (M + 31) / 32 * 32;
  const int64_t groups = nmat == 2 ? NB * 2 : NB;
  int64_t s_lo = 1, s_hi = std::min<int64_t>(64, std::max<int64_t>(1, KB / min_kb));
  if (force_s > 0) s_lo = s_hi = std::min(force_s, KB);
  int best_s = 1;
  double best_t = 0.0;
  for (int64_t S = s_lo; S <= s_hi; ++S) {
    const int64_t kbs = (KB + S - 1) / S;
    const int64_t s_eff = (KB + kbs - 1) / kbs;  // no empty splits
    const int64_t wgs = groups * s_eff;
    double t = (double)((wgs + target - 1) / target) * (double)kbs * 24576.0 / 30e9;
    if (s_eff > 1) t += 4e-6 + 2.0 * s_eff * nmat * rows * NB * 128 * 4 / 4e12;
    if (best_t == 0.0 || t < best_t) {
      best_t = t;
      best_s = (int)s_eff;
    }
  }
  return best_s;
}

// x == nullptr: plan for the worst case (X needs padding).  Precedence for
// each knob: a forced tunable, then the active schedule DB's entry
// (small-M: group width = BN / 32, splits = grain_size; tile: splits =
// grain_size; BN 0 or grain_size 0 = choose from the shape), then the cost
// models (small_m_choice, tile_splits).
// max_ws: the largest workspace the caller can provide (the no-allocation
// entry point's fixed buffer); a plan that needs more takes fewer k splits
// and, for a padded X, shorter row chunks.
// accumulate (GEMM, C += A B): the tile path takes the partial planes at any
// S (the reduce adds C) and no tail split.
Plan plan_launch_base(int nmat, int64_t M, int64_t K, int64_t KB, int64_t NB,
                      const llk_tensor2d* x, size_t max_ws, bool accumulate, bool out_bf16) {
  Plan p;
  llk::ScheduleEntry se;
  const bool have_db = db_entry(nmat, M, &se);
  if (M <= std::min<int64_t>(64, llk::tunable("decode_max_m"))) {
    p.skinny = true;
    int64_t gw = llk::tunable("decode_group_width");
    if (gw <= 0 && have_db && (se.BN == 32 || se.BN == 64 || se.BN == 128)) gw = se.BN / 32;
    int64_t S = llk::tunable("decode_splits");
    if (S <= 0 && have_db && se.grain_size > 0) S = se.grain_size;
    auto fit_splits = [&](int s) {
      size_t ws = llk_skinny_workspace_bytes(nmat, (int)M, (int)(NB * 128), s);
      while (ws > max_ws && s > 1) ws = llk_skinny_workspace_bytes(nmat, (int)M, (int)(NB * 128), --s);
      return std::make_pair(s, ws);
    };
    const SmallMChoice c = small_m_choice(nmat, M, KB, NB, gw, S);
    p.G = c.width;
    std::tie(p.S, p.ws_bytes) = fit_splits(c.splits);
    // The decode tile kernel unless a width is forced (the small-M kernel's
    // own knob, or its schedule record) or the shape does not fit it; when
    // X is unknown (sizing), the larger of the two workspaces.
    if (llk::tunable("decode_tile") != 0 && gw <= 0 &&
        llk_decode_tile_fits((int)M, K, x ? x->stride0 : K)) {
      const auto d = fit_splits(decode_tile_splits(nmat, M, KB, NB, S));
      if (!x) {
        p.ws_bytes = std::max(p.ws_bytes, d.second);
      } else if (x_vec_ok(x)) {
        p.dtile = true;
        std::tie(p.S, p.ws_bytes) = d;
      }
    }
    return p;
  }
  // The tile kernel's buffer offsets are 32-bit: 256 rows of X and one
  // weight panel (KB x 16 KiB) must each span less than 2 GiB.  A wider
  // caller stride is copied into a dense padded buffer; a longer K is an
  // error.
  constexpr int64_t kTileMaxLd = ((int64_t)1 << 31) / (256 * 2);
  p.pad = !(x && x_vec_ok(x) && K % 64 == 0 && x->stride0 < kTileMaxLd);
  p.too_large = KB * 64 >= kTileMaxLd;
  p.ld = p.pad ? KB * 64 : x->stride0;
  p.chunk = M;
  if (!llk_tile_x_fits((int)std::min<int64_t>(M, kMaxDim), p.ld))
    p.chunk = std::max<int64_t>(256, (((int64_t)1 << 31) - 1) / (p.ld * 2) / 256 * 256 - 256);
  const int64_t rows = std::min(p.chunk, M);
  if (p.pad) p.pad_bytes = ((size_t)rows * p.ld * 2 + 255) / 256 * 256;
  const TilePlan tp = tile_plan(nmat, rows, KB, NB, have_db ? se.grain_size : 0);
  p.S = tp.S;
  p.head_nb = accumulate ? 0 : tp.head_nb;
  // The wide kernel: fused SwiGLU, bf16 output.  A forced split count or a
  // DB entry with one keeps the 128-column kernel unless tile_wide forces a
  // width (which then takes the forced split count).
  const int64_t forced_s = llk::tunable("tile_splits");
  const bool split_forced = forced_s > 0 || (have_db && se.grain_size > 1);
  const bool wide_forced = llk::tunable("tile_wide") == 7 || llk::tunable("tile_wide") == 11;
  if (nmat == 2 && out_bf16 && !accumulate && (!split_forced || wide_forced)) {
    const WideChoice wc = wide_choice(rows, NB * 128, KB, tp.cost, forced_s);
    if (wc.B) {
      p.wide = wc.B;
      p.S = wc.S;
      p.head_nb = 0;
    }
  }
  if (accumulate && tp.head_nb > 0) p.S = best_split(nmat, rows, KB, NB, 0).S;
  auto body = [&](int64_t crows) {
    if (p.wide)
      return p.pad_bytes + llk_swiglu_wide_split_bytes(p.wide, (int)crows, (int)(NB * 128), p.S);
    return p.pad_bytes + llk_tile_split_bytes(nmat == 2 ? 1 : 0, (int)crows,
                                              (int)(NB - p.head_nb), p.S, accumulate);
  };
  p.ws_bytes = body(rows);
  if (p.ws_bytes <= max_ws) return p;
  // Over the caller's limit: a padded X in row chunks that fit (whole
  // 256-row tiles; fewer than 256 rows do not fit: ws_bytes stays above
  // max_ws and the call is rejected), then the most k splits whose partial
  // planes fit beside it.
  if (p.pad && p.pad_bytes > max_ws) {
    const int64_t fit = (int64_t)(max_ws / ((size_t)p.ld * 2)) / 256 * 256;
    if (fit < 256) return p;
    p.chunk = std::min(p.chunk, fit);
    p.pad_bytes = ((size_t)std::min(p.chunk, M) * p.ld * 2 + 255) / 256 * 256;
  }
  const int64_t crows = std::min(p.chunk, M);
  for (; p.S >= 1; --p.S) {
    // a split count whose splits would not all be non-empty runs as the
    // count it effectively is (KB = 7, S = 5: 4 splits of 2 blocks)
    const int64_t kbs = (KB + p.S - 1) / p.S;
    p.S = (int)((KB + kbs - 1) / kbs);
    if (p.S == 1) p.head_nb = 0;
    p.ws_bytes = body(crows);
    if (p.ws_bytes <= max_ws || p.S == 1) break;
  }
  return p;
}

// Mid M (64 < M <= midm_max_m, at most 256; 128 by default): the decode
// tile kernel's 128- and 256-row forms when K is a multiple of 64 and X
// rows are 16-byte aligned -- one m tile, so every weight byte is read by
// one workgroup, with k splits from the forced `decode_splits`, else the
// schedule DB entry's grain_size, else the decode tile model (config 5's MLP
// at M = 128: the SwiGLU's 216 workgroups unsplit, the down projection's 40
// in 6 splits); otherwise the tile kernels.  With X unknown (sizing), the
// larger of the two workspaces.
Plan plan_launch(int nmat, int64_t M, int64_t K, int64_t KB, int64_t NB, const llk_tensor2d* x,
                 size_t max_ws = SIZE_MAX, bool accumulate = false, bool out_bf16 = true) {
  if (M > 64 && M <= std::min<int64_t>(256, llk::tunable("midm_max_m")) &&
      llk::tunable("decode_tile") != 0 && llk_decode_tile_fits((int)M, K, x ? x->stride0 : K)) {
    int64_t forced = llk::tunable("decode_splits");
    llk::ScheduleEntry se;
    if (forced <= 0 && db_entry(nmat, M, &se) && se.grain_size > 0) forced = se.grain_size;
    int s = decode_tile_splits(nmat, M, KB, NB, forced);
    size_t ws = llk_skinny_workspace_bytes(nmat, (int)M, (int)(NB * 128), s);
    while (ws > max_ws && s > 1) ws = llk_skinny_workspace_bytes(nmat, (int)M, (int)(NB * 128), --s);
    if (x && x_vec_ok(x)) {
      Plan p;
      p.skinny = true;
      p.dtile = true;
      p.S = s;
      p.ws_bytes = ws;
      return p;
    }
    if (!x) {
      Plan p = plan_launch_base(nmat, M, K, KB, NB, x, max_ws, accumulate, out_bf16);
      p.ws_bytes = std::max(p.ws_bytes, ws);
      return p;
    }
  }
  return plan_launch_base(nmat, M, K, KB, NB, x, max_ws, accumulate, out_bf16);
}

// K == 0: the reference's verifiers accept an empty reduction
// (LLKOps.cpp:42-83, 336-348) and its zero-filled fp32 accumulators
// (FuseDoubleContraction.cpp:119-135) give SiLU(0) * 0 = +0 for SwiGLU and
// C = 0 for the matmul: the output is filled with zeros.
int empty_reduction(llk_tensor2d* y, int out_dtype, llk_kernel_context* ctx, const char* what,
                    const llk::ModuleFns* mod) {
  hipError_t e = llk_launch_zero_rows(y->data, y->stride0, y->dim0, y->dim1,
                                      (int)dtype_size(out_dtype), mod, stream_of(ctx));
  return e == hipSuccess ? LLK_OK : fail_hip(e, what);
}

int launch_contraction(int mode, const llk_tensor2d* x, const llk_packed_weights* w0,
                       const llk_packed_weights* w1, llk_tensor2d* y, int out_dtype,
                       const Plan& p, uint8_t* ws, hipStream_t s, const char* what,
                       const llk::ModuleFns* mod, bool accumulate);

int run_contraction(int mode, const llk_tensor2d* x, const llk_packed_weights* w0,
                    const llk_packed_weights* w1, llk_tensor2d* y, int out_dtype,
                    llk_kernel_context* ctx, int dev, const char* what,
                    const llk::ModuleFns* mod, size_t max_ws = SIZE_MAX,
                    bool accumulate = false) {
  const int64_t M = x->dim0, K = x->dim1;
  const int nmat = mode == 1 ? 2 : 1;
  const Plan p = plan_launch(nmat, M, K, w0->KB, w0->NB, x, max_ws, accumulate,
                             out_dtype == LLK_BF16);
  if (p.too_large)
    return fail(LLK_ERR_SHAPE, "%s: K=%lld too large for M=%lld (the tile kernel needs K <= %lld)",
                what, (long long)K, (long long)M, (long long)(((int64_t)1 << 31) / 512 - 64));
  if (p.ws_bytes > max_ws)
    return fail(LLK_ERR_SCRATCH,
                "%s: M=%lld K=%lld needs %zu workspace bytes, more than the %zu available",
                what, (long long)M, (long long)K, p.ws_bytes, max_ws);
  void* ws = nullptr;
  Workspace* held = nullptr;
  int rc = get_workspace(dev, p.ws_bytes, ctx, &ws, &held);
  if (rc) return rc;
  hipStream_t s = stream_of(ctx);
  BindDone bind(held, s);
  rc = launch_contraction(mode, x, w0, w1, y, out_dtype, p, static_cast<uint8_t*>(ws), s, what,
                          mod, accumulate);
  bind.end();
  release_workspace(dev, held, s, bind.bound());
  return rc;
}

// Enqueues the plan's launches.  Workspace layout: [padded X][partial planes].
int launch_contraction(int mode, const llk_tensor2d* x, const llk_packed_weights* w0,
                       const llk_packed_weights* w1, llk_tensor2d* y, int out_dtype,
                       const Plan& p, uint8_t* body, hipStream_t s, const char* what,
                       const llk::ModuleFns* mod, bool accumulate) {
  const int64_t M = x->dim0, K = x->dim1, N = w0->N;
  const bool yvec = y_vec_ok(y, out_dtype);
  hipError_t e = hipSuccess;
  if (p.dtile) {
    e = llk_launch_decode_tile(mode, static_cast<const uint16_t*>(x->data), x->stride0, w0->dev,
                               w1 ? w1->dev : nullptr, y->data, y->stride0, (int)M, (int)N,
                               (int)w0->KB, (int)w0->NB, p.S, body, out_dtype, yvec, accumulate,
                               mod, s);
    if (e != hipSuccess) return fail_hip(e, what);
    return LLK_OK;
  }
  if (p.skinny) {
    e = llk_launch_skinny(mode, static_cast<const uint16_t*>(x->data), x->stride0, w0->dev,
                          w1 ? w1->dev : nullptr, y->data, y->stride0, (int)M, (int)N, (int)K,
                          (int)w0->KB, (int)w0->NB, p.S, p.G, body, out_dtype, x_vec_ok(x), yvec,
                          accumulate, mod, s);
    if (e != hipSuccess) return fail_hip(e, what);
    return LLK_OK;
  }
  const size_t ysz = dtype_size(out_dtype);
  for (int64_t m0 = 0; m0 < M && e == hipSuccess; m0 += p.chunk) {
    const int rows = (int)std::min(p.chunk, M - m0);
    const uint16_t* xp = static_cast<const uint16_t*>(x->data) + m0 * x->stride0;
    if (p.pad) {
      e = llk_launch_pad_rows(xp, x->stride0, rows, (int)K, reinterpret_cast<uint16_t*>(body),
                              p.ld, mod, s);
      if (e != hipSuccess) break;
      xp = reinterpret_cast<const uint16_t*>(body);
    }
    uint8_t* yp = static_cast<uint8_t*>(y->data) + m0 * y->stride0 * ysz;
    if (p.wide) {
      e = llk_launch_swiglu_wide(p.wide, xp, p.ld, w0->dev, w1->dev, yp, y->stride0, rows, (int)N,
                                 (int)w0->KB, (int)w0->NB, p.S,
                                 p.S > 1 ? body + p.pad_bytes : nullptr, mod, s);
      continue;
    }
    if (p.head_nb > 0) {
      e = llk_launch_tile(mode, xp, p.ld, w0->dev, w1 ? w1->dev : nullptr, yp, y->stride0, rows,
                          (int)(p.head_nb * 128), (int)w0->KB, (int)p.head_nb, 1, nullptr,
                          out_dtype, yvec, accumulate, mod, s);
      if (e != hipSuccess) break;
    }
    // Columns from n-block head_nb on: the packed payload of a matrix is
    // n-block major (KB blocks of 16 KiB per n-block), so they start
    // head_nb * KB blocks in.
    const size_t w_off = (size_t)p.head_nb * w0->KB * 16384;
    const int64_t n0 = p.head_nb * 128;
    e = llk_launch_tile(mode, xp, p.ld, static_cast<const uint8_t*>(w0->dev) + w_off,
                        w1 ? static_cast<const uint8_t*>(w1->dev) + w_off : nullptr,
                        yp + n0 * ysz, y->stride0, rows, (int)(N - n0), (int)w0->KB,
                        (int)(w0->NB - p.head_nb), p.S,
                        p.S > 1 || accumulate ? body + p.pad_bytes : nullptr, out_dtype, yvec,
                        accumulate, mod, s);
  }
  if (e != hipSuccess) return fail_hip(e, what);
  return LLK_OK;
}

}  // namespace

extern "C" {

const char* llk_last_error(void) { return g_error.c_str(); }

int llk_abi_version(void) { return LLK_ABI_VERSION; }

int llk_device_info(char* arch_name, int cap, int* cu_count, int* lds_bytes, int* clock_khz) {
  int dev = -1;
  int rc = current_device(&dev);
  if (dev < 0) return rc;
  DeviceState& st = g_dev[dev];
  if (arch_name && cap > 0) std::snprintf(arch_name, cap, "%s", st.arch);
  if (cu_count) *cu_count = st.cu_count;
  if (lds_bytes) *lds_bytes = st.lds;
  if (clock_khz) *clock_khz = st.clock_khz;
  return rc;
}

// ---------------------------------------------------------------------------
// Packed weights
// ---------------------------------------------------------------------------

static int check_weight_input(const llk_tensor2d* w, int64_t bk) {
  int rc = check_tensor(w, "w");
  if (rc) return rc;
  if (bk <= 0) return fail(LLK_ERR_INVALID_ARGUMENT, "BK must be positive (got %lld)", (long long)bk);
  if (w->dim0 > kMaxDim || w->dim1 > kMaxDim)
    return fail(LLK_ERR_SHAPE, "weight dimensions too large");
  return LLK_OK;
}

static void fill_meta(llk_packed_weights* pw, int64_t K, int64_t N, int64_t bk) {
  pw->K = K;
  pw->N = N;
  pw->BK = bk;
  pw->K_blocks = (K + bk - 1) / bk;
  pw->block_size = bk * N * 2;
  pw->dtype = LLK_BF16;
  pw->KB = llk::deviceBlocksK(K);
  pw->NB = llk::deviceBlocksN(N);
}

int llk_pack_weights(const llk_tensor2d* w, int64_t bk, unsigned flags,
                     llk_packed_weights** out) {
  if (!out) return fail(LLK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  int rc = check_weight_input(w, bk);
  if (rc) return rc;
  const bool host_only = (flags & LLK_PACK_HOST_ONLY) != 0;
  int dev = -1;
  if (!host_only) {
    rc = current_device(&dev);
    if (rc) return rc;
  }
  auto* pw = new (std::nothrow) llk_packed_weights();
  if (!pw) return fail(LLK_ERR_OUT_OF_MEMORY, "handle allocation");
  fill_meta(pw, w->dim0, w->dim1, bk);
  const uint16_t* src = static_cast<const uint16_t*>(w->data);
  try {
    if (flags & (LLK_PACK_KEEP_HOST | LLK_PACK_HOST_ONLY)) {
      pw->host.resize(static_cast<size_t>(pw->K_blocks * bk * pw->N));
      if (!pw->host.empty()) llk::packReferenceLayout(src, pw->K, pw->N, w->stride0, bk, pw->host.data());
    }
    if (host_only) {
      *out = pw;
      return LLK_OK;
    }
    pw->dev_bytes = llk::deviceLayoutBytes(pw->K, pw->N);
    if (pw->dev_bytes == 0) {
      // Empty matrix: keep a small zeroed payload so the handle is usable.
      hipError_t e = hipMalloc(&pw->dev, 256);
      if (e == hipSuccess) e = hipMemset(pw->dev, 0, 256);
      if (e != hipSuccess) {
        llk_packed_weights_free(pw);
        return fail_hip(e, "hipMalloc(empty payload)");
      }
    } else {
      std::vector<uint8_t> staging(pw->dev_bytes);
      llk::packDeviceLayout(src, pw->K, pw->N, w->stride0, staging.data());
      hipError_t e = hipMalloc(&pw->dev, pw->dev_bytes);
      if (e != hipSuccess) {
        pw->dev = nullptr;
        llk_packed_weights_free(pw);
        return fail(LLK_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", pw->dev_bytes, hipGetErrorString(e));
      }
      e = hipMemcpy(pw->dev, staging.data(), pw->dev_bytes, hipMemcpyHostToDevice);
      if (e != hipSuccess) {
        llk_packed_weights_free(pw);
        return fail_hip(e, "hipMemcpy(packed weights)");
      }
    }
  } catch (const std::bad_alloc&) {
    llk_packed_weights_free(pw);
    return fail(LLK_ERR_OUT_OF_MEMORY, "host allocation while packing");
  }
  pw->device = dev;
  *out = pw;
  return LLK_OK;
}

int llk_pack_weights_device(const llk_tensor2d* w, int64_t bk, void* stream,
                            llk_packed_weights** out) {
  if (!out) return fail(LLK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  int rc = check_weight_input(w, bk);
  if (rc) return rc;
  int dev;
  rc = current_device(&dev);
  if (rc) return rc;
  auto* pw = new (std::nothrow) llk_packed_weights();
  if (!pw) return fail(LLK_ERR_OUT_OF_MEMORY, "handle allocation");
  fill_meta(pw, w->dim0, w->dim1, bk);
  pw->dev_bytes = llk::deviceLayoutBytes(pw->K, pw->N);
  if (pw->dev_bytes == 0) {
    // Empty matrix: a small zeroed payload, as llk_pack_weights keeps.
    hipError_t e = hipMalloc(&pw->dev, 256);
    if (e == hipSuccess) e = hipMemset(pw->dev, 0, 256);
    if (e != hipSuccess) {
      llk_packed_weights_free(pw);
      return fail_hip(e, "hipMalloc(empty payload)");
    }
  } else {
    hipError_t e = hipMalloc(&pw->dev, pw->dev_bytes);
    if (e != hipSuccess) {
      pw->dev = nullptr;
      llk_packed_weights_free(pw);
      return fail(LLK_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", pw->dev_bytes, hipGetErrorString(e));
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    e = llk_launch_pack(static_cast<const uint16_t*>(w->data), w->stride0, (int)pw->K, (int)pw->N,
                        (int)pw->KB, (int)pw->NB, pw->dev, nullptr, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      llk_packed_weights_free(pw);
      return fail_hip(e, "pack kernel");
    }
  }
  pw->device = dev;
  *out = pw;
  return LLK_OK;
}

int llk_repack(llk_packed_weights* pw, const llk_tensor2d* w) {
  if (!pw) return fail(LLK_ERR_INVALID_ARGUMENT, "handle is NULL");
  int rc = check_weight_input(w, pw->BK);
  if (rc) return rc;
  if (!pw->owns_dev)
    return fail(LLK_ERR_INVALID_ARGUMENT, "handle is a view over memory it does not own");
  if (w->dim0 != pw->K || w->dim1 != pw->N)
    return fail(LLK_ERR_SHAPE, "repack shape (%lld, %lld) differs from packed (%lld, %lld)",
                (long long)w->dim0, (long long)w->dim1, (long long)pw->K, (long long)pw->N);
  llk_packed_weights* fresh = nullptr;
  // A host-only handle repacks on the host; a device handle repacks on the
  // device it was packed for.
  const bool on_device = pw->dev != nullptr;
  int dev_saved = 0;
  if (on_device) {
    hipError_t e = hipGetDevice(&dev_saved);
    if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
    if (pw->device != dev_saved) {
      e = hipSetDevice(pw->device);
      if (e != hipSuccess) return fail_hip(e, "hipSetDevice");
    }
  }
  const unsigned fl =
      on_device ? (pw->host.empty() ? 0u : LLK_PACK_KEEP_HOST) : LLK_PACK_HOST_ONLY;
  rc = llk_pack_weights(w, pw->BK, fl, &fresh);
  if (on_device && pw->device != dev_saved) (void)hipSetDevice(dev_saved);
  if (rc) return rc;
  if (pw->dev) (void)hipFree(pw->dev);
  pw->host.swap(fresh->host);
  pw->dev = fresh->dev;
  pw->dev_bytes = fresh->dev_bytes;
  pw->device = fresh->device;
  fresh->dev = nullptr;
  llk_packed_weights_free(fresh);
  return LLK_OK;
}

void llk_packed_weights_free(llk_packed_weights* pw) {
  if (!pw) return;
  if (pw->dev && pw->owns_dev) (void)hipFree(pw->dev);
  delete pw;
}

int64_t llk_packed_weights_k_blocks(const llk_packed_weights* pw) { return pw ? pw->K_blocks : 0; }
int64_t llk_packed_weights_n(const llk_packed_weights* pw) { return pw ? pw->N : 0; }
int64_t llk_packed_weights_block_size(const llk_packed_weights* pw) { return pw ? pw->block_size : 0; }
int64_t llk_packed_weights_bk(const llk_packed_weights* pw) { return pw ? pw->BK : 0; }
int llk_packed_weights_dtype(const llk_packed_weights* pw) { return pw ? pw->dtype : -1; }
int64_t llk_packed_weights_k(const llk_packed_weights* pw) { return pw ? pw->K : 0; }
const void* llk_packed_weights_host_data(const llk_packed_weights* pw) {
  return (pw && !pw->host.empty()) ? pw->host.data() : nullptr;
}
const void* llk_packed_weights_device_data(const llk_packed_weights* pw) { return pw ? pw->dev : nullptr; }
size_t llk_packed_weights_device_bytes(const llk_packed_weights* pw) { return pw ? pw->dev_bytes : 0; }

size_t llk_pack_device_bytes(int64_t K, int64_t N) {
  if (K < 0 || N < 0) return 0;
  return llk::deviceLayoutBytes(K, N);
}

int llk_pack_device_layout(const llk_tensor2d* w, void* out) {
  int rc = check_tensor(w, "w");
  if (rc) return rc;
  if (!out) return fail(LLK_ERR_INVALID_ARGUMENT, "out is NULL");
  llk::packDeviceLayout(static_cast<const uint16_t*>(w->data), w->dim0, w->dim1, w->stride0,
                        static_cast<uint8_t*>(out));
  return LLK_OK;
}

// ---------------------------------------------------------------------------
// Serialized packed weights
// ---------------------------------------------------------------------------

}  // extern "C"

namespace {

struct BlobHeader {
  char magic[8];
  uint32_t version, dtype;
  int64_t K, N, BK, K_blocks, block_size, KB, NB;
  uint64_t payload_bytes, checksum, reserved;
};
static_assert(sizeof(BlobHeader) == 96, "blob header is 96 bytes");
constexpr char kBlobMagic[8] = {'L', 'L', 'K', 'P', 'W', '9', '5', '0'};

uint64_t fnv1a64(const uint8_t* p, size_t n) {
  uint64_t h = 0xcbf29ce484222325ULL;
  for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 0x100000001b3ULL;
  return h;
}

// Device-layout payload of a handle in host memory: copied back from the
// GPU, or computed from the host layout ([K_blocks][BK][N] holds the rows
// of W in order, so it is W itself with row stride N).
int payload_to_host(const llk_packed_weights* pw, uint8_t* out) {
  const size_t bytes = llk::deviceLayoutBytes(pw->K, pw->N);
  if (bytes == 0) return LLK_OK;
  if (pw->dev) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != pw->device) e = hipSetDevice(pw->device);
    if (e == hipSuccess) e = hipMemcpy(out, pw->dev, bytes, hipMemcpyDeviceToHost);
    if (cur != pw->device) (void)hipSetDevice(cur);
    return e == hipSuccess ? LLK_OK : fail_hip(e, "hipMemcpy(payload to host)");
  }
  if (pw->host.empty()) return fail(LLK_ERR_INVALID_ARGUMENT, "handle holds no payload");
  llk::packDeviceLayout(pw->host.data(), pw->K, pw->N, pw->N, out);
  return LLK_OK;
}

}  // namespace

namespace llk {
// Error hook for the runtime sources built outside this file.
int setError(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace llk

extern "C" {

int llk_packed_weights_serialize(const llk_packed_weights* pw, void* out, size_t cap,
                                 size_t* len) {
  if (!pw || !len) return fail(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  const size_t payload = llk::deviceLayoutBytes(pw->K, pw->N);
  *len = sizeof(BlobHeader) + payload;
  if (!out) return LLK_OK;
  if (cap < *len) return fail(LLK_ERR_INVALID_ARGUMENT, "blob needs %zu bytes, cap %zu", *len, cap);
  BlobHeader h{};
  std::memcpy(h.magic, kBlobMagic, 8);
  h.version = 1;
  h.dtype = static_cast<uint32_t>(pw->dtype);
  h.K = pw->K;
  h.N = pw->N;
  h.BK = pw->BK;
  h.K_blocks = pw->K_blocks;
  h.block_size = pw->block_size;
  h.KB = pw->KB;
  h.NB = pw->NB;
  h.payload_bytes = payload;
  uint8_t* body = static_cast<uint8_t*>(out) + sizeof(BlobHeader);
  int rc = payload_to_host(pw, body);
  if (rc) return rc;
  h.checksum = fnv1a64(body, payload);
  std::memcpy(out, &h, sizeof(h));
  return LLK_OK;
}

int llk_packed_weights_deserialize(const void* blob, size_t len, unsigned flags,
                                   llk_packed_weights** out) {
  if (!blob || !out) return fail(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  if (len < sizeof(BlobHeader)) return fail(LLK_ERR_INVALID_ARGUMENT, "blob shorter than its header");
  BlobHeader h;
  std::memcpy(&h, blob, sizeof(h));
  if (std::memcmp(h.magic, kBlobMagic, 8) != 0 || h.version != 1)
    return fail(LLK_ERR_INVALID_ARGUMENT, "not a version-1 packed-weights blob");
  if (h.dtype != LLK_BF16 || h.K < 0 || h.N < 0 || h.BK <= 0 || h.K > kMaxDim || h.N > kMaxDim ||
      h.K_blocks != (h.K + h.BK - 1) / h.BK || h.block_size != h.BK * h.N * 2 ||
      h.KB != llk::deviceBlocksK(h.K) || h.NB != llk::deviceBlocksN(h.N) ||
      h.payload_bytes != llk::deviceLayoutBytes(h.K, h.N))
    return fail(LLK_ERR_INVALID_ARGUMENT, "inconsistent packed-weights header");
  if (len < sizeof(BlobHeader) + h.payload_bytes)
    return fail(LLK_ERR_INVALID_ARGUMENT, "blob truncated: %zu < %zu bytes", len,
                (size_t)(sizeof(BlobHeader) + h.payload_bytes));
  const uint8_t* body = static_cast<const uint8_t*>(blob) + sizeof(BlobHeader);
  if (fnv1a64(body, h.payload_bytes) != h.checksum)
    return fail(LLK_ERR_INVALID_ARGUMENT, "packed-weights payload checksum mismatch");
  const bool host_only = (flags & LLK_PACK_HOST_ONLY) != 0;
  int dev = -1;
  if (!host_only) {
    int rc = current_device(&dev);
    if (rc) return rc;
  }
  auto* pw = new (std::nothrow) llk_packed_weights();
  if (!pw) return fail(LLK_ERR_OUT_OF_MEMORY, "handle allocation");
  fill_meta(pw, h.K, h.N, h.BK);
  try {
    if (flags & (LLK_PACK_KEEP_HOST | LLK_PACK_HOST_ONLY)) {
      pw->host.assign(static_cast<size_t>(pw->K_blocks * pw->BK * pw->N), 0);
      if (h.payload_bytes) llk::unpackDeviceLayout(body, h.K, h.N, pw->host.data(), h.N);
    }
  } catch (const std::bad_alloc&) {
    llk_packed_weights_free(pw);
    return fail(LLK_ERR_OUT_OF_MEMORY, "host allocation while unpacking");
  }
  if (!host_only) {
    pw->dev_bytes = h.payload_bytes;
    const size_t alloc = h.payload_bytes ? h.payload_bytes : 256;
    hipError_t e = hipMalloc(&pw->dev, alloc);
    if (e != hipSuccess) {
      pw->dev = nullptr;
      llk_packed_weights_free(pw);
      return fail(LLK_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", alloc, hipGetErrorString(e));
    }
    e = h.payload_bytes ? hipMemcpy(pw->dev, body, h.payload_bytes, hipMemcpyHostToDevice)
                        : hipMemset(pw->dev, 0, alloc);
    if (e != hipSuccess) {
      llk_packed_weights_free(pw);
      return fail_hip(e, "upload of packed weights");
    }
    pw->device = dev;
  }
  *out = pw;
  return LLK_OK;
}

int llk_packed_weights_save(const llk_packed_weights* pw, const char* path) {
  if (!pw || !path) return fail(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  size_t len = 0;
  int rc = llk_packed_weights_serialize(pw, nullptr, 0, &len);
  if (rc) return rc;
  std::vector<uint8_t> buf;
  try {
    buf.resize(len);
  } catch (const std::bad_alloc&) {
    return fail(LLK_ERR_OUT_OF_MEMORY, "host allocation of %zu bytes", len);
  }
  rc = llk_packed_weights_serialize(pw, buf.data(), len, &len);
  if (rc) return rc;
  FILE* f = std::fopen(path, "wb");
  if (!f) return fail(LLK_ERR_NOT_FOUND, "cannot open %s for writing", path);
  const bool ok = std::fwrite(buf.data(), 1, len, f) == len;
  const bool closed = std::fclose(f) == 0;
  if (!ok || !closed) return fail(LLK_ERR_NOT_FOUND, "short write to %s", path);
  return LLK_OK;
}

int llk_packed_weights_load(const char* path, unsigned flags, llk_packed_weights** out) {
  if (!path || !out) return fail(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  FILE* f = std::fopen(path, "rb");
  if (!f) return fail(LLK_ERR_NOT_FOUND, "cannot open %s", path);
  std::vector<uint8_t> buf;
  uint8_t chunk[1 << 16];
  size_t n;
  try {
    while ((n = std::fread(chunk, 1, sizeof(chunk), f)) > 0) buf.insert(buf.end(), chunk, chunk + n);
  } catch (const std::bad_alloc&) {
    std::fclose(f);
    return fail(LLK_ERR_OUT_OF_MEMORY, "host allocation while reading %s", path);
  }
  const bool err = std::ferror(f) != 0;
  std::fclose(f);
  if (err) return fail(LLK_ERR_NOT_FOUND, "read error on %s", path);
  return llk_packed_weights_deserialize(buf.data(), buf.size(), flags, out);
}

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------

size_t llk_swiglu_scratch_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // Either output type (the bf16 plan may take the wide kernel, which needs
  // no partial planes).
  const int64_t KB = llk::deviceBlocksK(K), NB = llk::deviceBlocksN(N);
  return std::max(plan_launch(2, M, K, KB, NB, nullptr, SIZE_MAX, false, true).ws_bytes,
                  plan_launch(2, M, K, KB, NB, nullptr, SIZE_MAX, false, false).ws_bytes);
}

int llk_describe_launch(int operation, int64_t M, int64_t N, int64_t K, unsigned flags,
                        llk_launch_plan* out) {
  if (!out) return fail(LLK_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = llk_launch_plan{};
  if (operation != 0 && operation != 3)
    return fail(LLK_ERR_INVALID_ARGUMENT, "operation %d has no gfx950 kernel", operation);
  if (flags & ~(LLK_PLAN_X_ALIGNED | LLK_PLAN_ACCUMULATE | LLK_PLAN_OUT_F32))
    return fail(LLK_ERR_INVALID_ARGUMENT, "unknown plan flags 0x%x", flags);
  const bool accumulate = (flags & LLK_PLAN_ACCUMULATE) != 0;
  if (accumulate && operation != 3)
    return fail(LLK_ERR_INVALID_ARGUMENT, "LLK_PLAN_ACCUMULATE applies to the matmul only");
  if (M < 1 || N < 1 || K < 1 || M > kMaxDim || N > kMaxDim || K > kMaxDim)
    return fail(LLK_ERR_SHAPE, "M, N, K must be in [1, 2^30]");
  const int nmat = operation == 0 ? 2 : 1;
  const int64_t KB = llk::deviceBlocksK(K), NB = llk::deviceBlocksN(N);
  // A stand-in X with the requested alignment (plan_launch reads only the
  // pointer's alignment, the row stride and K).
  const bool x_aligned = (flags & LLK_PLAN_X_ALIGNED) != 0;
  llk_tensor2d x{reinterpret_cast<void*>(x_aligned ? 256 : 2), M, K, x_aligned ? K : K + 1, 1};
  const Plan p = plan_launch(nmat, M, K, KB, NB, &x, SIZE_MAX, accumulate,
                             (flags & LLK_PLAN_OUT_F32) == 0);
  if (p.too_large)
    return fail(LLK_ERR_SHAPE, "K=%lld too large for M=%lld (the tile kernel needs K <= %lld)",
                (long long)K, (long long)M, (long long)(((int64_t)1 << 31) / 512 - 64));
  out->splits = p.S;
  out->workspace_bytes = p.ws_bytes;
  if (p.dtile) {
    out->kernel = 3;
    out->group_width = 0;
    out->tile_columns = nmat == 2 ? 64 : 128;
    out->workgroups = (nmat == 2 ? NB * 2 : NB) * p.S;
    out->threads_per_workgroup = 256;
    out->launches = p.S > 1 ? 2 : 1;
    return LLK_OK;
  }
  if (p.skinny) {
    out->kernel = 0;
    out->group_width = p.G;
    out->workgroups = NB * 4 / p.G * p.S;
    out->threads_per_workgroup = llk_skinny_threads(nmat, (int)M, p.G);
    out->launches = p.S > 1 ? 2 : 1;
    return LLK_OK;
  }
  out->kernel = 1;
  out->group_width = 0;
  out->pad_x = p.pad ? 1 : 0;
  const int64_t rows = std::min(p.chunk, M);
  const int64_t chunks = (M + p.chunk - 1) / p.chunk;
  out->threads_per_workgroup = 256;
  if (p.wide) {
    out->kernel = 2;
    out->tile_columns = 16 * p.wide;
    out->workgroups = (rows + 255) / 256 * ((N + 16 * p.wide - 1) / (16 * p.wide)) * p.S;
    out->launches = chunks * (1 + (p.pad ? 1 : 0) + (p.S > 1 ? 1 : 0));
    return LLK_OK;
  }
  out->tile_columns = nmat == 2 ? 128 : 256;
  const int64_t nb_per_tile = nmat == 2 ? 1 : 2, tail_nb = NB - p.head_nb;
  out->workgroups = (rows + 255) / 256 *
                    (p.head_nb / nb_per_tile + (tail_nb + nb_per_tile - 1) / nb_per_tile * p.S);
  // An accumulating launch always ends with the reduce (it adds C).
  out->launches = chunks * (1 + (p.head_nb > 0 ? 1 : 0) + (p.pad ? 1 : 0) +
                            (p.S > 1 || accumulate ? 1 : 0));
  out->head_blocks_n = p.head_nb;
  return LLK_OK;
}

int llk_workspace_stats(size_t* count, size_t* bytes) {
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  DeviceState& st = g_dev[dev];
  std::lock_guard<std::mutex> lk(st.mu);
  size_t n = 0, b = 0;
  for (const auto& kv : st.ws) {
    if (!kv.second.ptr) continue;
    ++n;
    b += kv.second.bytes;
  }
  if (count) *count = n;
  if (bytes) *bytes = b;
  return LLK_OK;
}

int llk_workspace_trim(void) {
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  DeviceState& st = g_dev[dev];
  std::lock_guard<std::mutex> lk(st.mu);
  while (evict_one_workspace(st, nullptr)) {
  }
  return LLK_OK;
}

int llk_verify_fused_swiglu(int64_t x_m, int64_t x_k, int64_t wg_k, int64_t wg_n, int64_t wu_k,
                            int64_t wu_n, int64_t init_m, int64_t init_n) {
  auto known = [](int64_t a, int64_t b) { return a >= 0 && b >= 0; };
  if (known(x_m, init_m) && x_m != init_m)
    return fail(LLK_ERR_SHAPE, "M dimension mismatch: X=%lld vs init=%lld", (long long)x_m,
                (long long)init_m);
  if (known(wg_n, init_n) && wg_n != init_n)
    return fail(LLK_ERR_SHAPE, "N dimension mismatch: Wg=%lld vs init=%lld", (long long)wg_n,
                (long long)init_n);
  if (known(x_k, wg_k) && x_k != wg_k)
    return fail(LLK_ERR_SHAPE, "K dimension mismatch between X=%lld and Wg=%lld", (long long)x_k,
                (long long)wg_k);
  if (known(x_k, wu_k) && x_k != wu_k)
    return fail(LLK_ERR_SHAPE, "K dimension mismatch between X=%lld and Wu=%lld", (long long)x_k,
                (long long)wu_k);
  if (known(wg_n, wu_n) && wg_n != wu_n)
    return fail(LLK_ERR_SHAPE, "N dimension mismatch between Wg=%lld and Wu=%lld", (long long)wg_n,
                (long long)wu_n);
  return LLK_OK;
}

int llk_verify_matmul(int64_t a_k, int64_t b_k) {
  if (a_k >= 0 && b_k >= 0 && a_k != b_k)
    return fail(LLK_ERR_SHAPE, "K dimension must match: %lld vs %lld", (long long)a_k,
                (long long)b_k);
  return LLK_OK;
}

}  // extern "C"

namespace {

// llk_swiglu_bf16 and its no-allocation variant (noalloc: the workspace is
// the device's `scratch` array, whatever ctx->scratch says); mod: the
// loaded code object whose kernels run (null: the library's own).
int swiglu_entry(const llk_tensor2d* x, const llk_packed_weights* wg,
                 const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                 llk_kernel_context* ctx, bool noalloc, const llk::ModuleFns* mod) {
  int rc;
  if ((rc = check_tensor(x, "x")) || (rc = check_tensor(y, "y"))) return rc;
  if (y_dtype != LLK_BF16 && y_dtype != LLK_FP32)
    return fail(LLK_ERR_DTYPE, "y_dtype %d unsupported (bf16 or f32)", y_dtype);
  if (!wg || !wu) return fail(LLK_ERR_INVALID_ARGUMENT, "packed weights handle is NULL");
  const int64_t M = x->dim0, K = x->dim1;
  if ((rc = llk_verify_fused_swiglu(M, K, wg->K, wg->N, wu->K, wu->N, y->dim0, y->dim1))) return rc;
  if (M > kMaxDim) return fail(LLK_ERR_SHAPE, "M too large");
  if (M == 0 || wg->N == 0) return LLK_OK;
  int dev;
  if ((rc = current_device(&dev))) return rc;
  if ((rc = check_packed(wg, "wg", dev)) || (rc = check_packed(wu, "wu", dev))) return rc;
  if (K == 0) return empty_reduction(y, y_dtype, ctx, "swiglu", mod);
  if (!noalloc) return run_contraction(1, x, wg, wu, y, y_dtype, ctx, dev, "swiglu", mod);
  llk_kernel_context fixed{nullptr, kNoAllocScratchBytes, ctx ? ctx->stream : nullptr};
  if ((rc = noalloc_scratch(dev, &fixed.scratch))) return rc;
  return run_contraction(1, x, wg, wu, y, y_dtype, &fixed, dev, "swiglu (no allocation)", mod,
                         kNoAllocScratchBytes);
}

// llk_gemm_bf16 (accumulate: llk_gemm_bf16_accumulate, C += A B).
int gemm_entry(const llk_tensor2d* a, const llk_packed_weights* b, llk_tensor2d* c, int c_dtype,
               llk_kernel_context* ctx, const llk::ModuleFns* mod, bool accumulate = false) {
  int rc;
  if ((rc = check_tensor(a, "a")) || (rc = check_tensor(c, "c"))) return rc;
  if (c_dtype != LLK_BF16 && c_dtype != LLK_FP16 && c_dtype != LLK_FP32)
    return fail(LLK_ERR_DTYPE, "c_dtype %d unsupported (bf16, f16 or f32)", c_dtype);
  if (!b) return fail(LLK_ERR_INVALID_ARGUMENT, "packed weights handle is NULL");
  const int64_t M = a->dim0, K = a->dim1, N = b->N;
  // llk.matmul / micro.mma contract: lhs [M,K], rhs [K,N], acc [M,N].
  if ((rc = llk_verify_matmul(K, b->K))) return rc;
  if (c->dim0 != M || c->dim1 != N)
    return fail(LLK_ERR_SHAPE, "c shape (%lld, %lld) != (%lld, %lld)", (long long)c->dim0,
                (long long)c->dim1, (long long)M, (long long)N);
  if (M > kMaxDim) return fail(LLK_ERR_SHAPE, "M too large");
  if (M == 0 || N == 0) return LLK_OK;
  int dev;
  if ((rc = current_device(&dev))) return rc;
  if ((rc = check_packed(b, "b", dev))) return rc;
  // An empty reduction adds nothing: C stays as it is (-0 included).
  if (K == 0) return accumulate ? LLK_OK : empty_reduction(c, c_dtype, ctx, "gemm", mod);
  return run_contraction(0, a, b, nullptr, c, c_dtype, ctx, dev,
                         accumulate ? "gemm (accumulate)" : "gemm", mod, SIZE_MAX, accumulate);
}

}  // namespace

extern "C" {

int llk_swiglu_bf16(const llk_tensor2d* x, const llk_packed_weights* wg,
                    const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                    llk_kernel_context* ctx) {
  return swiglu_entry(x, wg, wu, y, y_dtype, ctx, false, nullptr);
}

int llk_swiglu_bf16_noalloc(const llk_tensor2d* x, const llk_packed_weights* wg,
                            const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                            void* stream) {
  llk_kernel_context ctx{nullptr, 0, stream};
  return swiglu_entry(x, wg, wu, y, y_dtype, &ctx, true, nullptr);
}

int llk_gemm_bf16(const llk_tensor2d* a, const llk_packed_weights* b, llk_tensor2d* c,
                  int c_dtype, llk_kernel_context* ctx) {
  return gemm_entry(a, b, c, c_dtype, ctx, nullptr);
}

int llk_gemm_bf16_accumulate(const llk_tensor2d* a, const llk_packed_weights* b, llk_tensor2d* c,
                             int c_dtype, llk_kernel_context* ctx) {
  return gemm_entry(a, b, c, c_dtype, ctx, nullptr, true);
}

int llk_mlp_bf16(const llk_tensor2d* x, const llk_packed_weights* wg, const llk_packed_weights* wu,
                 const llk_packed_weights* wd, llk_tensor2d* y, llk_tensor2d* z,
                 llk_kernel_context* ctx) {
  if (!wd) return fail(LLK_ERR_INVALID_ARGUMENT, "wd is NULL");
  if (wg && wd->K != wg->N)
    return fail(LLK_ERR_SHAPE, "Wd rows (%lld) != SwiGLU N (%lld)", (long long)wd->K, (long long)wg->N);
  int rc = llk_swiglu_bf16(x, wg, wu, y, LLK_BF16, ctx);
  if (rc) return rc;
  return llk_gemm_bf16(y, wd, z, LLK_BF16, ctx);
}

}  // extern "C"

namespace llk {

int pack_into(const llk_tensor2d* w, int64_t bk, bool w_on_device, void* dst, hipStream_t s,
              const ModuleFns* mod, llk_packed_weights** view) {
  if (!view) return fail(LLK_ERR_INVALID_ARGUMENT, "view is NULL");
  int rc = check_weight_input(w, bk);
  if (rc) return rc;
  int dev = -1;
  if ((rc = current_device(&dev))) return rc;
  if (!*view) {
    *view = new (std::nothrow) llk_packed_weights();
    if (!*view) return fail(LLK_ERR_OUT_OF_MEMORY, "handle allocation");
  }
  llk_packed_weights* v = *view;
  fill_meta(v, w->dim0, w->dim1, bk);
  v->host.clear();
  v->owns_dev = false;
  v->dev = dst;
  v->dev_bytes = llk::deviceLayoutBytes(v->K, v->N);
  v->device = dev;
  if (v->dev_bytes == 0) return LLK_OK;
  if (!dst) return fail(LLK_ERR_INVALID_ARGUMENT, "pack destination is NULL");
  const uint16_t* src = static_cast<const uint16_t*>(w->data);
  hipError_t e;
  if (w_on_device) {
    e = llk_launch_pack(src, w->stride0, (int)v->K, (int)v->N, (int)v->KB, (int)v->NB, dst, mod, s);
    return e == hipSuccess ? LLK_OK : fail_hip(e, "pack kernel");
  }
  std::vector<uint8_t> staging;
  try {
    staging.resize(v->dev_bytes);
  } catch (const std::bad_alloc&) {
    return fail(LLK_ERR_OUT_OF_MEMORY, "host allocation while packing");
  }
  llk::packDeviceLayout(src, v->K, v->N, w->stride0, staging.data());
  e = hipMemcpyAsync(dst, staging.data(), v->dev_bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);  // staging is freed on return
  return e == hipSuccess ? LLK_OK : fail_hip(e, "upload of packed weights");
}

// Row-major weights straight into the kernels, for the KernelFn path
// (kernel_fn.cpp), which otherwise packs the caller's weights on every call:
// x, wg (and wu for SwiGLU, mode 1; GEMM: mode 0, accumulate adds the
// existing y) and y in device memory, weights bf16 [K, N].  Taken (*taken =
// true) where
//  * the dispatcher's plan for the shape and X is the decode tile kernel
//    with at most 128 rows and the weights' rows suit its loads
//    (llk_decode_rowmajor_fits): that plan, with the same grid, k splits and
//    MFMA operands, so the result equals the packed path's bit for bit;
//  * otherwise, on the tile path (X aligned, K a multiple of 64,
//    llk_tile_rowmajor_fits), the tile kernel's row-major form: for the
//    fused SwiGLU (bf16 or fp32 result), the 128-column kernel's plan -- k
//    splits, and the unsplit head columns launched first where the plan
//    splits only the tail (a column offset into the weights and Y) -- never
//    the wide tiles, whose unsplit and equal-split bits are the 128-column
//    kernel's anyway; for the accumulating GEMM, the plan itself (k-split
//    planes, the reduce adding y).
// Otherwise nothing is launched and the caller packs.
int rowmajor_with_module(int mode, const llk_tensor2d* x, const llk_tensor2d* wg,
                         const llk_tensor2d* wu, llk_tensor2d* y, int out_dtype,
                         llk_kernel_context* ctx, const ModuleFns* mod, bool accumulate,
                         bool* taken) {
  *taken = false;
  if (llk::tunable("kernel_fn_rowmajor") == 0) return LLK_OK;
  const int64_t M = x->dim0, K = x->dim1, N = wg->dim1;
  if (M < 1 || N < 1 || K < 1 || y->dim0 != M || y->dim1 != N || !x_vec_ok(x)) return LLK_OK;
  if (wg->stride1 != 1 || (mode == 1 && (!wu || wu->stride1 != 1 || wu->dim1 != N))) return LLK_OK;
  const int nmat = mode == 1 ? 2 : 1;
  const int64_t KB = llk::deviceBlocksK(K), NB = llk::deviceBlocksN(N);
  const Plan p = plan_launch(nmat, M, K, KB, NB, x, SIZE_MAX, accumulate, out_dtype == LLK_BF16);
  auto fits = [&](bool (*f)(int, int64_t, int64_t, const void*, int64_t, int64_t)) {
    return f((int)M, K, x->stride0, wg->data, wg->stride0, N) &&
           (mode != 1 || f((int)M, K, x->stride0, wu->data, wu->stride0, N));
  };
  int S = p.S;
  size_t ws_bytes = p.ws_bytes;
  bool tile = false;
  int64_t head_cols = 0;  // tile form: columns of the unsplit head launch
  if (p.dtile && M <= 128) {
    if (!fits(&llk_decode_rowmajor_fits)) return LLK_OK;
  } else if (!p.skinny && mode == 1 && (out_dtype == LLK_BF16 || out_dtype == LLK_FP32) &&
             !accumulate && !p.pad && p.chunk >= M && fits(&llk_tile_rowmajor_fits)) {
    llk::ScheduleEntry se;
    const bool have_db = db_entry(nmat, M, &se);
    const TilePlan tp = tile_plan(nmat, M, KB, NB, have_db ? se.grain_size : 0);
    S = tp.S;
    head_cols = std::min<int64_t>(tp.head_nb * 128, N);
    ws_bytes = llk_tile_split_bytes(1, (int)M, (int)(NB - tp.head_nb), S, false);
    tile = true;
  } else if (!p.skinny && mode == 0 && accumulate && !p.pad && p.chunk >= M && p.head_nb == 0 &&
             fits(&llk_tile_rowmajor_fits)) {
    ws_bytes = llk_tile_split_bytes(0, (int)M, (int)NB, S, true);
    tile = true;
  } else {
    return LLK_OK;
  }
  int dev = -1;
  int rc = current_device(&dev);
  if (rc) return rc;
  void* ws = nullptr;
  Workspace* held = nullptr;
  if ((rc = get_workspace(dev, ws_bytes, ctx, &ws, &held))) return rc;
  *taken = true;
  hipStream_t s = stream_of(ctx);
  BindDone bind(held, s);
  const uint16_t* const xd = static_cast<const uint16_t*>(x->data);
  const uint16_t* const wgd = static_cast<const uint16_t*>(wg->data);
  const uint16_t* const wud = mode == 1 ? static_cast<const uint16_t*>(wu->data) : nullptr;
  hipError_t e = hipSuccess;
  if (tile) {
    // head columns unsplit, then the rest with the plan's splits (offsets of
    // 128-column multiples keep every row 16-byte aligned)
    const bool yv = y_vec_ok(y, out_dtype);
    const int64_t ldu = mode == 1 ? wu->stride0 : 0;
    if (head_cols > 0)
      e = llk_launch_tile_rowmajor(1, xd, x->stride0, wgd, wg->stride0, wud, ldu, y->data,
                                   y->stride0, (int)M, (int)head_cols, (int)K, 1, nullptr,
                                   out_dtype, yv, false, mod, s);
    if (e == hipSuccess && head_cols < N)
      e = llk_launch_tile_rowmajor(
          mode, xd, x->stride0, wgd + head_cols, wg->stride0,
          mode == 1 ? wud + head_cols : nullptr, ldu,
          static_cast<uint8_t*>(y->data) + head_cols * (int64_t)dtype_size(out_dtype), y->stride0,
          (int)M, (int)(N - head_cols), (int)K, S, ws, out_dtype, yv, accumulate, mod, s);
  } else {
    e = llk_launch_decode_rowmajor(mode, xd, x->stride0, wgd, wg->stride0, wud,
                                   mode == 1 ? wu->stride0 : 0, y->data, y->stride0, (int)M, (int)N,
                                   (int)K, S, ws, out_dtype, y_vec_ok(y, out_dtype), accumulate,
                                   mod, s);
  }
  bind.end();
  release_workspace(dev, held, s, bind.bound());
  return e == hipSuccess ? LLK_OK
                         : fail_hip(e, tile ? "tile kernel (row-major weights)"
                                            : "decode tile kernel (row-major weights)");
}

// The SwiGLU and GEMM entry points with the kernels of a loaded code object
// (code_object.cpp).
int swiglu_with_module(const llk_tensor2d* x, const llk_packed_weights* wg,
                       const llk_packed_weights* wu, llk_tensor2d* y, int y_dtype,
                       llk_kernel_context* ctx, const ModuleFns* mod) {
  return swiglu_entry(x, wg, wu, y, y_dtype, ctx, false, mod);
}
int gemm_with_module(const llk_tensor2d* a, const llk_packed_weights* b, llk_tensor2d* c,
                     int c_dtype, llk_kernel_context* ctx, const ModuleFns* mod,
                     bool accumulate) {
  return gemm_entry(a, b, c, c_dtype, ctx, mod, accumulate);
}
}  // namespace llk

extern "C" {

// ---------------------------------------------------------------------------
// Shape specialisation, tiling, keys, schedules
// ---------------------------------------------------------------------------

int llk_classify_m(int64_t M) { return llk::classifyM(M); }

int llk_set_tunable(const char* name, int64_t value) {
  if (!name || !llk::setTunable(name, value))
    return fail(LLK_ERR_INVALID_ARGUMENT, "unknown tunable %s", name ? name : "(null)");
  return LLK_OK;
}

int llk_get_tunable(const char* name, int64_t* value) {
  if (!name || !value) return fail(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  if (!llk::getTunable(name, value)) return fail(LLK_ERR_INVALID_ARGUMENT, "unknown tunable %s", name);
  return LLK_OK;
}

int64_t llk_num_tiles(int64_t dim, int64_t tile) {
  if (tile == 0) return 1;
  return (dim + tile - 1) / tile;
}
int64_t llk_tile_size(int64_t dim, int64_t tile, int64_t idx) {
  int64_t start = idx * tile;
  if (start >= dim) return 0;
  int64_t rem = dim - start;
  return rem < tile ? rem : tile;
}
int64_t llk_num_inner_tiles(int64_t outer, int64_t inner) {
  if (inner == 0) return 1;
  return (outer + inner - 1) / inner;
}

uint64_t llk_kernel_key_hash(uint8_t operation, uint8_t input_type, uint8_t output_type,
                             int64_t m_bucket, int64_t n, int64_t k, uint8_t weight_layout,
                             uint8_t isa, uint8_t math_mode, uint16_t thread_count,
                             uint64_t compiler_version, uint64_t schedule_version) {
  llk::KernelKey key;
  key.operation = static_cast<llk::OperationKind>(operation);
  key.input_type = static_cast<llk::DType>(input_type);
  key.output_type = static_cast<llk::DType>(output_type);
  key.M_bucket = m_bucket;
  key.N = n;
  key.K = k;
  key.weight_layout = static_cast<llk::Layout>(weight_layout);
  key.isa = static_cast<llk::Isa>(isa);
  key.math_mode = static_cast<llk::MathMode>(math_mode);
  key.thread_count = thread_count;
  key.compiler_version = compiler_version;
  key.schedule_version = schedule_version;
  return key.hash();
}

int llk_set_schedule_db(const char* path) {
  std::lock_guard<std::mutex> lk(g_db.mu);
  g_db.env_checked = true;
  g_db.sel.clear();
  if (!path || !*path) {
    g_db.path.clear();
    return LLK_OK;
  }
  bool ok = false;
  (void)llk::loadScheduleDB(path, 0, "fused_swiglu", &ok);
  if (!ok) {
    g_db.path.clear();
    return fail(LLK_ERR_NOT_FOUND, "cannot read or parse schedule DB %s", path);
  }
  g_db.path = path;
  return LLK_OK;
}

int llk_select_schedule(const char* db_path, const char* op_name, int m_bucket,
                        llk_schedule_entry* out, int* n_matches) {
  if (!db_path || !op_name || !out) return fail(LLK_ERR_INVALID_ARGUMENT, "NULL argument");
  bool ok = false;
  std::vector<llk::ScheduleEntry> m = llk::loadScheduleDB(db_path, m_bucket, op_name, &ok);
  llk::ScheduleEntry se = llk::selectBest(m);
  out->BM = se.BM;
  out->BN = se.BN;
  out->BK = se.BK;
  out->VM = se.VM;
  out->VN = se.VN;
  out->vector_width = se.vector_width;
  out->num_threads = se.num_threads;
  out->grain_size = se.grain_size;
  std::snprintf(out->parallel_axis, sizeof(out->parallel_axis), "%s", se.parallel_axis.c_str());
  if (n_matches) *n_matches = static_cast<int>(m.size());
  if (!ok) return fail(LLK_ERR_NOT_FOUND, "cannot read or parse schedule DB %s", db_path);
  return LLK_OK;
}

}  // extern "C"
