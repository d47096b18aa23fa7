// tunables.cpp -- storage for the knobs declared in tunables.h.
#include "tunables.h"

#include <atomic>
#include <cstring>

namespace llk {
namespace {

struct Knob {
  const char* name;
  std::atomic<int64_t> value;
};

// decode_max_m:      largest M (<= 64) routed to the small-M bandwidth kernel.
// decode_splits:     force its cross-workgroup k-split count (0 = cost model).
// decode_target_wgs: workgroups per round in the small-M cost model (1 per CU).
// decode_min_kb:     fewest 64-k steps per split.
// decode_group_width: force the 32-column groups per small-M workgroup (1, 2
//                    or 4; 0 = cost model, 2 or 1); a forced width runs the
//                    small-M kernel of that width.
// decode_tile:       1 = M <= 64 with K a multiple of 64 and 16-byte aligned
//                    X rows runs on the decode tile kernel (LDS-DMA ring);
//                    0 = always the small-M kernel (and no mid-M form).
// midm_max_m:        largest M (<= 256) above 64 that runs on the decode
//                    tile kernel's 128- and 256-row forms (K a multiple of
//                    64, 16-byte aligned X rows) instead of the tile
//                    kernels; 64 or less = never.  128 by default: the
//                    256-row form re-reads 32 KiB of X per 64-k step beside
//                    16 KiB of weights and loses to the tile kernels (config
//                    5 MLP at M = 200 / 255: 146 / 156 us against 140 / 143).
// tile_splits:       force the tile kernel's k-split count (0 = cost model).
// tile_wgs_per_wave: workgroups the tile kernel runs at once (1 per CU).
// tile_min_kb:       fewest 64-k steps per tile-kernel split.
// tile_tail_split:   1 = the tile kernel may run the columns of its last,
//                    partial wave as a separate k-split launch; 0 = never.
// tile_wide:         fused SwiGLU with bf16 output: 1 = the cost model may
//                    take the wide tile kernel (16 B columns per matrix, B = 7
//                    or 11) where its whole waves beat the 128-column tile;
//                    0 = never; 7 or 11 = that width whenever it applies.
// kernel_fn_rowmajor: 1 = the KernelFn entries read device weights with
//                    aligned rows straight into the kernels' row-major forms
//                    (the decode tile kernel's up to 128 rows, the tile
//                    kernel's above: SwiGLU and the accumulating matmul);
//                    0 = they pack the weights on every call.
// max_workspaces:    library-owned workspaces kept per device (one per
//                    stream, or per thread on the per-thread default
//                    stream); beyond it the least recently used idle one is
//                    freed once its last call has finished.
Knob g_knobs[] = {
    {"decode_max_m", {64}},
    {"decode_splits", {0}},
    {"decode_target_wgs", {256}},
    {"decode_min_kb", {2}},
    {"decode_group_width", {0}},
    {"decode_tile", {1}},
    {"midm_max_m", {128}},
    {"tile_splits", {0}},
    {"tile_wgs_per_wave", {256}},
    {"tile_min_kb", {4}},
    {"tile_tail_split", {1}},
    {"tile_wide", {1}},
    {"kernel_fn_rowmajor", {1}},
    {"max_workspaces", {16}},
};

}  // namespace

int64_t tunable(const char* name) {
  for (auto& k : g_knobs)
    if (std::strcmp(k.name, name) == 0) return k.value.load(std::memory_order_relaxed);
  return 0;
}

bool setTunable(const char* name, int64_t value) {
  for (auto& k : g_knobs)
    if (std::strcmp(k.name, name) == 0) {
      k.value.store(value, std::memory_order_relaxed);
      return true;
    }
  return false;
}

bool getTunable(const char* name, int64_t* value) {
  for (auto& k : g_knobs)
    if (std::strcmp(k.name, name) == 0) {
      *value = k.value.load(std::memory_order_relaxed);
      return true;
    }
  return false;
}

}  // namespace llk
