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

// decode_max_m:      largest M routed to the split-K decode kernel.
// decode_splits:     force the decode k-split count (0 = heuristic).
// decode_target_wgs: workgroups the decode heuristic aims for.
// decode_min_kb:     fewest 64-k steps per decode split.
// tile_load:         force the tile kernel's operand path (-1 = automatic,
//                    0 = direct-to-LDS, 1 = staged 16-byte, 2 = staged scalar).
Knob g_knobs[] = {
    {"tile_load", {-1}},
    {"decode_max_m", {64}},
    {"decode_splits", {0}},
    {"decode_target_wgs", {1536}},
    {"decode_min_kb", {2}},
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

}  // namespace llk
