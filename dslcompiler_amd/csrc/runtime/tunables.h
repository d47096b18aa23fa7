// tunables.h -- named integer knobs of the gfx950 dispatch heuristics
// (decode/prefill crossover, split-K factors).  Defaults are the values
// measured best on MI355X; llk_set_tunable() overrides them at run time.
#pragma once

#include <cstdint>

namespace llk {

// Returns the current value of a knob (0 for an unknown name).
int64_t tunable(const char* name);
// Sets a knob; returns false for an unknown name.
bool setTunable(const char* name, int64_t value);
// Reads a knob into *value; returns false for an unknown name.
bool getTunable(const char* name, int64_t* value);

}  // namespace llk
