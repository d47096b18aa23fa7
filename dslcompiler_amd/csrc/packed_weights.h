// packed_weights.h -- the packed-weights handle behind the C ABI's opaque
// llk_packed_weights (PackedWeights.h:13-43 counterpart), shared by the
// sources of the library that build or read handles.  Not part of the C
// ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "llk/llk_abi.h"

namespace llk {
struct ModuleFns;  // functions of a loaded code object (code_object.cpp)
}

struct llk_packed_weights {
  // Reference metadata (PackedWeights.h:13-19).
  int64_t K_blocks = 0, N = 0, block_size = 0, BK = 0;
  int dtype = LLK_BF16;
  // Backend fields.
  int64_t K = 0;
  std::vector<uint16_t> host;  // reference layout, when kept
  void* dev = nullptr;
  size_t dev_bytes = 0;
  int device = -1;
  int64_t KB = 0, NB = 0;  // device layout blocks (64 k, 128 n)
  bool owns_dev = true;    // false: a view over device memory its creator owns
};

namespace llk {

// Packs bf16 W[K, N] into `dst` -- device memory on the current device of at
// least deviceLayoutBytes(K, N) bytes -- and points *view at it as a handle
// that does not own the memory (created on the first call with *view null,
// retargeted after that; llk_packed_weights_free deletes it and leaves dst
// alone).  W in device memory (w_on_device) is packed by the pack kernel of
// `mod` (null: the library's own) on stream s, asynchronously; W in host
// memory is packed on the host and copied, and the call returns when the
// copy is done.  Metadata as llk_pack_weights with BK = bk.
int pack_into(const llk_tensor2d* w, int64_t bk, bool w_on_device, void* dst, hipStream_t s,
              const ModuleFns* mod, llk_packed_weights** view);

}  // namespace llk
