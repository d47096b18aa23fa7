// launch.h -- how the host launchers start a kernel: through the library's
// own code object (the kernel's host stub) or through a gfx950 code object
// loaded at run time with hipModuleLoadData (code_object.cpp), where the
// same kernel is the function of the same symbol name.
//
// Symbol names are the kernels' Itanium-mangled names, written out by the
// launchers from the template arguments (e.g. mfma_tile_kernel<1, 0, true,
// false>(TileArgs) is _ZN10llk_gfx95016mfma_tile_kernelILi1ELi0ELb1ELb0EEEvNS_8TileArgsE):
// a name a loaded object does not define makes the launch fail with
// hipErrorNotFound, which the C ABI reports as a status.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace llk {
// Functions of one loaded code object on one device (code_object.cpp).
struct ModuleFns;
// The function named `symbol`, or nullptr when the object has none.
hipFunction_t module_function(const ModuleFns* m, const char* symbol);
}  // namespace llk

namespace llk_gfx950 {

// Completion event bound to this thread's launches while set (by a library
// call that holds a workspace, for the duration of its launches): each
// launch names it as the kernel's stop event (hipExtLaunchKernel /
// hipExtModuleLaunchKernel), so after the call it completes with the last
// of them.  Unlike hipEventRecord, which enqueues a marker packet of its own
// that the stream's next kernel waits behind (~6 us on MI355X), the event
// rides on the kernel's own dispatch.
inline thread_local hipEvent_t t_launch_done = nullptr;

// Launches with the host stub `stub` when mod is null, else the function
// `symbol()` of the loaded object.  args are the kernel's parameters, by
// value, in order.  Returns the launch call's own status, so an error left
// by an unrelated earlier call on the thread is neither reported here nor
// cleared.
template <class... Args>
hipError_t launch_kernel(const llk::ModuleFns* mod, const void* stub, const char* (*symbol)(),
                         dim3 grid, dim3 block, unsigned lds, hipStream_t s, Args... args) {
  void* params[] = {static_cast<void*>(&args)...};
  hipEvent_t done = t_launch_done;
  if (!mod)
    return done ? hipExtLaunchKernel(stub, grid, block, params, lds, s, nullptr, done, 0)
                : hipLaunchKernel(stub, grid, block, params, lds, s);
  hipFunction_t f = llk::module_function(mod, symbol());
  if (!f) return hipErrorNotFound;
  // hipExtModuleLaunchKernel takes the grid in work-items (32-bit)
  const uint64_t gx = (uint64_t)grid.x * block.x, gy = (uint64_t)grid.y * block.y,
                 gz = (uint64_t)grid.z * block.z;
  if (!done || gx > UINT32_MAX || gy > UINT32_MAX || gz > UINT32_MAX) {
    const hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y,
                                               block.z, lds, s, params, nullptr);
    return e == hipSuccess && done ? hipEventRecord(done, s) : e;
  }
  return hipExtModuleLaunchKernel(f, (uint32_t)gx, (uint32_t)gy, (uint32_t)gz, block.x, block.y,
                                  block.z, lds, s, params, nullptr, nullptr, done, 0);
}

// Pieces of mangled names: a template argument of type int or bool.
inline std::string mangle_int(int v) { return "Li" + std::to_string(v) + "E"; }
inline std::string mangle_bool(bool v) { return v ? "Lb1E" : "Lb0E"; }

}  // namespace llk_gfx950
