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

#include <hip/hip_runtime.h>

#include <string>

namespace llk {
// Functions of one loaded code object on one device (code_object.cpp).
struct ModuleFns;
// The function named `symbol`, or nullptr when the object has none.
hipFunction_t module_function(const ModuleFns* m, const char* symbol);
}  // namespace llk

namespace llk_gfx950 {

// Launches with the host stub `stub` when mod is null, else the function
// `symbol()` of the loaded object.  args are the kernel's parameters, by
// value, in order.  Returns the launch call's own status, so an error left
// by an unrelated earlier call on the thread is neither reported here nor
// cleared.
template <class... Args>
hipError_t launch_kernel(const llk::ModuleFns* mod, const void* stub, const char* (*symbol)(),
                         dim3 grid, dim3 block, unsigned lds, hipStream_t s, Args... args) {
  void* params[] = {static_cast<void*>(&args)...};
  if (!mod) return hipLaunchKernel(stub, grid, block, params, lds, s);
  hipFunction_t f = llk::module_function(mod, symbol());
  if (!f) return hipErrorNotFound;
  return hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, lds, s,
                               params, nullptr);
}

// Pieces of mangled names: a template argument of type int or bool.
inline std::string mangle_int(int v) { return "Li" + std::to_string(v) + "E"; }
inline std::string mangle_bool(bool v) { return v ? "Lb1E" : "Lb0E"; }

}  // namespace llk_gfx950
