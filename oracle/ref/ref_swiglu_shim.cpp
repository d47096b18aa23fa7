// Exports the reference's own SwiGLU test routines, compiled from the
// reference tree where it lies (the include path points at /root/reference).
// Test infrastructure: builds into oracle/_ref only.
//
// test/Execution/swiglu_reference.cpp:19-32  bf16 helpers
// test/Execution/swiglu_reference.cpp:38-70  fp32 naive SwiGLU
// test/Execution/swiglu_reference.cpp:77-99  fp64 SwiGLU
#include "test/Execution/swiglu_reference.cpp"

extern "C" {
void ref_swiglu_fp32(const float* x, const float* wg, const float* wu, float* y,
                     int64_t M, int64_t N, int64_t K) {
  swiglu_reference(x, wg, wu, y, M, N, K);
}
void ref_swiglu_fp64(const double* x, const double* wg, const double* wu,
                     double* y, int64_t M, int64_t N, int64_t K) {
  swiglu_reference_fp64(x, wg, wu, y, M, N, K);
}
uint16_t ref_f32_to_bf16(float f) { return f32_to_bf16(f); }
float ref_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
}
