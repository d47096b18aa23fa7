// Exports the fp64 routine of the reference's edge-case test, compiled from
// the reference tree where it lies.  Test infrastructure (oracle/_ref only).
// test/Execution/edge_cases.cpp:18-40
#include "test/Execution/edge_cases.cpp"

extern "C" void ref_edge_swiglu_fp64(const double* x, const double* wg,
                                     const double* wu, double* y, int64_t M,
                                     int64_t N, int64_t K) {
  swiglu_reference_fp64(x, wg, wu, y, M, N, K);
}
