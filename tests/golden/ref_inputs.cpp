// Reproduces the input streams of the reference's own SwiGLU tests:
// std::mt19937(42) + std::normal_distribution<float>(0, 1) from libstdc++
// (the library the reference tests build against on Linux), drawn in the
// order the tests draw them, and the tests' own f32->bf16 helper
// (bits + 0x8000 + lsb, swiglu_vector_avx2.cpp:80-86).
//
//   ref_inputs vec  M N K   -> swiglu_vector_avx2.cpp:248-270 / swiglu_scalar.cpp:386-407
//                              (x: M*K normals; then for each of K*N: vg, vu)
//                              writes bf16 bits x, wg, wu (uint16, row-major)
//   ref_inputs ref  M N K   -> swiglu_reference.cpp:116-131
//                              (x: M*K normals; then for each of K*N: wg, wu)
//                              writes float32 x, wg, wu
// Output: raw little-endian arrays to stdout, in the order x, wg, wu.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

static uint16_t test_f32_to_bf16(float f) {
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  bits += 0x8000u + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}

int main(int argc, char** argv) {
  if (argc != 5) return 2;
  const std::string mode = argv[1];
  const long M = std::atol(argv[2]), N = std::atol(argv[3]), K = std::atol(argv[4]);
  std::mt19937 rng(42);
  std::normal_distribution<float> dist(0.0f, 1.0f);
  if (mode == "vec") {
    std::vector<uint16_t> x(M * K), wg(K * N), wu(K * N);
    for (auto& v : x) v = test_f32_to_bf16(dist(rng));
    for (long i = 0; i < K * N; ++i) {
      float vg = dist(rng), vu = dist(rng);
      wg[i] = test_f32_to_bf16(vg);
      wu[i] = test_f32_to_bf16(vu);
    }
    fwrite(x.data(), 2, x.size(), stdout);
    fwrite(wg.data(), 2, wg.size(), stdout);
    fwrite(wu.data(), 2, wu.size(), stdout);
  } else if (mode == "ref") {
    std::vector<float> x(M * K), wg(K * N), wu(K * N);
    for (auto& v : x) v = dist(rng);
    for (long i = 0; i < K * N; ++i) {
      wg[i] = dist(rng);
      wu[i] = dist(rng);
    }
    fwrite(x.data(), 4, x.size(), stdout);
    fwrite(wg.data(), 4, wg.size(), stdout);
    fwrite(wu.data(), 4, wu.size(), stdout);
  } else {
    return 2;
  }
  return 0;
}
