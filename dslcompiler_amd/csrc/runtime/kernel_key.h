// kernel_key.h -- KernelKey / WeightKey for the gfx950 backend.
//
// Field set, order, enum values and hash follow the reference's
// include/LLK/Runtime/KernelKey.h:20-142, so a key hashes to the same value
// in both: twelve fields fed in declaration order through the splitmix64
// finaliser with seed 0x9ae16a3b2f90404f (KernelKey.h:60-86).  The ISA enum
// gains GFX950 = 7 after UNKNOWN = 6, so every existing value keeps its hash.
#pragma once

#include <cstdint>
#include <cstring>
#include <sstream>
#include <string>

namespace llk {

enum class DType : uint8_t { BF16 = 0, FP16 = 1, FP32 = 2 };

enum class Isa : uint8_t {
  AVX2 = 0,
  AVX512_BF16 = 1,
  AVX512_VNNI = 2,
  AMX_BF16 = 3,
  NEON = 4,
  SVE = 5,
  UNKNOWN = 6,
  GFX950 = 7,  // MI355X (CDNA4)
};

// FusedSwiGLU/RoPE/Attention keep the reference values; Matmul is the
// micro.mma GEMM of this backend.
enum class OperationKind : uint8_t { FusedSwiGLU = 0, RoPE = 1, Attention = 2, Matmul = 3 };

// RowMajor/PackedKN as in the reference; PackedMfma32 is the device payload
// layout of this backend (1 KiB v_mfma_f32_32x32x16_bf16 operand blocks).
enum class Layout : uint8_t { RowMajor = 0, PackedKN = 1, PackedMfma32 = 2 };

enum class MathMode : uint8_t { Strict = 0, BoundedFast = 1, UnsafeFast = 2 };

inline uint64_t key_mix(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
  return x ^ (x >> 31);
}

struct KernelKey {
  OperationKind operation{OperationKind::FusedSwiGLU};
  DType input_type{DType::BF16};
  DType output_type{DType::BF16};
  int64_t M_bucket{0};
  int64_t N{0};
  int64_t K{0};
  Layout weight_layout{Layout::RowMajor};
  Isa isa{Isa::AVX2};
  MathMode math_mode{MathMode::BoundedFast};
  uint16_t thread_count{1};
  uint64_t compiler_version{0};
  uint64_t schedule_version{0};

  uint64_t hash() const {
    uint64_t h = 0x9ae16a3b2f90404fULL;
    const uint64_t f[12] = {static_cast<uint8_t>(operation),
                            static_cast<uint8_t>(input_type),
                            static_cast<uint8_t>(output_type),
                            static_cast<uint64_t>(M_bucket),
                            static_cast<uint64_t>(N),
                            static_cast<uint64_t>(K),
                            static_cast<uint8_t>(weight_layout),
                            static_cast<uint8_t>(isa),
                            static_cast<uint8_t>(math_mode),
                            static_cast<uint64_t>(thread_count),
                            compiler_version,
                            schedule_version};
    for (uint64_t v : f) h = key_mix(h ^ v);
    return h;
  }

  std::string toString() const {
    std::ostringstream o;
    o << "KernelKey{op=" << static_cast<int>(operation)
      << " dtype_in=" << static_cast<int>(input_type)
      << " dtype_out=" << static_cast<int>(output_type) << " M_bucket=" << M_bucket
      << " N=" << N << " K=" << K << " layout=" << static_cast<int>(weight_layout)
      << " isa=" << static_cast<int>(isa) << " math=" << static_cast<int>(math_mode)
      << " threads=" << thread_count << " compiler=" << compiler_version
      << " schedule=" << schedule_version << "}";
    return o.str();
  }

  // Field-wise equality (the reference compares raw bytes, padding
  // included, which requires value-initialised keys; comparing fields
  // avoids that trap and agrees with it on value-initialised keys).
  bool operator==(const KernelKey& o) const {
    return operation == o.operation && input_type == o.input_type &&
           output_type == o.output_type && M_bucket == o.M_bucket && N == o.N && K == o.K &&
           weight_layout == o.weight_layout && isa == o.isa && math_mode == o.math_mode &&
           thread_count == o.thread_count && compiler_version == o.compiler_version &&
           schedule_version == o.schedule_version;
  }
  bool operator!=(const KernelKey& o) const { return !(*this == o); }

  // 48-byte binary key of the object-code level (JitCache.cpp:94-114):
  // op@0 dtype_in@1 dtype_out@2 M_bucket@3 N@11 K@19 layout@27 isa@28
  // math@29 threads@30 compiler@32 schedule@40, little-endian.
  std::string serialize() const {
    std::string s(48, '\0');
    char* p = &s[0];
    p[0] = static_cast<char>(operation);
    p[1] = static_cast<char>(input_type);
    p[2] = static_cast<char>(output_type);
    std::memcpy(p + 3, &M_bucket, 8);
    std::memcpy(p + 11, &N, 8);
    std::memcpy(p + 19, &K, 8);
    p[27] = static_cast<char>(weight_layout);
    p[28] = static_cast<char>(isa);
    p[29] = static_cast<char>(math_mode);
    std::memcpy(p + 30, &thread_count, 2);
    std::memcpy(p + 32, &compiler_version, 8);
    std::memcpy(p + 40, &schedule_version, 8);
    return s;
  }
};

// WeightKey (KernelKey.h:114-124): identifies a packed-weight buffer.
struct WeightKey {
  const void* weight_ptr{nullptr};
  uint64_t shape_hash{0};
  int64_t BK{0};
  int64_t BN{0};
  bool operator==(const WeightKey& o) const {
    return weight_ptr == o.weight_ptr && shape_hash == o.shape_hash && BK == o.BK && BN == o.BN;
  }
  // 32-byte binary key of the weight level (JitCache.cpp:117-126):
  // ptr@0 shape_hash@8 BK@16 BN@24.
  std::string serialize() const {
    std::string s(32, '\0');
    uint64_t p = reinterpret_cast<uintptr_t>(weight_ptr);
    std::memcpy(&s[0], &p, 8);
    std::memcpy(&s[8], &shape_hash, 8);
    std::memcpy(&s[16], &BK, 8);
    std::memcpy(&s[24], &BN, 8);
    return s;
  }
};

}  // namespace llk
