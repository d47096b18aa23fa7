// Exports llk::KernelKey::hash / toString / sizeof from the reference's own
// header (include/LLK/Runtime/KernelKey.h, header-only, no MLIR), compiled
// where it lies.  Test infrastructure (oracle/_ref only).
#include "LLK/Runtime/KernelKey.h"

#include <cstring>

extern "C" {
uint64_t ref_kernel_key_hash(uint8_t op, uint8_t in_t, uint8_t out_t,
                             int64_t m_bucket, int64_t n, int64_t k,
                             uint8_t layout, uint8_t isa, uint8_t math,
                             uint16_t threads, uint64_t compiler_version,
                             uint64_t schedule_version) {
  llk::KernelKey key{};
  key.operation = static_cast<llk::OperationKind>(op);
  key.input_type = static_cast<llk::DType>(in_t);
  key.output_type = static_cast<llk::DType>(out_t);
  key.M_bucket = m_bucket;
  key.N = n;
  key.K = k;
  key.weight_layout = static_cast<llk::Layout>(layout);
  key.isa = static_cast<llk::CpuIsa>(isa);
  key.math_mode = static_cast<llk::MathMode>(math);
  key.thread_count = threads;
  key.compiler_version = compiler_version;
  key.schedule_version = schedule_version;
  return key.hash();
}
// Default-constructed key's hash (all member initialisers).
uint64_t ref_kernel_key_default_hash(void) {
  llk::KernelKey key{};
  return key.hash();
}
int ref_kernel_key_sizeof(void) { return static_cast<int>(sizeof(llk::KernelKey)); }
int ref_kernel_key_to_string(uint64_t m_bucket, int64_t n, int64_t k, char* buf,
                             int cap) {
  llk::KernelKey key{};
  key.M_bucket = static_cast<int64_t>(m_bucket);
  key.N = n;
  key.K = k;
  std::string s = key.toString();
  std::strncpy(buf, s.c_str(), cap - 1);
  buf[cap - 1] = 0;
  return static_cast<int>(s.size());
}
}
