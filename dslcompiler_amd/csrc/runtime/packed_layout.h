// packed_layout.h -- host-side packers for weight matrices.
#pragma once

#include <cstddef>
#include <cstdint>

namespace llk {

// Reference host layout (PackedWeights.cpp:5-33): [K_blocks][BK][N] bf16,
// zero-padded, rows copied from w + k*stride0.  `out` holds
// ceil(K/BK)*BK*N elements.
void packReferenceLayout(const uint16_t* w, int64_t K, int64_t N, int64_t stride0, int64_t BK,
                         uint16_t* out);

// Device payload layout (MFMA operand order, 128 n x 64 k blocks of 16 KiB,
// 1 KiB sub-blocks of 32 n x 16 k in v_mfma_f32_32x32x16_bf16 lane order).
int64_t deviceBlocksN(int64_t N);  // ceil(N / 128)
int64_t deviceBlocksK(int64_t K);  // ceil(K / 64)
size_t deviceLayoutBytes(int64_t K, int64_t N);
void packDeviceLayout(const uint16_t* w, int64_t K, int64_t N, int64_t stride0, uint8_t* out);
// Inverse of packDeviceLayout: writes W [K, N] (row stride stride0).
void unpackDeviceLayout(const uint8_t* in, int64_t K, int64_t N, uint16_t* w, int64_t stride0);

}  // namespace llk
