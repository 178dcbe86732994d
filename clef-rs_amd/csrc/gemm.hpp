// Internal launch interface of the projection GEMMs.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace clef {

struct GemmParams {
  const void* x;   // [M, K], row stride ldx
  const void* w;   // [N, K], row stride ldw (gate weights for SwiGLU)
  const void* w2;  // [N, K] up weights (SwiGLU only)
  void* y;         // [M, N], row stride ldy
  int64_t ldx, ldw, ldy;
  int M, N, K;
  int dtype_in, dtype_out;
  int vec;  // rows 16-byte aligned and K a multiple of 16 bytes
};

// epilogue: 0 store, 1 residual add into f32 y, 2 SwiGLU
int gemm_launch(const GemmParams& p, int epilogue, hipStream_t stream);

// f16 large-M path (gemm_f16.hip)
bool gemm_f16_dma_ok(const GemmParams& p);
int gemm_f16_dma_launch(const GemmParams& p, int epilogue, hipStream_t stream);

}  // namespace clef
