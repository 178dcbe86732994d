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
int gemm_f16_tile_shape(const GemmParams& p, int epilogue, int* bm);  // width 256, 192 or 128; rows 256 or 128

// a/b projections fused with the DeltaNet gates (gemm_f16.hip); f16 operands,
// Hv in {16, 32, 64}, K % 256 == 0, K <= 4096, rows 16-byte aligned (checked
// by the caller).  The weights are first packed into MFMA fragment order.
int ab_pack_f16_launch(const void* w_ab, int64_t ldw, int K, int Hv, void* packed, hipStream_t stream);
int ab_gates_f16_launch(const void* x, int64_t ldx, const void* packed, int K, const float* dt, const float* a_log,
                        float* g, float* beta, int T, int Hv, hipStream_t stream);

}  // namespace clef
