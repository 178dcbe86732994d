// C ABI: projection GEMM entry points (validation before any launch).
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/clef_hip.h"
#include "common.hpp"
#include "gemm.hpp"

static int gemm_checks(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* w2,
                       void* y, int64_t ldy, int M, int N, int K, int dtype_in, int dtype_out) {
  CLEF_REQUIRE(x && w && y, "GEMM: null operand");
  CLEF_REQUIRE(M >= 1 && N >= 1 && K >= 1 && M <= (1 << 24) && N <= (1 << 20) && K <= (1 << 20),
               "GEMM: dimensions out of range");
  CLEF_REQUIRE(dtype_in == CLEF_F32 || dtype_in == CLEF_F16, "GEMM: unsupported input dtype");
  CLEF_REQUIRE(dtype_out == CLEF_F32 || dtype_out == CLEF_F16, "GEMM: unsupported output dtype");
  CLEF_REQUIRE(ldx >= K && ldw >= K && ldy >= N, "GEMM: leading dimension smaller than the row");
  return 0;
}

static int vec_ok(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* w2, int K,
                  int dtype_in) {
  const int ve = dtype_in == CLEF_F16 ? 8 : 4;
  auto aligned = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  return K % ve == 0 && ldx % ve == 0 && ldw % ve == 0 && aligned(x) && aligned(w) && (!w2 || aligned(w2));
}

extern "C" int clef_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                         int64_t ldy, int M, int N, int K, int dtype_in, int dtype_out,
                         int epilogue, void* stream) {
  if (ldx == 0) ldx = K;
  if (ldw == 0) ldw = K;
  if (ldy == 0) ldy = N;
  if (int rc = gemm_checks(x, ldx, w, ldw, nullptr, y, ldy, M, N, K, dtype_in, dtype_out)) return rc;
  CLEF_REQUIRE(epilogue == CLEF_EPI_STORE || epilogue == CLEF_EPI_RESIDUAL, "GEMM: unknown epilogue");
  clef::GemmParams p{x, w, nullptr, y, ldx, ldw, ldy, M, N, K, dtype_in, dtype_out,
                     vec_ok(x, ldx, w, ldw, nullptr, K, dtype_in)};
  return clef::gemm_launch(p, epilogue, static_cast<hipStream_t>(stream));
}

extern "C" int clef_gemm_swiglu(const void* x, int64_t ldx, const void* wg, const void* wu,
                                int64_t ldw, void* y, int64_t ldy, int M, int N, int K, int dtype,
                                void* stream) {
  if (ldx == 0) ldx = K;
  if (ldw == 0) ldw = K;
  if (ldy == 0) ldy = N;
  CLEF_REQUIRE(wu != nullptr, "GEMM: null up weights");
  if (int rc = gemm_checks(x, ldx, wg, ldw, wu, y, ldy, M, N, K, dtype, dtype)) return rc;
  clef::GemmParams p{x, wg, wu, y, ldx, ldw, ldy, M, N, K, dtype, dtype, vec_ok(x, ldx, wg, ldw, wu, K, dtype)};
  return clef::gemm_launch(p, 2, static_cast<hipStream_t>(stream));
}

static int gates_proj_dims(int K, int Hv) {
  CLEF_REQUIRE(K >= 256 && K % 256 == 0 && K <= 4096 && (Hv == 16 || Hv == 32 || Hv == 64),
               "gates projection: K must be a multiple of 256 up to 4096 and Hv 16, 32 or 64");
  return 0;
}

extern "C" size_t clef_delta_gates_pack_bytes(int K, int Hv) {
  if (gates_proj_dims(K, Hv)) return 0;
  return (size_t)K * 2 * Hv * 2;
}

extern "C" int clef_delta_gates_pack(const void* w_ab, int64_t ldw, int K, int Hv, int dtype, void* packed,
                                     void* stream) {
  if (ldw == 0) ldw = K;
  CLEF_REQUIRE(w_ab && packed, "gates projection: null pointer");
  CLEF_REQUIRE(dtype == CLEF_F16, "gates projection: f16 operands only");
  if (int rc = gates_proj_dims(K, Hv)) return rc;
  CLEF_REQUIRE(ldw >= K && vec_ok(w_ab, ldw, w_ab, ldw, nullptr, K, dtype) &&
                   (reinterpret_cast<uintptr_t>(packed) & 15) == 0,
               "gates projection: rows must be 16-byte aligned");
  return clef::ab_pack_f16_launch(w_ab, ldw, K, Hv, packed, static_cast<hipStream_t>(stream));
}

extern "C" int clef_delta_gates_proj(const void* x, int64_t ldx, const void* packed, int K, int dtype,
                                     const float* dt, const float* a_log, float* g, float* beta, int T, int Hv,
                                     void* stream) {
  if (ldx == 0) ldx = K;
  CLEF_REQUIRE(x && packed && dt && a_log && g && beta, "gates projection: null pointer");
  CLEF_REQUIRE(dtype == CLEF_F16, "gates projection: f16 operands only");
  if (int rc = gates_proj_dims(K, Hv)) return rc;
  CLEF_REQUIRE(T >= 1 && T <= (1 << 24) && ldx >= K, "gates projection: dimensions");
  CLEF_REQUIRE(vec_ok(x, ldx, x, ldx, nullptr, K, dtype) && (reinterpret_cast<uintptr_t>(packed) & 15) == 0,
               "gates projection: rows must be 16-byte aligned");
  return clef::ab_gates_f16_launch(x, ldx, packed, K, dt, a_log, g, beta, T, Hv, static_cast<hipStream_t>(stream));
}
