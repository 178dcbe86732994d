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
