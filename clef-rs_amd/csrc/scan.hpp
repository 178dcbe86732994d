// Internal launch interface of the chunked gated-DeltaNet scan.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace clef {

struct ScanParams {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  int64_t sqk, sv, sgb, so;  // token strides (elements)
  int dtype_qkv, dtype_gb, dtype_out;
  int T, Hk, Hv, dk, dv, nchunks;
  int vec_qk;    // q/k rows may be read as 16-byte vectors
  float qscale;  // 1/sqrt(dk) rounded to f32
  const float* initial;
  int capture;
  void* out;
  float* captured;
  float* final_state;
  // workspace views
  void* Tm;      // [nchunks][Hv][64][64] compute dtype: (I + A)^-1
  void* Mm;      // [nchunks][Hv][64][64] compute dtype: masked decayed Q K^T
  void* Kt;      // [nchunks][Hk][DK][64] compute dtype: normalised K^T
  float* eg;     // [nchunks][Hv][64]   exp(gam_r)
  float* wl;     // [nchunks][Hv][64]   exp(gam_last - gam_r)
  float* bt;     // [nchunks][Hv][64]   beta
  float* gam_ws; // [nchunks][Hv][64]   in-chunk cumulative log-decay
  float* invk;   // [nchunks][Hk][64]   1/|k| (0 on padding rows)
  float* scq;    // [nchunks][Hk][64]   qscale/|q| (0 on padding rows)
};

size_t scan_workspace_bytes(int T, int Hk, int Hv, int dk, int precision);
void scan_carve_workspace(ScanParams& p, void* ws, int precision);
int scan_launch(const ScanParams& p, int precision, hipStream_t stream);

}  // namespace clef
