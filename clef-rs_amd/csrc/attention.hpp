// Internal launch interface of the gated causal attention core.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace clef {

struct AttnParams {
  const void* q;     // [heads][ldq][d]
  const void* k;     // [kvh][ldk][d]
  const void* vt;    // [kvh][d][ldv]  (values transposed: keys contiguous)
  const void* gate;  // gate of (token, head, e) at token * ldg + head * hsg + e
  void* y;           // [qn][ldy], head h at columns h * d ..
  int64_t ldq, ldk, ldv, ldg, hsg, ldy;
  int heads, kvh, qn, kn, d;
  float scale;
  // Ragged batch (cu_q non-null; qn = packed tokens T, kn unused): sequence s
  // owns rows cu_q[s] .. cu_q[s+1]-1 of q, k, vt, gate and y, and its queries
  // see the np prefix keys (pk, pvt; all visible) before its own, causally.
  const int* cu_q;   // [nseq + 1] (device)
  int2* pairs;       // [blocks / heads] {sequence, query tile}, most keys first
  int* npairs;       // valid entries of pairs
  int* spans;        // [nseq + 1] cu_q made monotone in [0, T] (ragged.hpp)
  int nseq;
  const void* pk;    // [kvh][ldpk][d] or null
  const void* pvt;   // [kvh][d][ldpv]
  int64_t ldpk, ldpv;
  int np;
  int vec_io;        // set at launch: gate and y rows allow 8-byte accesses
  // Fused query preparation (single sequences, f16, d = 256, rotary on 64
  // features; null q-raw: q holds prepared rows).  Row t of head h is read
  // at qraw + t * ldqr + h * hsr, RMS-normalised with weights qw (eps qeps,
  // 1/d = qinv) and rotated by qrot[t] ([qn][32] (cos, sin) pairs), with the
  // roundings of the per-token q/k norm + rotary kernel.
  const void* qraw = nullptr;
  int64_t ldqr = 0, hsr = 0;
  const float* qw = nullptr;
  const float2* qrot = nullptr;
  float qeps = 0.0f, qinv = 0.0f;
};

// whether attn_f16_launch takes the fused query path for p (f16 data)
bool attn_qfuse_ok(const AttnParams& p);

// device tables of a ragged batch (workspace: attn_tables_bytes)
size_t attn_tables_bytes(int T, int nseq);
void attn_carve_tables(AttnParams& p, void* ws);
int attn_f16_tables(AttnParams& p, hipStream_t s);

// f16 flash-attention path (MFMA 32x32x16, LDS-DMA key/value tiles); false if
// the shape is outside what it handles, in which case nothing is launched.
bool attn_f16_ok(const AttnParams& p);
int attn_f16_launch(const AttnParams& p, hipStream_t s);

}  // namespace clef
