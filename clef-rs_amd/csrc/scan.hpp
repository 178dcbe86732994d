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
  // Workspace views.  A "block" is one MFMA operand fragment of a 64-lane
  // wave: 64 x 16 bytes, lane-major, in the compute dtype.
  void* Kf;   // [chunks][Hk][4 x dk-blocks]  normalised keys  (rows of X = K^ S)
  void* Qf;   // [chunks][Hk][4 x dk-blocks]  scaled normalised queries
  void* Uf;   // [chunks][Hv][state tiles x token blocks]  U = K^T W (I+A)^-1 diag(beta)
  void* Nf;   // [chunks][Hv][4 x token blocks]            N = M (I+A)^-1 diag(beta)
  void* Ucf;  // [Hv][state tiles x token blocks]  U weighted for the capture token
  float* sc;  // [chunks][Hv][4][64]  beta, exp(gam), gam, 0
  // Ragged batches (packed sequences, cu_seqlens): chunks never cross a
  // sequence.  Tables built on the device by scan_tables; all null for one
  // sequence (chunk c then spans tokens 64 c .. min(64 c + 64, T)).
  const int* cu_seqlens;  // [nseq + 1] token offsets (device)
  int* spans;             // [nseq + 1] the offsets made monotone in [0, T] (ragged.hpp)
  int2* chunk_tab;        // [chunks] {first token, tokens}
  int4* seq_tab;          // [nseq] {sequence, first chunk, chunks, 0}, most chunks first
  int* nchunk_total;      // valid entries of chunk_tab
  int nseq;
  int64_t init_stride;    // floats between consecutive sequences' initial states (0: shared)
  // Conv prologue (qwen.rs:609-618, 765-796, 4 taps): when `mixed` is set, q,
  // k and v are the raw projection columns [q | k | v] of `mixed` (token
  // stride ld_mixed, dtype_qkv); scan_prepare applies the causal conv + SiLU
  // (rounded to dtype_qkv, as the separate conv kernel stores it), and writes
  // the convolved v to `v` (token stride sv) for the carry.  Rows before a
  // sequence's first token come from its f32 history (hist_rows rows of
  // conv_channels, sequence s at conv_hist + s * hist_stride), else zero.
  const void* mixed;
  int64_t ld_mixed;
  const float* conv_w;     // [conv_channels][4]
  const float* conv_hist;
  int hist_rows;
  int64_t hist_stride;
  int conv_channels;       // 2 Hk dk + Hv dv
};

// nseq > 1 (or a cu_seqlens table) sizes for a ragged batch of T tokens
size_t scan_workspace_bytes(int T, int Hk, int Hv, int dk, int precision, int nseq = 0);
void scan_carve_workspace(ScanParams& p, void* ws, int precision);
int scan_launch(const ScanParams& p, int precision, hipStream_t stream);

}  // namespace clef
