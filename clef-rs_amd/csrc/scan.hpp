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
  void* Uf;   // [chunks][Hv][state tiles x token blocks]  U = K^T W (I+A)^-1 diag(beta)
  void* Nf;   // [chunks][Hv][4 x token blocks]            N = M (I+A)^-1 diag(beta)
  void* Ucf;  // [Hv][state tiles x token blocks]  U weighted for the capture token
  float* sc;  // [chunks][Hv][4][64]  e^gam/|k| and qscale e^gam/|q| (0 past the chunk's tokens), gam, e^gam
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
};

// nseq > 1 (or a cu_seqlens table) sizes for a ragged batch of T tokens
size_t scan_workspace_bytes(int T, int Hk, int Hv, int dk, int precision, int nseq = 0);
void scan_carve_workspace(ScanParams& p, void* ws, int precision);
int scan_launch(const ScanParams& p, int precision, hipStream_t stream);

}  // namespace clef
