// Chunked gated-DeltaNet scan: workspace layout and dispatch, and the f32
// (strict profile) kernels.  The algorithm is described in
// delta_scan_kernels.hpp; the f16 kernels are built in delta_scan_f16.hip.
#include "delta_scan_kernels.hpp"
#include "ragged.hpp"

namespace clef {

int scan_launch_f16(const ScanParams& p, hipStream_t stream);  // delta_scan_f16.hip

namespace {

int dk_pad(int dk) { return dk <= 32 ? 32 : dk <= 64 ? 64 : 128; }

// Workspace (every region 256-byte aligned; a block is 1 KiB):
//   Uf [chunks][Hv] x DK*64*ct bytes; Nf [chunks][Hv] x 64*64*ct;
//   sc [chunks][Hv] x 1 KiB; Ucf [Hv] x DK*64*ct;
//   ragged batches (nseq > 0): chunk_tab, seq_tab, the chunk count.  A batch
//   of nseq sequences and T tokens has at most T/64 + nseq chunks.
size_t carve(ScanParams* p, char* b, int T, int Hv, int dk, int precision, int nseq) {
  const size_t nchunks = (size_t)(T + kC - 1) / kC + (nseq > 0 ? nseq : 0);
  const size_t ct = precision == 0 ? 4 : 2;
  const size_t DK = dk_pad(dk);
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = b ? b + off : nullptr;
    off += al(bytes);
    return q;
  };
  char* Uf = take(nchunks * Hv * DK * kC * ct);
  char* Nf = take(nchunks * Hv * kC * kC * ct);
  char* sc = take(nchunks * Hv * 1024);
  char* Ucf = take((size_t)Hv * DK * kC * ct);
  char* ctab = nseq > 0 ? take(nchunks * sizeof(int2)) : nullptr;
  char* stab = nseq > 0 ? take((size_t)nseq * sizeof(int4)) : nullptr;
  char* ntot = nseq > 0 ? take(sizeof(int)) : nullptr;
  char* spans = nseq > 0 ? take(((size_t)nseq + 1) * sizeof(int)) : nullptr;
  if (p) {
    p->spans = reinterpret_cast<int*>(spans);
    p->chunk_tab = reinterpret_cast<int2*>(ctab);
    p->seq_tab = reinterpret_cast<int4*>(stab);
    p->nchunk_total = reinterpret_cast<int*>(ntot);
    p->Uf = Uf;
    p->Nf = Nf;
    p->sc = reinterpret_cast<float*>(sc);
    p->Ucf = Ucf;
  }
  return off;
}

}  // namespace

// Tables of a ragged batch from cu_seqlens (one work-group, ragged.hpp):
// the monotone spans (written to `spans` for the scan kernels), per sequence
// its chunk count and first chunk ranked by chunk count (most first), and
// per chunk its token span.  Any offset table keeps every access inside the
// T-token buffers and the chunk table inside its T/64 + nseq entries.
__global__ __launch_bounds__(kTabThreads) void scan_tables(const int* __restrict__ cu, int nseq, int T,
                                                           int* __restrict__ spans, int2* __restrict__ ctab,
                                                           int4* __restrict__ stab, int* __restrict__ ntot) {
  __shared__ int s_part[kTabThreads];
  __shared__ int s_R[kMaxRaggedSeq + 1];
  const int tid = threadIdx.x;
  const Ragged g{cu, nseq, T, s_part, s_R};
  rg_spans_1(g, tid);
  __syncthreads();
  rg_spans_2(g, tid);
  __syncthreads();
  rg_spans_3(g, tid);
  __syncthreads();
  for (int j = tid; j <= nseq; j += kTabThreads) spans[j] = s_R[j];
  rg_count_4(g, tid, kC);
  __syncthreads();
  rg_count_5(g, tid, ntot);
  __syncthreads();
  rg_scan_6(g, tid, kC, reinterpret_cast<int*>(ctab), reinterpret_cast<int*>(stab));
}

size_t scan_workspace_bytes(int T, int Hk, int Hv, int dk, int precision, int nseq) {
  return carve(nullptr, nullptr, T, Hv, dk, precision, nseq);
}

void scan_carve_workspace(ScanParams& p, void* ws, int precision) {
  carve(&p, static_cast<char*>(ws), p.T, p.Hv, p.dk, precision, p.cu_seqlens ? p.nseq : 0);
}

int scan_launch(const ScanParams& p0, int precision, hipStream_t stream) {
  ScanParams p = p0;
  if (p.cu_seqlens) {
    if (p.nseq < 1 || p.nseq > kMaxRaggedSeq) return fail(-1, "DeltaNet scan: 1..4096 sequences");
    hipLaunchKernelGGL(scan_tables, dim3(1), dim3(kTabThreads), 0, stream, p.cu_seqlens, p.nseq, p.T, p.spans,
                       p.chunk_tab, p.seq_tab, p.nchunk_total);
    if (int rc = check_launch("scan tables")) return rc;
    p.cu_seqlens = p.spans;  // the kernels read the monotone spans
  }
  if (precision == 0)
    return p.dtype_qkv == 0 ? launch_it<float, float>(p, stream) : launch_it<float, half_t>(p, stream);
  return scan_launch_f16(p, stream);
}

}  // namespace clef
