// Chunked gated-DeltaNet scan: workspace layout and dispatch, and the f32
// (strict profile) kernels.  The algorithm is described in
// delta_scan_kernels.hpp; the f16 kernels are built in delta_scan_f16.hip.
#include "delta_scan_kernels.hpp"

namespace clef {

int scan_launch_f16(const ScanParams& p, hipStream_t stream);  // delta_scan_f16.hip

namespace {

int dk_pad(int dk) { return dk <= 32 ? 32 : dk <= 64 ? 64 : 128; }

// Workspace (every region 256-byte aligned; a block is 1 KiB):
//   Kf, Qf [chunks][Hk] x 64*DK*ct bytes; Uf [chunks][Hv] x DK*64*ct;
//   Nf [chunks][Hv] x 64*64*ct; sc [chunks][Hv] x 1 KiB; Ucf [Hv] x DK*64*ct;
//   ragged batches (nseq > 0): chunk_tab, seq_tab, the chunk count.  A batch
//   of nseq sequences and T tokens has at most T/64 + nseq chunks.
size_t carve(ScanParams* p, char* b, int T, int Hk, int Hv, int dk, int precision, int nseq) {
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
  char* Kf = take(nchunks * Hk * kC * DK * ct);
  char* Qf = take(nchunks * Hk * kC * DK * ct);
  char* Uf = take(nchunks * Hv * DK * kC * ct);
  char* Nf = take(nchunks * Hv * kC * kC * ct);
  char* sc = take(nchunks * Hv * 1024);
  char* Ucf = take((size_t)Hv * DK * kC * ct);
  char* ctab = nseq > 0 ? take(nchunks * sizeof(int2)) : nullptr;
  char* stab = nseq > 0 ? take((size_t)nseq * sizeof(int4)) : nullptr;
  char* ntot = nseq > 0 ? take(sizeof(int)) : nullptr;
  if (p) {
    p->chunk_tab = reinterpret_cast<int2*>(ctab);
    p->seq_tab = reinterpret_cast<int4*>(stab);
    p->nchunk_total = reinterpret_cast<int*>(ntot);
    p->Kf = Kf;
    p->Qf = Qf;
    p->Uf = Uf;
    p->Nf = Nf;
    p->sc = reinterpret_cast<float*>(sc);
    p->Ucf = Ucf;
  }
  return off;
}

}  // namespace

// Tables of a ragged batch from cu_seqlens (one work-group): per sequence its
// chunk count and first chunk; sequences ranked by chunk count (descending,
// ties by index) so that the carry starts the longest first; per chunk its
// token span.  Offsets are clamped to [0, T], so any table keeps every access
// inside the T-token buffers.
__global__ __launch_bounds__(256) void scan_tables(const int* __restrict__ cu, int nseq, int T,
                                                   int2* __restrict__ ctab, int4* __restrict__ stab,
                                                   int* __restrict__ ntot) {
  __shared__ int s_sum[256];
  const int tid = threadIdx.x;
  const int per = (nseq + 255) / 256;  // consecutive sequences per thread
  const int s0 = min(tid * per, nseq), s1 = min(s0 + per, nseq);
  auto start = [&](int s) { return min(max(cu[s], 0), T); };
  auto length = [&](int s) { return max(min(max(cu[s + 1], 0), T) - start(s), 0); };
  auto chunks = [&](int s) { return (length(s) + kC - 1) / kC; };
  int sum = 0;
  for (int s = s0; s < s1; ++s) sum += chunks(s);
  s_sum[tid] = sum;
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int i = 0; i < 256; ++i) {
      const int v = s_sum[i];
      s_sum[i] = acc;
      acc += v;
    }
    *ntot = acc;
  }
  __syncthreads();
  int first = s_sum[tid];
  for (int s = s0; s < s1; ++s) {
    const int nc = chunks(s);
    int rank = 0;
    for (int j = 0; j < nseq; ++j) {
      const int nj = chunks(j);
      rank += (nj > nc) || (nj == nc && j < s);
    }
    stab[rank] = make_int4(s, first, nc, 0);
    const int t0 = start(s), len = length(s);
    for (int c = 0; c < nc; ++c) ctab[first + c] = make_int2(t0 + c * kC, min(kC, len - c * kC));
    first += nc;
  }
}

size_t scan_workspace_bytes(int T, int Hk, int Hv, int dk, int precision, int nseq) {
  return carve(nullptr, nullptr, T, Hk, Hv, dk, precision, nseq);
}

void scan_carve_workspace(ScanParams& p, void* ws, int precision) {
  carve(&p, static_cast<char*>(ws), p.T, p.Hk, p.Hv, p.dk, precision, p.cu_seqlens ? p.nseq : 0);
}

int scan_launch(const ScanParams& p, int precision, hipStream_t stream) {
  if (p.cu_seqlens) {
    hipLaunchKernelGGL(scan_tables, dim3(1), dim3(256), 0, stream, p.cu_seqlens, p.nseq, p.T, p.chunk_tab,
                       p.seq_tab, p.nchunk_total);
    if (int rc = check_launch("scan tables")) return rc;
  }
  if (precision == 0)
    return p.dtype_qkv == 0 ? launch_it<float, float>(p, stream) : launch_it<float, half_t>(p, stream);
  return scan_launch_f16(p, stream);
}

}  // namespace clef
