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
//   Nf [chunks][Hv] x 64*64*ct; sc [chunks][Hv] x 1 KiB; Ucf [Hv] x DK*64*ct.
size_t carve(ScanParams* p, char* b, int T, int Hk, int Hv, int dk, int precision) {
  const size_t nchunks = (size_t)(T + kC - 1) / kC;
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
  if (p) {
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

size_t scan_workspace_bytes(int T, int Hk, int Hv, int dk, int precision) {
  return carve(nullptr, nullptr, T, Hk, Hv, dk, precision);
}

void scan_carve_workspace(ScanParams& p, void* ws, int precision) {
  carve(&p, static_cast<char*>(ws), p.T, p.Hk, p.Hv, p.dk, precision);
}

int scan_launch(const ScanParams& p, int precision, hipStream_t stream) {
  if (precision == 0)
    return p.dtype_qkv == 0 ? launch_it<float, float>(p, stream) : launch_it<float, half_t>(p, stream);
  return scan_launch_f16(p, stream);
}

}  // namespace clef
