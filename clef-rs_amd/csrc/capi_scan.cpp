// C ABI: error plumbing and the gated-DeltaNet scan entry points.
// Validation happens here, before any launch (metal.rs:280-290, 303-307).
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/clef_hip.h"
#include "common.hpp"
#include "ragged.hpp"
#include "scan.hpp"

namespace clef {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(static_cast<int>(e), std::string(what) + ": " + hipGetErrorString(e));
  return 0;
}

}  // namespace clef

using clef::fail;

extern "C" const char* clef_hip_last_error(void) { return clef::g_last_error.c_str(); }

extern "C" int clef_hip_abi_version(void) { return 2; }

static bool valid_dtype(int d) { return d == CLEF_F32 || d == CLEF_F16; }

static int scan_dims(int T, int Hk, int Hv, int dk, int dv, int chunk, int precision) {
  CLEF_REQUIRE(T >= 1 && T <= (1 << 20), "DeltaNet scan: tokens must be in 1..1048576");
  CLEF_REQUIRE(Hk >= 1 && Hv >= Hk && Hv <= 256 && Hv % Hk == 0,
               "DeltaNet scan: heads must satisfy 1 <= Hk <= Hv <= 256, Hv % Hk == 0");
  CLEF_REQUIRE(dk >= 1 && dk <= 128 && dv >= 1 && dv <= 128,
               "DeltaNet scan: key and value widths must be in 1..128");
  CLEF_REQUIRE(chunk == 64, "DeltaNet scan: chunk must be 64");
  CLEF_REQUIRE(precision == CLEF_SCAN_STRICT || precision == CLEF_SCAN_MIXED,
               "DeltaNet scan: unknown precision profile");
  return 0;
}

extern "C" size_t clef_delta_scan_workspace(int T, int Hk, int Hv, int dk, int dv, int chunk,
                                            int precision) {
  if (scan_dims(T, Hk, Hv, dk, dv, chunk, precision)) return 0;
  return clef::scan_workspace_bytes(T, Hk, Hv, dk, precision);
}

// shared validation and parameter set-up of both scan entry points
static int scan_params(clef::ScanParams& p, const void* q, const void* k, const void* v, int64_t sqk, int64_t sv,
                       int dtype_qkv, const void* g, const void* beta, int64_t sgb, int dtype_gb, int T, int Hk,
                       int Hv, int dk, int dv, int chunk, int precision, void* out, int64_t so, int dtype_out,
                       void* workspace, size_t workspace_bytes, int nseq) {
  if (int rc = scan_dims(T, Hk, Hv, dk, dv, chunk, precision)) return rc;
  CLEF_REQUIRE(q && k && v && g && beta && out, "DeltaNet scan: null input or output");
  CLEF_REQUIRE(valid_dtype(dtype_qkv) && valid_dtype(dtype_gb) && valid_dtype(dtype_out),
               "DeltaNet scan: unsupported dtype");
  if (sqk == 0) sqk = static_cast<int64_t>(Hk) * dk;
  if (sv == 0) sv = static_cast<int64_t>(Hv) * dv;
  if (sgb == 0) sgb = Hv;
  if (so == 0) so = static_cast<int64_t>(Hv) * dv;
  CLEF_REQUIRE(sqk >= static_cast<int64_t>(Hk) * dk && sv >= static_cast<int64_t>(Hv) * dv &&
                   sgb >= Hv && so >= static_cast<int64_t>(Hv) * dv,
               "DeltaNet scan: token stride smaller than a token row");
  // a chunk's rows of v and out are addressed with 32-bit byte offsets
  CLEF_REQUIRE(sv < (int64_t(1) << 22) && so < (int64_t(1) << 22),
               "DeltaNet scan: token stride of v or out above 2^22 elements");
  const size_t need = clef::scan_workspace_bytes(T, Hk, Hv, dk, precision, nseq);
  CLEF_REQUIRE(workspace && workspace_bytes >= need, "DeltaNet scan: workspace too small");
  CLEF_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
               "DeltaNet scan: workspace must be 256-byte aligned");
  p = clef::ScanParams{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta;
  p.sqk = sqk; p.sv = sv; p.sgb = sgb; p.so = so;
  p.dtype_qkv = dtype_qkv; p.dtype_gb = dtype_gb; p.dtype_out = dtype_out;
  p.T = T; p.Hk = Hk; p.Hv = Hv; p.dk = dk; p.dv = dv;
  p.nchunks = (T + 63) / 64 + nseq;  // ragged: the most chunks nseq sequences of T tokens can have
  const int vi = dtype_qkv == CLEF_F32 ? 4 : 8;
  p.vec_qk = (dk % vi == 0) && (sqk % vi == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0) &&
             ((reinterpret_cast<uintptr_t>(k) & 15) == 0);
  p.qscale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(dk)));
  p.out = out;
  p.nseq = nseq;
  return 0;
}

extern "C" int clef_delta_scan(const void* q, const void* k, const void* v, int64_t sqk,
                               int64_t sv, int dtype_qkv, const void* g, const void* beta,
                               int64_t sgb, int dtype_gb, int T, int Hk, int Hv, int dk, int dv,
                               int chunk, int precision, const float* initial, int capture,
                               void* out, int64_t so, int dtype_out, float* captured,
                               float* final_state, void* workspace, size_t workspace_bytes,
                               void* stream) {
  clef::ScanParams p;
  if (int rc = scan_params(p, q, k, v, sqk, sv, dtype_qkv, g, beta, sgb, dtype_gb, T, Hk, Hv, dk, dv, chunk,
                           precision, out, so, dtype_out, workspace, workspace_bytes, 0))
    return rc;
  CLEF_REQUIRE(capture >= 0 && capture <= T, "DeltaNet scan: capture must be in 0..T");
  CLEF_REQUIRE(capture == 0 || captured, "DeltaNet scan: capture requested without a buffer");
  p.initial = initial; p.capture = capture;
  p.captured = captured; p.final_state = final_state;
  clef::scan_carve_workspace(p, workspace, precision);
  return clef::scan_launch(p, precision, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// clef_delta_scan_noalloc: the scan's workspace in a file-scope device array
// (one copy per GPU, held until the process ends).  Host code never passes
// `scratch` itself to a kernel or a copy: its name is a host-side stand-in.
// The device address of each GPU's copy comes from hipGetSymbolAddress, once
// per device with that device current, and only that address is used.
namespace {

__device__ __attribute__((aligned(256))) unsigned char scratch[CLEF_SCAN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(static_cast<int>(e), std::string("scan scratch: hipGetDevice: ") + hipGetErrorString(e));
  CLEF_REQUIRE(dev >= 0 && dev < kMaxDevices, "scan scratch: device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(e != hipSuccess ? static_cast<int>(e) : -2,
                  std::string("scan scratch: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace

extern "C" int clef_delta_scan_noalloc(const void* q, const void* k, const void* v, int64_t sqk, int64_t sv,
                                       int dtype_qkv, const void* g, const void* beta, int64_t sgb, int dtype_gb,
                                       int T, int Hk, int Hv, int dk, int dv, int chunk, int precision,
                                       const float* initial, int capture, void* out, int64_t so, int dtype_out,
                                       float* captured, float* final_state, void* stream) {
  if (int rc = scan_dims(T, Hk, Hv, dk, dv, chunk, precision)) return rc;
  const size_t need = clef::scan_workspace_bytes(T, Hk, Hv, dk, precision);
  CLEF_REQUIRE(need <= CLEF_SCAN_SCRATCH_BYTES,
               "DeltaNet scan (no-alloc): the workspace this shape needs exceeds the "
               "CLEF_SCAN_SCRATCH_BYTES scratch array");
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  // every scratch byte the kernels read is written earlier in the same call,
  // so nothing left by an earlier call needs clearing
  return clef_delta_scan(q, k, v, sqk, sv, dtype_qkv, g, beta, sgb, dtype_gb, T, Hk, Hv, dk, dv, chunk, precision,
                         initial, capture, out, so, dtype_out, captured, final_state, ws, CLEF_SCAN_SCRATCH_BYTES,
                         stream);
}

extern "C" size_t clef_delta_scan_varlen_workspace(int T, int nseq, int Hk, int Hv, int dk, int dv, int chunk,
                                                   int precision) {
  if (scan_dims(T, Hk, Hv, dk, dv, chunk, precision) || nseq < 1 || nseq > 4096) return 0;
  return clef::scan_workspace_bytes(T, Hk, Hv, dk, precision, nseq);
}

extern "C" int clef_delta_scan_varlen(const void* q, const void* k, const void* v, int64_t sqk, int64_t sv,
                                      int dtype_qkv, const void* g, const void* beta, int64_t sgb, int dtype_gb,
                                      const int32_t* cu_seqlens, int nseq, int T, int Hk, int Hv, int dk, int dv,
                                      int chunk, int precision, const float* initial, int64_t initial_stride,
                                      void* out, int64_t so, int dtype_out, float* final_states, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  CLEF_REQUIRE(cu_seqlens && nseq >= 1 && nseq <= 4096, "DeltaNet scan: cu_seqlens and 1 <= nseq <= 4096");
  CLEF_REQUIRE(initial_stride >= 0, "DeltaNet scan: negative initial-state stride");
  clef::ScanParams p;
  if (int rc = scan_params(p, q, k, v, sqk, sv, dtype_qkv, g, beta, sgb, dtype_gb, T, Hk, Hv, dk, dv, chunk,
                           precision, out, so, dtype_out, workspace, workspace_bytes, nseq))
    return rc;
  p.initial = initial;
  p.init_stride = initial_stride;
  p.final_state = final_states;
  p.cu_seqlens = cu_seqlens;
  clef::scan_carve_workspace(p, workspace, precision);
  return clef::scan_launch(p, precision, static_cast<hipStream_t>(stream));
}

// the mixer's conv + SiLU folded into the scan (see include/clef_hip.h)
// The ragged launch tables on the host, by the device kernels' own steps
// (ragged.hpp) run for every thread index in turn.
extern "C" int clef_ragged_plan(const int32_t* cu_seqlens, int nseq, int T, int unit, int32_t* spans,
                                int32_t* table, size_t table_entries) {
  using namespace clef;
  CLEF_REQUIRE(cu_seqlens && spans, "ragged plan: null pointer");
  CLEF_REQUIRE(nseq >= 1 && nseq <= kMaxRaggedSeq && T >= 1 && T <= (1 << 20), "ragged plan: 1..4096 sequences");
  CLEF_REQUIRE(unit == 64 || unit == 128, "ragged plan: unit 64 (scan chunks) or 128 (attention query tiles)");
  const size_t cap = (size_t)(T + unit - 1) / unit + nseq;
  CLEF_REQUIRE(!table || table_entries >= cap, "ragged plan: table smaller than ceil(T / unit) + nseq entries");
  std::vector<int> part(kTabThreads), R(nseq + 1), stab(4 * (size_t)nseq), ctab(2 * cap);
  const Ragged g{cu_seqlens, nseq, T, part.data(), R.data()};
  int total = 0;
  for (int t = 0; t < kTabThreads; ++t) rg_spans_1(g, t);
  for (int t = 0; t < kTabThreads; ++t) rg_spans_2(g, t);
  for (int t = 0; t < kTabThreads; ++t) rg_spans_3(g, t);
  for (int t = 0; t < kTabThreads; ++t) rg_count_4(g, t, unit);
  for (int t = 0; t < kTabThreads; ++t) rg_count_5(g, t, &total);
  if ((size_t)total > cap) return fail(-3, "ragged plan: the tables exceed their capacity");
  if (unit == 64) {
    for (int t = 0; t < kTabThreads; ++t) rg_scan_6(g, t, unit, ctab.data(), stab.data());
  } else {
    for (int t = 0; t < kTabThreads; ++t) rg_attn_6(g, t, unit, total, ctab.data());
  }
  for (int j = 0; j <= nseq; ++j) spans[j] = R[j];
  if (table)
    for (int i = 0; i < 2 * total; ++i) table[i] = ctab[i];
  return total;
}
