// Host orchestration of the hybrid prefill: the C++ counterpart of
// Backbone::{load, prefill} (crates/core/src/models/qwen.rs:193-426), with
// Delta::forward (:589-688) and FullAttention::forward (:451-525) issuing the
// gfx950 kernels of this library on one stream.  Nothing here touches tensor
// values on the host; the only host/device transfer is the token ids.
#include <hip/hip_runtime.h>

#include <time.h>

#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/clef_hip.h"
#include "common.hpp"

namespace clef {
namespace {

size_t al256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// y[r, c] = f32(x[r, c]) for rows of `cols` (conv history capture).
__global__ void rows_to_f32(const void* x, int64_t ldx, int dtype, float* y, int rows, int cols) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * cols) return;
  const int r = static_cast<int>(i / cols), c = static_cast<int>(i % cols);
  const int64_t s = (int64_t)r * ldx + c;
  y[i] = dtype == CLEF_F32 ? static_cast<const float*>(x)[s] : static_cast<float>(static_cast<const half_t*>(x)[s]);
}

// y = x + 1 (offset norms, normalization.rs:44-45), or a plain f32 copy.
__global__ void norm_weight(const float* x, float* y, int n, float add) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = x[i] + add;
}

}  // namespace

struct LayerState {
  int kind = 0;
  // owned
  void* in_w = nullptr;        // fused [qkv | z | a | b] or [q | k | v], act dtype
  void* ab_packed = nullptr;   // [a | b] rows in fragment order (clef_delta_gates_pack)
  float* in_norm = nullptr;    // input_norm offset
  float* post_norm = nullptr;  // post_attention_layernorm offset
  float* conv = nullptr;       // [W, taps]
  float* dt = nullptr;
  float* a_log = nullptr;
  float* gnorm = nullptr;      // gated norm (no offset)
  float* q_norm = nullptr;     // offset
  float* k_norm = nullptr;     // offset
  // referenced
  const void* gate = nullptr;
  const void* up = nullptr;
  const void* down = nullptr;
  const void* out = nullptr;   // DeltaNet out_proj or attention o_proj
};

}  // namespace clef

struct TimingRecord {
  int cat;
  hipEvent_t start, stop;
  double flops, bytes;
};

struct clef_backbone {
  clef_backbone_config c;
  bool timing = false;
  std::vector<TimingRecord> records;
  std::vector<hipEvent_t> event_pool;
  std::vector<clef::LayerState> layers;
  const void* embeddings = nullptr;
  float* final_norm = nullptr;
  std::vector<void*> owned;
  int ad = CLEF_F32;      // activation / projection dtype
  int conv_dt = CLEF_F32; // dtype of the conv output fed to the scan
  int key = 0, value = 0, W = 0, NP = 0, NA = 0;  // widths
  // f16 profile: the a/b projections run fused with the gates
  // (clef_delta_gates_proj), so the in-projection GEMM covers [qkv | z] only
  bool ab_fused = false;
  // cooperative cancellation / deadline (clef_backbone_set_control)
  clef_control control{nullptr, 0.0};
};

namespace clef {
namespace {

int hip_fail(hipError_t e, const char* what) {
  return fail(static_cast<int>(e), std::string(what) + ": " + hipGetErrorString(e));
}

#define CLEF_TRY(expr)        \
  do {                        \
    int rc_ = (expr);         \
    if (rc_ != 0) return rc_; \
  } while (0)
#define HIP_TRY(expr, what)                          \
  do {                                               \
    hipError_t e_ = (expr);                          \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// Control::check (models/mod.rs:49-58): cancellation first, then the deadline.
int control_check(const clef_backbone* b) {
  const clef_control& c = b->control;
  if (c.cancel && __atomic_load_n(c.cancel, __ATOMIC_ACQUIRE) != 0) return fail(CLEF_CANCELLED, "prefill cancelled");
  if (c.deadline > 0.0 && clef_monotonic_seconds() >= c.deadline)
    return fail(CLEF_DEADLINE_EXCEEDED, "prefill deadline exceeded");
  return 0;
}

struct Workspace {
  int32_t* ids;
  void* n;        // [T, H] act
  void* proj;     // [T, max(NP, NA)] act
  void* mixed;    // [T, W] conv_dt
  float* g;       // [T, Hv]
  float* beta;    // [T, Hv]
  void* scan_out;   // [T, Hv*dv] in the activation dtype
  void* gated;    // [T, max(value, heads*d)] act
  void* mlp;      // [T, I] act
  void* qh;       // [heads, T, d] act
  float* rot;     // [T, rotary_dim / 2] (cos, sin) pairs of the new tokens' positions
  void* kh;       // [kvh, Ttot, d] act
  void* vt;       // [kvh, d, ldv] act
  void* scan_ws;
  size_t scan_ws_bytes;
  int ldv;
  // ragged batches
  int32_t* cu;      // [nseq + 1] token offsets
  void* attn_ws;    // attention tables (mixed profile)
  size_t attn_ws_bytes;
  void* kseq;       // f32 profile: one sequence's [prefix; own] keys [kvh, prefix + T, d]
  void* vseq;       // and values [kvh, d, ldvs]
  int ldvs;
};

size_t elt(int dtype) { return dtype == CLEF_F32 ? 4 : 2; }

// A ragged batch runs its attention one sequence at a time over copied
// [prefix; own] keys in the f32 profile, and in the mixed profile when the
// shared prefix is not a multiple of 8 tokens (the packed kernel reads
// 8-key runs that must not straddle the prefix / own boundary).
bool varlen_per_sequence_attention(const clef_backbone* b, int prefix) {
  return b->ad == CLEF_F32 || prefix % 8 != 0;
}

// nseq > 0: a ragged batch of nseq sequences, T tokens in all, each after the
// same `prefix` cached tokens (which stay in the prefix state: kh / vt hold
// the packed new tokens only).
size_t carve(const clef_backbone* b, int T, int prefix, Workspace* w, char* base, int nseq = 0) {
  const clef_backbone_config& c = b->c;
  const size_t a = elt(b->ad);
  const int Ttot = (nseq > 0 ? 0 : prefix) + T;
  const int ldv = static_cast<int>(((Ttot + 63) / 64) * 64);
  const size_t scan_ws =
      nseq > 0 ? clef_delta_scan_varlen_workspace(T, nseq, c.lin_k_heads, c.lin_v_heads, c.lin_dk, c.lin_dv, 64,
                                                  c.scan_precision)
               : clef_delta_scan_workspace(T, c.lin_k_heads, c.lin_v_heads, c.lin_dk, c.lin_dv, 64,
                                           c.scan_precision);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += al256(bytes);
    return static_cast<void*>(p);
  };
  Workspace tmp{};
  Workspace& W = w ? *w : tmp;
  const int proj_cols = b->NP > b->NA ? b->NP : b->NA;
  const int gated_cols = b->value > c.heads * c.head_dim ? b->value : c.heads * c.head_dim;
  W.ids = static_cast<int32_t*>(take(sizeof(int32_t) * T));
  W.n = take(a * T * c.hidden);
  W.proj = take(a * T * proj_cols);
  W.mixed = take(elt(b->conv_dt) * T * b->W);
  W.g = static_cast<float*>(take(4ull * T * c.lin_v_heads));
  W.beta = static_cast<float*>(take(4ull * T * c.lin_v_heads));
  W.scan_out = take(4ull * T * b->value);
  W.gated = take(a * T * gated_cols);
  W.mlp = take(a * T * c.intermediate);
  W.qh = take(a * (size_t)c.heads * T * c.head_dim);
  W.rot = static_cast<float*>(take(4ull * T * (c.rotary_dim > 0 ? c.rotary_dim : 2)));
  W.kh = take(a * (size_t)c.kv_heads * Ttot * c.head_dim);
  W.vt = take(a * (size_t)c.kv_heads * c.head_dim * ldv);
  W.scan_ws = take(scan_ws);
  W.scan_ws_bytes = scan_ws;
  W.ldv = ldv;
  if (nseq > 0) {
    W.cu = static_cast<int32_t*>(take(sizeof(int32_t) * (nseq + 1)));
    W.attn_ws_bytes = clef_attention_varlen_workspace(T, nseq);
    W.attn_ws = take(W.attn_ws_bytes);
    if (varlen_per_sequence_attention(b, prefix)) {
      W.ldvs = static_cast<int>(((prefix + T + 63) / 64) * 64);
      W.kseq = take(a * (size_t)c.kv_heads * (prefix + T) * c.head_dim);
      W.vseq = take(a * (size_t)c.kv_heads * c.head_dim * W.ldvs);
    }
  }
  return off;
}

// Prefix-state layout: hidden [tokens, H] f32, then per layer either
// recurrent [Hv, dk, dv] f32 + history [taps-1, W] f32, or keys
// [kvh, tokens, d] + values [kvh, d, tokens] in the activation dtype.
struct PrefixView {
  float* hidden;
  std::vector<float*> rec, hist;
  std::vector<void*> key, val;
};

size_t prefix_layout(const clef_backbone* b, int tokens, char* base, PrefixView* v) {
  const clef_backbone_config& c = b->c;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += al256(bytes);
    return p;
  };
  PrefixView tmp;
  PrefixView& P = v ? *v : tmp;
  P.rec.assign(c.n_layers, nullptr);
  P.hist.assign(c.n_layers, nullptr);
  P.key.assign(c.n_layers, nullptr);
  P.val.assign(c.n_layers, nullptr);
  P.hidden = reinterpret_cast<float*>(take(4ull * tokens * c.hidden));
  for (int i = 0; i < c.n_layers; ++i) {
    if (b->layers[i].kind == 0) {
      P.rec[i] = reinterpret_cast<float*>(take(4ull * c.lin_v_heads * c.lin_dk * c.lin_dv));
      P.hist[i] = reinterpret_cast<float*>(take(4ull * (c.conv_taps - 1) * b->W));
    } else {
      P.key[i] = take(elt(b->ad) * (size_t)c.kv_heads * tokens * c.head_dim);
      P.val[i] = take(elt(b->ad) * (size_t)c.kv_heads * c.head_dim * tokens);
    }
  }
  return off;
}


hipEvent_t pooled_event(clef_backbone* b) {
  if (!b->event_pool.empty()) {
    hipEvent_t e = b->event_pool.back();
    b->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Runs `launch` and, while timing is enabled, brackets it with an event pair.
template <class F>
int timed(clef_backbone* b, int cat, double flops, double bytes, hipStream_t s, F&& launch) {
  if (!b->timing) return launch();
  TimingRecord r{cat, pooled_event(b), pooled_event(b), flops, bytes};
  if (!r.start || !r.stop) return fail(-2, "timing: event creation failed");
  HIP_TRY(hipEventRecord(r.start, s), "timing event");
  const int rc = launch();
  HIP_TRY(hipEventRecord(r.stop, s), "timing event");
  b->records.push_back(r);
  return rc;
}

int copy_rows(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (bytes == 0) return 0;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s), "device copy");
  return 0;
}

}  // namespace
}  // namespace clef

using namespace clef;

extern "C" int clef_backbone_create(const clef_backbone_config* config, const clef_layer_weights* lw,
                                    const void* embeddings, const void* final_norm,
                                    clef_backbone** out) {
  CLEF_REQUIRE(config && lw && embeddings && final_norm && out, "backbone: null argument");
  const clef_backbone_config& c = *config;
  CLEF_REQUIRE(c.hidden >= 1 && c.intermediate >= 1 && c.vocab >= 1 && c.n_layers >= 1,
               "backbone: hidden, intermediate, vocab and layer count must be positive");
  CLEF_REQUIRE(c.profile == CLEF_PROFILE_F32 || c.profile == CLEF_PROFILE_MIXED_F16, "backbone: profile");
  CLEF_REQUIRE(c.scan_precision == CLEF_SCAN_STRICT || c.scan_precision == CLEF_SCAN_MIXED,
               "backbone: scan precision");
  CLEF_REQUIRE(c.eps > 0.0f && c.eps <= 1.0f, "backbone: epsilon");
  CLEF_REQUIRE(c.max_tokens >= 1 && c.max_tokens <= (1 << 20), "backbone: max_tokens");
  bool any_attn = false, any_delta = false;
  for (int i = 0; i < c.n_layers; ++i) {
    CLEF_REQUIRE(lw[i].kind == 0 || lw[i].kind == 1, "backbone: layer kind");
    (lw[i].kind ? any_attn : any_delta) = true;
  }
  if (any_delta)
    CLEF_REQUIRE(c.lin_k_heads >= 1 && c.lin_v_heads % c.lin_k_heads == 0 && c.lin_dk >= 1 &&
                     c.lin_dk <= 128 && c.lin_dv >= 1 && c.lin_dv <= 128 && c.conv_taps >= 1 &&
                     c.conv_taps <= 8,
                 "backbone: DeltaNet head layout");
  if (any_attn)
    CLEF_REQUIRE(c.heads >= 1 && c.kv_heads >= 1 && c.heads % c.kv_heads == 0 && c.head_dim >= 1 &&
                     c.head_dim <= 256 && c.rotary_dim % 2 == 0 && c.rotary_dim <= c.head_dim &&
                     c.head_dim % (c.profile == CLEF_PROFILE_F32 ? 4 : 8) == 0,
                 "backbone: attention head layout");

  std::unique_ptr<clef_backbone> b(new (std::nothrow) clef_backbone());
  CLEF_REQUIRE(b, "backbone: out of host memory");
  b->c = c;
  if (!any_delta) b->c.lin_k_heads = b->c.lin_v_heads = b->c.lin_dk = b->c.lin_dv = 1, b->c.conv_taps = 1;
  if (!any_attn) b->c.heads = b->c.kv_heads = 1, b->c.head_dim = 8, b->c.rotary_dim = 0;
  const clef_backbone_config& C = b->c;
  b->ad = c.profile == CLEF_PROFILE_F32 ? CLEF_F32 : CLEF_F16;
  b->conv_dt = (c.profile == CLEF_PROFILE_F32 || c.scan_precision == CLEF_SCAN_STRICT) ? CLEF_F32 : CLEF_F16;
  b->key = C.lin_k_heads * C.lin_dk;
  b->value = C.lin_v_heads * C.lin_dv;
  b->W = 2 * b->key + b->value;
  b->NP = b->W + b->value + 2 * C.lin_v_heads;
  b->ab_fused = C.profile == CLEF_PROFILE_MIXED_F16 &&
                (C.lin_v_heads == 16 || C.lin_v_heads == 32 || C.lin_v_heads == 64) && C.hidden % 256 == 0;
  b->NA = 2 * C.heads * C.head_dim + 2 * C.kv_heads * C.head_dim;
  b->embeddings = embeddings;
  const size_t a = elt(b->ad);
  const int H = C.hidden;

  auto alloc = [&](size_t bytes) -> void* {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    b->owned.push_back(p);
    return p;
  };
  auto offset_norm = [&](const void* src, int n, float add) -> float* {
    float* dst = static_cast<float*>(alloc(4ull * n));
    if (!dst) return nullptr;
    hipLaunchKernelGGL(norm_weight, dim3((n + 255) / 256), dim3(256), 0, 0, static_cast<const float*>(src), dst,
                       n, add);
    return dst;
  };
  auto cleanup = [&]() {
    for (void* p : b->owned) (void)hipFree(p);
    b->owned.clear();
  };
  b->final_norm = offset_norm(final_norm, H, 1.0f);
  if (!b->final_norm) return cleanup(), fail(-2, "backbone: device allocation failed");
  for (int i = 0; i < c.n_layers; ++i) {
    const clef_layer_weights& L = lw[i];
    LayerState S;
    S.kind = L.kind;
    if (!L.input_norm || !L.post_norm || !L.gate || !L.up || !L.down)
      return cleanup(), fail(-1, "backbone: missing norm or MLP weights");
    S.in_norm = offset_norm(L.input_norm, H, 1.0f);
    S.post_norm = offset_norm(L.post_norm, H, 1.0f);
    S.gate = L.gate;
    S.up = L.up;
    S.down = L.down;
    if (L.kind == 0) {
      if (!L.qkv || !L.z || !L.a || !L.b || !L.out || !L.conv || !L.dt || !L.a_log || !L.norm)
        return cleanup(), fail(-1, "backbone: missing DeltaNet weights");
      // fused in-projection [qkv | z | a | b]: one GEMM over x
      char* w = static_cast<char*>(alloc(a * (size_t)b->NP * H));
      if (!w) return cleanup(), fail(-2, "backbone: device allocation failed");
      size_t o = 0;
      for (auto [src, rows] : {std::pair<const void*, int>{L.qkv, b->W}, {L.z, b->value},
                               {L.a, C.lin_v_heads}, {L.b, C.lin_v_heads}}) {
        if (hipMemcpy(w + o, src, a * (size_t)rows * H, hipMemcpyDeviceToDevice) != hipSuccess)
          return cleanup(), fail(-2, "backbone: weight copy failed");
        o += a * (size_t)rows * H;
      }
      S.in_w = w;
      if (b->ab_fused) {
        S.ab_packed = alloc(clef_delta_gates_pack_bytes(H, C.lin_v_heads));
        if (!S.ab_packed) return cleanup(), fail(-2, "backbone: device allocation failed");
        if (int rc = clef_delta_gates_pack(w + a * (size_t)(b->W + b->value) * H, H, H, C.lin_v_heads, CLEF_F16,
                                           S.ab_packed, nullptr))
          return cleanup(), rc;
      }
      S.out = L.out;
      S.conv = offset_norm(L.conv, b->W * C.conv_taps, 0.0f);
      S.dt = offset_norm(L.dt, C.lin_v_heads, 0.0f);
      S.a_log = offset_norm(L.a_log, C.lin_v_heads, 0.0f);
      S.gnorm = offset_norm(L.norm, C.lin_dv, 0.0f);
    } else {
      if (!L.q || !L.k || !L.v || !L.o || !L.q_norm || !L.k_norm)
        return cleanup(), fail(-1, "backbone: missing attention weights");
      char* w = static_cast<char*>(alloc(a * (size_t)b->NA * H));
      if (!w) return cleanup(), fail(-2, "backbone: device allocation failed");
      size_t o = 0;
      const int qrows = 2 * C.heads * C.head_dim, kvrows = C.kv_heads * C.head_dim;
      for (auto [src, rows] : {std::pair<const void*, int>{L.q, qrows}, {L.k, kvrows}, {L.v, kvrows}}) {
        if (hipMemcpy(w + o, src, a * (size_t)rows * H, hipMemcpyDeviceToDevice) != hipSuccess)
          return cleanup(), fail(-2, "backbone: weight copy failed");
        o += a * (size_t)rows * H;
      }
      S.in_w = w;
      S.out = L.o;
      S.q_norm = offset_norm(L.q_norm, C.head_dim, 1.0f);
      S.k_norm = offset_norm(L.k_norm, C.head_dim, 1.0f);
    }
    b->layers.push_back(S);
  }
  if (hipDeviceSynchronize() != hipSuccess) return cleanup(), fail(-2, "backbone: weight preparation failed");
  *out = b.release();
  return 0;
}

extern "C" void clef_backbone_destroy(clef_backbone* b) {
  if (!b) return;
  for (auto& r : b->records) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  for (hipEvent_t e : b->event_pool) (void)hipEventDestroy(e);
  for (void* p : b->owned) (void)hipFree(p);
  delete b;
}

extern "C" int clef_backbone_enable_timing(clef_backbone* b, int enable) {
  CLEF_REQUIRE(b, "timing: null backbone");
  b->timing = enable != 0;
  return 0;
}

extern "C" int clef_backbone_timings(clef_backbone* b, double* ms, int* launches, double* flops, double* bytes) {
  CLEF_REQUIRE(b && ms && launches && flops && bytes, "timing: null argument");
  for (int i = 0; i < CLEF_CAT_COUNT; ++i) ms[i] = flops[i] = bytes[i] = 0.0, launches[i] = 0;
  int rc = 0;
  for (auto& r : b->records) {
    float t = 0.0f;
    hipError_t e = hipEventSynchronize(r.stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&t, r.start, r.stop);
    if (e != hipSuccess && rc == 0) rc = fail(static_cast<int>(e), "timing: event query failed");
    ms[r.cat] += t;
    launches[r.cat] += 1;
    flops[r.cat] += r.flops;
    bytes[r.cat] += r.bytes;
    b->event_pool.push_back(r.start);
    b->event_pool.push_back(r.stop);
  }
  b->records.clear();
  return rc;
}

extern "C" size_t clef_backbone_workspace(const clef_backbone* b, int T, int prefix_tokens) {
  if (!b || T < 1 || prefix_tokens < 0) return 0;
  return carve(b, T, prefix_tokens, nullptr, nullptr) + 256;
}

extern "C" size_t clef_backbone_prefix_bytes(const clef_backbone* b, int tokens) {
  if (!b || tokens < 1) return 0;
  return prefix_layout(b, tokens, nullptr, nullptr);
}

extern "C" double clef_monotonic_seconds(void) {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return static_cast<double>(ts.tv_sec) + 1e-9 * static_cast<double>(ts.tv_nsec);
}

extern "C" int clef_backbone_set_control(clef_backbone* b, const clef_control* control) {
  CLEF_REQUIRE(b, "control: null backbone");
  b->control = control ? *control : clef_control{nullptr, 0.0};
  return 0;
}

extern "C" int clef_backbone_prefill(clef_backbone* b, const int32_t* ids, int T, const void* initial,
                                     int initial_tokens, size_t initial_bytes, int capture, void* saved,
                                     size_t saved_bytes, float* hidden, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  CLEF_REQUIRE(b && ids && hidden && workspace, "prefill: null argument");
  CLEF_TRY(control_check(b));  // qwen.rs:344
  const clef_backbone_config& c = b->c;
  const int offset = initial ? initial_tokens : 0;
  // request validation, qwen.rs:345-359 (a state of another shape: :355)
  CLEF_REQUIRE(T >= 1 && offset >= 0 && (!initial || offset >= 1) && (int64_t)offset + T <= c.max_tokens,
               "prefill boundary or vocabulary");
  CLEF_REQUIRE(capture >= 0 && (capture == 0 || capture < T) && !(initial && capture) &&
                   (capture == 0 || saved),
               "prefill boundary or vocabulary");
  CLEF_REQUIRE(!initial || initial_bytes == prefix_layout(b, offset, nullptr, nullptr),
               "prefill boundary or vocabulary: the initial state's size does not match this backbone at "
               "initial_tokens");
  CLEF_REQUIRE(!capture || saved_bytes >= prefix_layout(b, capture, nullptr, nullptr),
               "prefill: the capture buffer is smaller than clef_backbone_prefix_bytes(capture)");
  for (int t = 0; t < T; ++t) CLEF_REQUIRE(ids[t] >= 0 && ids[t] < c.vocab, "prefill boundary or vocabulary");
  const size_t need = carve(b, T, offset, nullptr, nullptr);
  char* base = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(workspace) + 255) & ~static_cast<uintptr_t>(255));
  CLEF_REQUIRE(workspace_bytes >= need + static_cast<size_t>(base - static_cast<char*>(workspace)),
               "prefill: workspace too small");
  Workspace w;
  carve(b, T, offset, &w, base);
  PrefixView init, sav;
  if (initial) prefix_layout(b, offset, static_cast<char*>(const_cast<void*>(initial)), &init);
  if (capture) prefix_layout(b, capture, static_cast<char*>(saved), &sav);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int H = c.hidden, ad = b->ad;
  const size_t a = elt(ad);
  float* h = hidden + (size_t)offset * H;  // residual stream of the new tokens
  HIP_TRY(hipMemcpyAsync(w.ids, ids, sizeof(int32_t) * T, hipMemcpyHostToDevice, s), "ids upload");
#define TIMED(cat, flops, bytes, expr) \
  CLEF_TRY(timed(b, cat, static_cast<double>(flops), static_cast<double>(bytes), s, [&]() { return (expr); }))
  const double da = static_cast<double>(a);
  auto gemm_bytes = [&](double M, double N, double K, bool residual) {
    return da * (M * K + N * K) + (residual ? 8.0 * M * N : da * M * N);
  };
  // the embedding and the first layer's input norm in one pass where it applies
  const bool normed0 =
      c.n_layers > 0 && embed_rms_applies(b->embeddings, H, h, b->layers[0].in_norm, w.n, H);
  if (normed0)
    TIMED(CLEF_CAT_OTHER, 4.0 * T * H, (4.0 + 2.0 * da) * T * H,
          embed_rms_launch(w.ids, T, b->embeddings, ad, c.vocab, H, h, b->layers[0].in_norm, w.n, H, ad, c.eps, s));
  else
    TIMED(CLEF_CAT_OTHER, 0, (4.0 + da) * T * H, clef_embed(w.ids, T, b->embeddings, ad, c.vocab, H, h, s));
  const int Hv = c.lin_v_heads, dv = c.lin_dv, taps = c.conv_taps;
  const int heads = c.heads, kvh = c.kv_heads, d = c.head_dim;
  const int Ttot = offset + T;
  const double rms_bytes = (4.0 + da) * T * H;

  for (int li = 0; li < c.n_layers; ++li) {
    const LayerState& L = b->layers[li];
    CLEF_TRY(control_check(b));  // qwen.rs:380
    if (li > 0 || !normed0)
      TIMED(CLEF_CAT_NORM, 4.0 * T * H, rms_bytes, clef_rms_norm(h, H, CLEF_F32, L.in_norm, w.n, H, ad, T, H, c.eps, s));
    if (L.kind == 0) {
      const int NP = b->NP, Wc = b->W;
      char* proj = static_cast<char*>(w.proj);
      const int NG = b->ab_fused ? Wc + b->value : NP;  // GEMM columns
      TIMED(CLEF_CAT_GEMM, 2.0 * T * NG * H, gemm_bytes(T, NG, H, false),
            clef_gemm(w.n, H, L.in_w, H, proj, NP, T, NG, H, ad, ad, CLEF_EPI_STORE, s));
      const int hist_rows = initial ? (offset < taps - 1 ? offset : taps - 1) : 0;
      const double ce = static_cast<double>(elt(b->conv_dt));
      TIMED(CLEF_CAT_CONV, 2.0 * T * Wc * taps, (da + ce) * T * Wc,
            clef_conv_silu(proj, NP, ad, initial ? init.hist[li] : nullptr, hist_rows, L.conv, taps, w.mixed, Wc,
                           b->conv_dt, T, Wc, s));
      if (b->ab_fused) {
        TIMED(CLEF_CAT_OTHER, 2.0 * T * 2 * Hv * H, da * (T * H + 2.0 * Hv * H) + 8.0 * T * Hv,
              clef_delta_gates_proj(w.n, H, L.ab_packed, H, ad, L.dt, L.a_log, w.g, w.beta, T, Hv, s));
      } else {
        TIMED(CLEF_CAT_OTHER, 0, (2.0 * da + 8.0) * T * Hv,
              clef_delta_gates(proj + a * (Wc + b->value), NP, proj + a * (Wc + b->value + Hv), NP, ad, L.dt,
                               L.a_log, w.g, w.beta, T, Hv, s));
      }
      const char* mixed = static_cast<const char*>(w.mixed);
      const size_t ces = elt(b->conv_dt);
      const double nchunk = (T + 63) / 64;
      const double scan_flops =
          nchunk * (c.lin_k_heads * 4.0 * 64 * 64 * c.lin_dk +
                    Hv * (2.0 * 64 * 64 * c.lin_dk + 4.0 * 64 * 64 * dv + 6.0 * 64 * c.lin_dk * dv + 64.0 * 64 * 64 * 2 / 3));
      const double state = 4.0 * Hv * c.lin_dk * dv;
      // the scan writes o in the activation dtype: the gated norm rounds it
      // there first (qwen.rs:671), so f16 output is the same value
      const double scan_bytes = ce * T * (2.0 * b->key + b->value) + 8.0 * T * Hv + da * T * b->value +
                                (initial ? state : 0.0) + (capture ? state : 0.0);
      TIMED(CLEF_CAT_SCAN, scan_flops, scan_bytes,
            clef_delta_scan(mixed, mixed + ces * b->key, mixed + ces * 2 * b->key, Wc, Wc, b->conv_dt, w.g, w.beta, Hv,
                            CLEF_F32, T, c.lin_k_heads, Hv, c.lin_dk, dv, 64, c.scan_precision,
                            initial ? init.rec[li] : nullptr, capture, w.scan_out, (int64_t)Hv * dv, ad,
                            capture ? sav.rec[li] : nullptr, nullptr, w.scan_ws, w.scan_ws_bytes, s));
      TIMED(CLEF_CAT_NORM, 6.0 * T * b->value, 3.0 * da * T * b->value,
            clef_gated_rms_silu(w.scan_out, ad, proj + a * Wc, NP, ad, L.gnorm, w.gated, ad, T, Hv, dv, c.eps, s));
      TIMED(CLEF_CAT_GEMM, 2.0 * T * H * b->value, gemm_bytes(T, H, b->value, true),
            clef_gemm(w.gated, b->value, L.out, b->value, h, H, T, H, b->value, ad, ad, CLEF_EPI_RESIDUAL, s));
      if (capture) {  // conv history: last min(capture, taps-1) projected rows (qwen.rs:677-685)
        const int count = capture < taps - 1 ? capture : taps - 1;
        if (count > 0) {
          hipLaunchKernelGGL(rows_to_f32, dim3((count * Wc + 255) / 256), dim3(256), 0, s,
                             proj + a * (size_t)(capture - count) * NP, (int64_t)NP, ad, sav.hist[li], count, Wc);
          CLEF_TRY(check_launch("history capture"));
        }
      }
    } else {
      const int NA = b->NA;
      char* proj = static_cast<char*>(w.proj);
      TIMED(CLEF_CAT_GEMM, 2.0 * T * NA * H, gemm_bytes(T, NA, H, false),
            clef_gemm(w.n, H, L.in_w, H, proj, NA, T, NA, H, ad, ad, CLEF_EPI_STORE, s));
      const size_t koff = a * 2 * heads * d, voff = koff + a * kvh * d;
      // mixed profile, d = 256, rotary on 64 features: the query norm and
      // rotary run inside the attention core (rotated by the key pass's
      // table of the same positions); otherwise as their own pass
      const bool qfuse = ad == CLEF_F16 && d == 256 && c.rotary_dim == 64 && NA % 8 == 0 &&
                         ((reinterpret_cast<uintptr_t>(L.q_norm) | reinterpret_cast<uintptr_t>(proj)) & 15) == 0;
      if (!qfuse)
        TIMED(CLEF_CAT_NORM, 0, 2.0 * da * T * heads * d,
              clef_qk_norm_rotary(proj, NA, 2 * d, ad, L.q_norm, w.qh, T, ad, T, heads, d, c.rotary_dim,
                                  c.rope_theta, offset, 0, c.eps, s));
      if (initial) {  // cached keys and values precede the new ones (qwen.rs:486-496)
        for (int g = 0; g < kvh; ++g)
          CLEF_TRY(copy_rows(static_cast<char*>(w.kh) + a * (size_t)g * Ttot * d,
                             static_cast<char*>(init.key[li]) + a * (size_t)g * offset * d, a * (size_t)offset * d, s));
        HIP_TRY(hipMemcpy2DAsync(w.vt, a * w.ldv, init.val[li], a * offset, a * offset, (size_t)kvh * d,
                                 hipMemcpyDeviceToDevice, s),
                "value prefix copy");
      }
      if (qfuse)
        TIMED(CLEF_CAT_NORM, 0, 2.0 * da * T * kvh * d,
              qk_norm_rotary_table_launch(proj + koff, NA, d, L.k_norm, w.kh, Ttot, T, kvh, d, c.rotary_dim,
                                          c.rope_theta, offset, offset, c.eps, w.rot, s));
      else
        TIMED(CLEF_CAT_NORM, 0, 2.0 * da * T * kvh * d,
              clef_qk_norm_rotary(proj + koff, NA, d, ad, L.k_norm, w.kh, Ttot, ad, T, kvh, d, c.rotary_dim,
                                  c.rope_theta, offset, offset, c.eps, s));
      TIMED(CLEF_CAT_OTHER, 0, 2.0 * da * T * kvh * d,
            clef_values_transposed(proj + voff, NA, ad, w.vt, w.ldv, ad, T, kvh, d, offset, s));
      if (capture) {
        for (int g = 0; g < kvh; ++g)
          CLEF_TRY(copy_rows(static_cast<char*>(sav.key[li]) + a * (size_t)g * capture * d,
                             static_cast<char*>(w.kh) + a * (size_t)g * Ttot * d, a * (size_t)capture * d, s));
        HIP_TRY(hipMemcpy2DAsync(sav.val[li], a * capture, w.vt, a * w.ldv, a * capture, (size_t)kvh * d,
                                 hipMemcpyDeviceToDevice, s),
                "value capture");
      }
      const double pairs = static_cast<double>(T) * offset + 0.5 * T * (T + 1.0);
      if (qfuse)
        TIMED(CLEF_CAT_ATTENTION, 4.0 * d * heads * pairs, da * (3.0 * T * heads * d + 2.0 * Ttot * kvh * d),
              clef_attention_gated_qnorm(proj, NA, 2 * d, L.q_norm, c.eps, w.rot, w.kh, Ttot, w.vt, w.ldv, heads,
                                         kvh, T, Ttot, d, proj + a * d, NA, 2 * d, w.gated, (int64_t)heads * d, s));
      else
        TIMED(CLEF_CAT_ATTENTION, 4.0 * d * heads * pairs, da * (3.0 * T * heads * d + 2.0 * Ttot * kvh * d),
              clef_attention_gated(w.qh, T, w.kh, Ttot, w.vt, w.ldv, ad, heads, kvh, T, Ttot, d, proj + a * d, NA,
                                   2 * d, w.gated, (int64_t)heads * d, s));
      TIMED(CLEF_CAT_GEMM, 2.0 * T * H * heads * d, gemm_bytes(T, H, heads * d, true),
            clef_gemm(w.gated, heads * d, L.out, heads * d, h, H, T, H, heads * d, ad, ad, CLEF_EPI_RESIDUAL, s));
    }
    TIMED(CLEF_CAT_NORM, 4.0 * T * H, rms_bytes, clef_rms_norm(h, H, CLEF_F32, L.post_norm, w.n, H, ad, T, H, c.eps, s));
    const double I = c.intermediate;
    TIMED(CLEF_CAT_GEMM, 4.0 * T * I * H, da * (T * H + 2.0 * I * H + T * I),
          clef_gemm_swiglu(w.n, H, L.gate, L.up, H, w.mlp, c.intermediate, T, c.intermediate, H, ad, s));
    TIMED(CLEF_CAT_GEMM, 2.0 * T * I * H, gemm_bytes(T, H, I, true),
          clef_gemm(w.mlp, c.intermediate, L.down, c.intermediate, h, H, T, H, c.intermediate, ad, ad,
                    CLEF_EPI_RESIDUAL, s));
  }
  TIMED(CLEF_CAT_NORM, 4.0 * T * H, 8.0 * T * H, clef_rms_norm(h, H, CLEF_F32, b->final_norm, h, H, CLEF_F32, T, H, c.eps, s));
#undef TIMED
  if (initial) CLEF_TRY(copy_rows(hidden, init.hidden, 4ull * offset * H, s));
  if (capture) CLEF_TRY(copy_rows(sav.hidden, h, 4ull * capture * H, s));
  return 0;
}

extern "C" size_t clef_backbone_varlen_workspace(const clef_backbone* b, int T, int nseq, int prefix_tokens) {
  if (!b || T < 1 || nseq < 1 || nseq > 4096 || prefix_tokens < 0) return 0;
  return carve(b, T, prefix_tokens, nullptr, nullptr, nseq) + 256;
}

// Ragged batch of requests that share one cached prefix (a prefix-cache hit
// for every request, prefix_cache.rs:135-177): each sequence's hidden states
// equal clef_backbone_prefill of its ids resumed from `initial`.
extern "C" int clef_backbone_prefill_varlen(clef_backbone* b, const int32_t* ids, const int32_t* cu_seqlens,
                                            int nseq, const void* initial, int initial_tokens, size_t initial_bytes,
                                            float* hidden, void* workspace, size_t workspace_bytes, void* stream) {
  CLEF_REQUIRE(b && ids && cu_seqlens && hidden && workspace, "prefill: null argument");
  CLEF_TRY(control_check(b));
  CLEF_REQUIRE(nseq >= 1 && nseq <= 4096 && cu_seqlens[0] == 0, "prefill: 1..4096 sequences from offset 0");
  const clef_backbone_config& c = b->c;
  const int offset = initial ? initial_tokens : 0;
  CLEF_REQUIRE(offset >= 0 && (!initial || offset >= 1), "prefill boundary or vocabulary");
  CLEF_REQUIRE(!initial || initial_bytes == prefix_layout(b, offset, nullptr, nullptr),
               "prefill boundary or vocabulary: the initial state's size does not match this backbone at "
               "initial_tokens");
  for (int s = 0; s < nseq; ++s)
    CLEF_REQUIRE(cu_seqlens[s + 1] > cu_seqlens[s] && (int64_t)offset + cu_seqlens[s + 1] - cu_seqlens[s] <= c.max_tokens,
                 "prefill: every sequence needs 1..max_tokens - prefix tokens");
  const int T = cu_seqlens[nseq];
  CLEF_REQUIRE(T <= (1 << 20), "prefill: at most 2^20 tokens per batch");
  for (int t = 0; t < T; ++t) CLEF_REQUIRE(ids[t] >= 0 && ids[t] < c.vocab, "prefill boundary or vocabulary");
  const size_t need = carve(b, T, offset, nullptr, nullptr, nseq);
  char* base = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(workspace) + 255) & ~static_cast<uintptr_t>(255));
  CLEF_REQUIRE(workspace_bytes >= need + static_cast<size_t>(base - static_cast<char*>(workspace)),
               "prefill: workspace too small");
  Workspace w;
  carve(b, T, offset, &w, base, nseq);
  PrefixView init;
  if (initial) prefix_layout(b, offset, static_cast<char*>(const_cast<void*>(initial)), &init);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int H = c.hidden, ad = b->ad;
  const size_t a = elt(ad);
  float* h = hidden;
  HIP_TRY(hipMemcpyAsync(w.ids, ids, sizeof(int32_t) * T, hipMemcpyHostToDevice, s), "ids upload");
  HIP_TRY(hipMemcpyAsync(w.cu, cu_seqlens, sizeof(int32_t) * (nseq + 1), hipMemcpyHostToDevice, s),
          "cu_seqlens upload");
#define TIMED(cat, flops, bytes, expr) \
  CLEF_TRY(timed(b, cat, static_cast<double>(flops), static_cast<double>(bytes), s, [&]() { return (expr); }))
  const double da = static_cast<double>(a);
  auto gemm_bytes = [&](double M, double N, double K, bool residual) {
    return da * (M * K + N * K) + (residual ? 8.0 * M * N : da * M * N);
  };
  // the embedding and the first layer's input norm in one pass where it applies
  const bool normed0 =
      c.n_layers > 0 && embed_rms_applies(b->embeddings, H, h, b->layers[0].in_norm, w.n, H);
  if (normed0)
    TIMED(CLEF_CAT_OTHER, 4.0 * T * H, (4.0 + 2.0 * da) * T * H,
          embed_rms_launch(w.ids, T, b->embeddings, ad, c.vocab, H, h, b->layers[0].in_norm, w.n, H, ad, c.eps, s));
  else
    TIMED(CLEF_CAT_OTHER, 0, (4.0 + da) * T * H, clef_embed(w.ids, T, b->embeddings, ad, c.vocab, H, h, s));
  const int Hv = c.lin_v_heads, dv = c.lin_dv, taps = c.conv_taps;
  const int heads = c.heads, kvh = c.kv_heads, d = c.head_dim;
  const double rms_bytes = (4.0 + da) * T * H;
  // attention pairs: each query sees the prefix and its own earlier tokens
  double pairs = 0.0;
  for (int q = 0; q < nseq; ++q) {
    const double L = cu_seqlens[q + 1] - cu_seqlens[q];
    pairs += L * offset + 0.5 * L * (L + 1.0);
  }

  for (int li = 0; li < c.n_layers; ++li) {
    const LayerState& L = b->layers[li];
    CLEF_TRY(control_check(b));  // qwen.rs:380
    if (li > 0 || !normed0)
      TIMED(CLEF_CAT_NORM, 4.0 * T * H, rms_bytes, clef_rms_norm(h, H, CLEF_F32, L.in_norm, w.n, H, ad, T, H, c.eps, s));
    if (L.kind == 0) {
      const int NP = b->NP, Wc = b->W;
      char* proj = static_cast<char*>(w.proj);
      const int NG = b->ab_fused ? Wc + b->value : NP;  // GEMM columns
      TIMED(CLEF_CAT_GEMM, 2.0 * T * NG * H, gemm_bytes(T, NG, H, false),
            clef_gemm(w.n, H, L.in_w, H, proj, NP, T, NG, H, ad, ad, CLEF_EPI_STORE, s));
      const int hist_rows = initial ? (offset < taps - 1 ? offset : taps - 1) : 0;
      const double ce = static_cast<double>(elt(b->conv_dt));
      TIMED(CLEF_CAT_CONV, 2.0 * T * Wc * taps, (da + ce) * T * Wc,
            clef_conv_silu_varlen(proj, NP, ad, initial ? init.hist[li] : nullptr, hist_rows, 0, w.cu, nseq,
                                  L.conv, taps, w.mixed, Wc, b->conv_dt, T, Wc, s));
      if (b->ab_fused) {
        TIMED(CLEF_CAT_OTHER, 2.0 * T * 2 * Hv * H, da * (T * H + 2.0 * Hv * H) + 8.0 * T * Hv,
              clef_delta_gates_proj(w.n, H, L.ab_packed, H, ad, L.dt, L.a_log, w.g, w.beta, T, Hv, s));
      } else {
        TIMED(CLEF_CAT_OTHER, 0, (2.0 * da + 8.0) * T * Hv,
              clef_delta_gates(proj + a * (Wc + b->value), NP, proj + a * (Wc + b->value + Hv), NP, ad, L.dt,
                               L.a_log, w.g, w.beta, T, Hv, s));
      }
      const char* mixed = static_cast<const char*>(w.mixed);
      const size_t ces = elt(b->conv_dt);
      const double state = 4.0 * Hv * c.lin_dk * dv;
      const double scan_bytes = ce * T * (2.0 * b->key + b->value) + 8.0 * T * Hv + da * T * b->value +
                                (initial ? state : 0.0);
      TIMED(CLEF_CAT_SCAN, 0, scan_bytes,
            clef_delta_scan_varlen(mixed, mixed + ces * b->key, mixed + ces * 2 * b->key, Wc, Wc, b->conv_dt, w.g,
                                   w.beta, Hv, CLEF_F32, w.cu, nseq, T, c.lin_k_heads, Hv, c.lin_dk, dv, 64,
                                   c.scan_precision, initial ? init.rec[li] : nullptr, 0, w.scan_out,
                                   (int64_t)Hv * dv, ad, nullptr, w.scan_ws, w.scan_ws_bytes, s));
      TIMED(CLEF_CAT_NORM, 6.0 * T * b->value, 3.0 * da * T * b->value,
            clef_gated_rms_silu(w.scan_out, ad, proj + a * Wc, NP, ad, L.gnorm, w.gated, ad, T, Hv, dv, c.eps, s));
      TIMED(CLEF_CAT_GEMM, 2.0 * T * H * b->value, gemm_bytes(T, H, b->value, true),
            clef_gemm(w.gated, b->value, L.out, b->value, h, H, T, H, b->value, ad, ad, CLEF_EPI_RESIDUAL, s));
    } else {
      const int NA = b->NA;
      char* proj = static_cast<char*>(w.proj);
      TIMED(CLEF_CAT_GEMM, 2.0 * T * NA * H, gemm_bytes(T, NA, H, false),
            clef_gemm(w.n, H, L.in_w, H, proj, NA, T, NA, H, ad, ad, CLEF_EPI_STORE, s));
      const size_t koff = a * 2 * heads * d, voff = koff + a * kvh * d;
      TIMED(CLEF_CAT_NORM, 0, 2.0 * da * T * heads * d,
            clef_qk_norm_rotary_varlen(proj, NA, 2 * d, ad, L.q_norm, w.qh, T, ad, T, heads, d, c.rotary_dim,
                                       c.rope_theta, offset, w.cu, nseq, 0, c.eps, s));
      TIMED(CLEF_CAT_NORM, 0, 2.0 * da * T * kvh * d,
            clef_qk_norm_rotary_varlen(proj + koff, NA, d, ad, L.k_norm, w.kh, T, ad, T, kvh, d, c.rotary_dim,
                                       c.rope_theta, offset, w.cu, nseq, 0, c.eps, s));
      TIMED(CLEF_CAT_OTHER, 0, 2.0 * da * T * kvh * d,
            clef_values_transposed(proj + voff, NA, ad, w.vt, w.ldv, ad, T, kvh, d, 0, s));
      if (!varlen_per_sequence_attention(b, offset)) {
        TIMED(CLEF_CAT_ATTENTION, 4.0 * d * heads * pairs, da * (3.0 * T * heads * d + 2.0 * (T + offset) * kvh * d),
              clef_attention_gated_varlen(w.qh, T, w.kh, T, w.vt, w.ldv, w.cu, nseq, T,
                                          initial ? init.key[li] : nullptr, offset,
                                          initial ? init.val[li] : nullptr, offset, offset, ad, heads, kvh, d,
                                          proj + a * d, NA, 2 * d, w.gated, (int64_t)heads * d, w.attn_ws,
                                          w.attn_ws_bytes, s));
      } else {
        // one launch per sequence over [prefix; own] keys
        for (int q = 0; q < nseq; ++q) {
          const int t0 = cu_seqlens[q], Lq = cu_seqlens[q + 1] - t0, kn = offset + Lq;
          for (int gk = 0; gk < kvh; ++gk) {
            char* kd = static_cast<char*>(w.kseq) + a * (size_t)gk * kn * d;
            if (initial)
              CLEF_TRY(copy_rows(kd, static_cast<char*>(init.key[li]) + a * (size_t)gk * offset * d,
                                 a * (size_t)offset * d, s));
            CLEF_TRY(copy_rows(kd + a * (size_t)offset * d,
                               static_cast<char*>(w.kh) + a * ((size_t)gk * T + t0) * d, a * (size_t)Lq * d, s));
          }
          if (initial)
            HIP_TRY(hipMemcpy2DAsync(w.vseq, a * w.ldvs, init.val[li], a * offset, a * offset, (size_t)kvh * d,
                                     hipMemcpyDeviceToDevice, s),
                    "value prefix copy");
          HIP_TRY(hipMemcpy2DAsync(static_cast<char*>(w.vseq) + a * offset, a * w.ldvs,
                                   static_cast<char*>(w.vt) + a * t0, a * w.ldv, a * Lq, (size_t)kvh * d,
                                   hipMemcpyDeviceToDevice, s),
                  "value copy");
          const double pq = static_cast<double>(Lq) * offset + 0.5 * Lq * (Lq + 1.0);
          TIMED(CLEF_CAT_ATTENTION, 4.0 * d * heads * pq, da * (3.0 * Lq * heads * d + 2.0 * kn * kvh * d),
                clef_attention_gated(static_cast<char*>(w.qh) + a * (size_t)t0 * d, T, w.kseq, kn, w.vseq, w.ldvs,
                                     ad, heads, kvh, Lq, kn, d, proj + a * ((size_t)t0 * NA + d), NA, 2 * d,
                                     static_cast<char*>(w.gated) + a * (size_t)t0 * heads * d, (int64_t)heads * d,
                                     s));
        }
      }
      TIMED(CLEF_CAT_GEMM, 2.0 * T * H * heads * d, gemm_bytes(T, H, heads * d, true),
            clef_gemm(w.gated, heads * d, L.out, heads * d, h, H, T, H, heads * d, ad, ad, CLEF_EPI_RESIDUAL, s));
    }
    TIMED(CLEF_CAT_NORM, 4.0 * T * H, rms_bytes, clef_rms_norm(h, H, CLEF_F32, L.post_norm, w.n, H, ad, T, H, c.eps, s));
    const double I = c.intermediate;
    TIMED(CLEF_CAT_GEMM, 4.0 * T * I * H, da * (T * H + 2.0 * I * H + T * I),
          clef_gemm_swiglu(w.n, H, L.gate, L.up, H, w.mlp, c.intermediate, T, c.intermediate, H, ad, s));
    TIMED(CLEF_CAT_GEMM, 2.0 * T * I * H, gemm_bytes(T, H, I, true),
          clef_gemm(w.mlp, c.intermediate, L.down, c.intermediate, h, H, T, H, c.intermediate, ad, ad,
                    CLEF_EPI_RESIDUAL, s));
  }
  TIMED(CLEF_CAT_NORM, 4.0 * T * H, 8.0 * T * H, clef_rms_norm(h, H, CLEF_F32, b->final_norm, h, H, CLEF_F32, T, H, c.eps, s));
#undef TIMED
  return 0;
}
