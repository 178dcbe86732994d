// Memory-bound pieces around the scan and the attention core, with their C ABI
// entry points.  Each kernel keeps the reference's op order and rounding
// points (crates/core/src/models/qwen.rs, ops.rs, pointwise.metal); the
// multiplies and adds that the reference rounds separately use mul_rn /
// add_rn, inside which the compiler may not contract or fold roundings.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>
#include <vector>

#include "../../include/clef_hip.h"
#include "common.hpp"

namespace clef {
namespace {

__device__ __forceinline__ float ld(const void* p, int64_t i, int dtype) {
  return dtype == CLEF_F32 ? static_cast<const float*>(p)[i]
                           : static_cast<float>(static_cast<const half_t*>(p)[i]);
}
__device__ __forceinline__ void st(void* p, int64_t i, int dtype, float v) {
  if (dtype == CLEF_F32)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<half_t*>(p)[i] = to_f16(v);
}
__device__ __forceinline__ float rnd(float v, int dtype) {
  return dtype == CLEF_F16 ? static_cast<float>(to_f16(v)) : v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---- RMSNorm: one wave per row (ops.rs:17-32; pointwise.metal:7-43) --------
__global__ __launch_bounds__(256) void rms_kernel(const void* x, int64_t ldx, int dti, const float* w,
                                                  void* y, int64_t ldy, int dto, int rows, int width,
                                                  float eps, float inv_width) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float s = 0.0f;
  for (int i = lane; i < width; i += 64) {
    const float v = ld(x, (int64_t)row * ldx + i, dti);
    s += v * v;
  }
  s = wave_sum(s);
  const float inverse = 1.0f / sqrtf(add_rn(mul_rn(s, inv_width), eps));
  for (int i = lane; i < width; i += 64) {
    const float v = ld(x, (int64_t)row * ldx + i, dti);
    st(y, (int64_t)row * ldy + i, dto, mul_rn(mul_rn(v, inverse), w[i]));
  }
}

// ---- causal conv + SiLU (qwen.rs:609-618, 765-796) --------------------------
__global__ __launch_bounds__(256) void conv_silu_kernel(const void* x, int64_t ldx, int dti,
                                                        const float* hist, int hrows, const float* w,
                                                        int taps, void* y, int64_t ldy, int dto, int T,
                                                        int W) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * W) return;
  const int t = static_cast<int>(idx / W), c = static_cast<int>(idx % W);
  const int pos = hrows + t;  // position in [history; x]
  float acc = 0.0f;
  for (int tap = 0; tap < taps; ++tap) {
    const int src = pos - (taps - 1 - tap);
    if (src < 0) continue;
    const float v = src < hrows ? hist[(int64_t)src * W + c] : ld(x, (int64_t)(src - hrows) * ldx + c, dti);
    acc = add_rn(acc, mul_rn(v, w[(int64_t)c * taps + tap]));
  }
  st(y, (int64_t)t * ldy + c, dto, acc / (1.0f + expf(-acc)));
}

// Eight consecutive channels of one input row, as loaded (f16 or f32).
template <class TI>
struct Row8;
template <>
struct Row8<half_t> {
  half8 v;
  __device__ __forceinline__ void load(const half_t* p) { v = *reinterpret_cast<const half8*>(p); }
  __device__ __forceinline__ float at(int j) const { return static_cast<float>(v[j]); }
};
template <>
struct Row8<float> {
  float4_t a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const float4_t*>(p);
    b = *reinterpret_cast<const float4_t*>(p + 4);
  }
  __device__ __forceinline__ float at(int j) const { return j < 4 ? a[j] : b[j - 4]; }
};


// Vectorised conv + SiLU: 8 consecutive channels per thread and a run of
// kConvRun tokens (taps <= 4; T4: taps == 4 known at compile time).  The
// run's kConvRun + 3 input rows are all requested before the first product,
// so a thread keeps that many 16-byte loads in flight; rows before token 0
// come from the f32 history.  Only the first run (t0 = 0) can reach before
// the history, so the others are compiled without the per-tap checks.
constexpr int kConvRun = 16;
template <class TI, class TO, bool T4>
__global__ __launch_bounds__(256) void conv_silu_vec_kernel(const TI* __restrict__ x, int64_t ldx,
                                                            const float* __restrict__ hist, int hrows,
                                                            const float* __restrict__ w, int taps_rt,
                                                            TO* __restrict__ y, int64_t ldy, int T, int W) {
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c0 >= W) return;
  const int taps = T4 ? 4 : taps_rt;
  const int t0 = blockIdx.y * kConvRun;
  constexpr int R = kConvRun + 3;
  Row8<TI> raw[R];  // raw[r]: token t0 - 3 + r
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int tp = t0 - 3 + r;
    if (tp >= 0 && tp < T) raw[r].load(x + (int64_t)tp * ldx + c0);
  }
  float hv[3][8];  // tokens -3..-1 (history rows hrows-3..hrows-1), zero before the history
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) hv[k][j] = 0.0f;
  if (t0 == 0) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int hr = hrows - 3 + k;
      if (hr >= 0)
#pragma unroll
        for (int j = 0; j < 8; ++j) hv[k][j] = hist[(int64_t)hr * W + c0 + j];
    }
  }
  // the thread's 8 x taps weights are contiguous: 16-byte loads when taps = 4
  float wt[8][4];
  if (taps == 4 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4_t q = *reinterpret_cast<const float4_t*>(w + (int64_t)(c0 + j) * 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) wt[j][k] = q[k];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) wt[j][k] = k < taps ? w[(int64_t)(c0 + j) * taps + k] : 0.0f;
  }
  auto run = [&](auto edge) {
    constexpr bool EDGE = decltype(edge)::value;
#pragma unroll
    for (int u = 0; u < kConvRun; ++u) {
      const int t = t0 + u;
      if (t >= T) break;
      TO out[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float acc = 0.0f;  // taps oldest -> newest, each product rounded before the add
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int tap = k - (4 - taps);  // slot k: delay 3-k, token t-3+k = raw[u + k]
          if (tap >= 0 && (!EDGE || hrows + t - (3 - k) >= 0)) {
            // token t-3+k < 0 only in the first run, at slots u + k < 3
            const float v = (EDGE && u + k < 3) ? hv[u + k < 3 ? u + k : 0][j] : raw[u + k].at(j);
            acc = add_rn(acc, mul_rn(v, wt[j][tap]));
          }
        }
        out[j] = cvt_out<TO>(silu_hw(acc));
      }
      TO* dst = y + (int64_t)t * ldy + c0;
      if (sizeof(TO) == 2) {
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = to_f16(out[j]);
        *reinterpret_cast<half8*>(dst) = h;
      } else {
        float4_t a, b;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = static_cast<float>(out[j]), b[j] = static_cast<float>(out[4 + j]);
        *reinterpret_cast<float4_t*>(dst) = a;
        *reinterpret_cast<float4_t*>(dst + 4) = b;
      }
    }
  };
  if (t0 == 0)
    run(std::true_type{});
  else
    run(std::false_type{});
}

// Sequence of packed token t: the last s with cu[s] <= t (cu has nseq + 1
// entries; any table gives an index in 0..nseq-1).
__device__ __forceinline__ int seq_of(const int* __restrict__ cu, int nseq, int t) {
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}
// First token of t's sequence, clamped into [0, t] (a no-op for a valid
// table; for any other, rows derived from it stay inside the batch).
__device__ __forceinline__ int seq_start(const int* __restrict__ cu, int nseq, int t) {
  return min(max(cu[seq_of(cu, nseq, t)], 0), t);
}

// Ragged batch of the vectorised conv: tokens cu[s] .. cu[s+1]-1 form sequence
// s, whose first taps-1 inputs come from its history rows (hist + s * hs, f32
// [hrows, W]).  The run's input rows are prefetched as in the single-sequence
// kernel; a run whose window lies inside one sequence takes the unchecked
// path, one that meets a sequence start resolves every tap's source (own
// token, history row or nothing).
template <class TI, class TO, bool T4>
__global__ __launch_bounds__(256) void conv_silu_varlen_kernel(const TI* __restrict__ x, int64_t ldx,
                                                               const float* __restrict__ hist, int hrows,
                                                               int64_t hs, const int* __restrict__ cu, int nseq,
                                                               const float* __restrict__ w, int taps_rt,
                                                               TO* __restrict__ y, int64_t ldy, int T, int W) {
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c0 >= W) return;
  const int taps = T4 ? 4 : taps_rt;
  const int t0 = blockIdx.y * kConvRun;
  const int t1 = min(t0 + kConvRun, T);
  constexpr int R = kConvRun + 3;
  // raw[r]: packed token t0 - 3 + r, the row index clamped into [0, T) so
  // every load is unconditional and all stay in flight together (loads under
  // per-row branches were each awaited before the next); rows outside the
  // batch are never used (the first run resolves its taps per token, and no
  // tap reads past the last token)
  Row8<TI> raw[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int tp = min(max(t0 - 3 + r, 0), T - 1);
    raw[r].load(x + (int64_t)tp * ldx + c0);
  }
  float wt[8][4];
  if (taps == 4 && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4_t q = *reinterpret_cast<const float4_t*>(w + (int64_t)(c0 + j) * 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) wt[j][k] = q[k];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) wt[j][k] = k < taps ? w[(int64_t)(c0 + j) * taps + k] : 0.0f;
  }
  int s = seq_of(cu, nseq, t0);
  const bool inside = cu[s] <= t0 - 3 && (s + 1 >= nseq || cu[s + 1] >= t1);
  auto store = [&](int t, const float (&o)[8]) {
    TO* dst = y + (int64_t)t * ldy + c0;
    if (sizeof(TO) == 2) {
      half8 h;
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = to_f16(o[j]);
      *reinterpret_cast<half8*>(dst) = h;
    } else {
      float4_t a, b;
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = o[j], b[j] = o[4 + j];
      *reinterpret_cast<float4_t*>(dst) = a;
      *reinterpret_cast<float4_t*>(dst + 4) = b;
    }
  };
  if (inside) {
#pragma unroll
    for (int u = 0; u < kConvRun; ++u) {
      if (t0 + u >= t1) break;
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float acc = 0.0f;  // taps oldest -> newest, each product rounded before the add
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int tap = k - (4 - taps);
          if (tap >= 0) acc = add_rn(acc, mul_rn(raw[u + k].at(j), wt[j][tap]));
        }
        o[j] = silu_hw(acc);
      }
      store(t0 + u, o);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < kConvRun; ++u) {
    const int t = t0 + u;
    if (t >= t1) break;
    while (s + 1 < nseq && cu[s + 1] <= t) ++s;
    // the sequence's first token clamped into [0, t]: a no-op for a valid
    // table, and for any other every row read below stays inside x or the
    // history rows
    const int start = min(max(cu[s], 0), t);
    // a delay reaching before the sequence's history contributes no term (as
    // the single-sequence kernel does before row 0)
    const int avail = hrows + (t - start);
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int tap = k - (4 - taps);
        const int tp = t - 3 + k;
        if (tap >= 0 && avail - (3 - k) >= 0) {
          // own tokens read again from x (L2-resident: the run's rows were
          // just loaded) rather than from raw[]: this loop stays rolled, and
          // indexing raw[] in it would put the array in scratch memory for
          // every run, the unchecked ones included
          const float v = tp >= start ? static_cast<float>(x[(int64_t)tp * ldx + c0 + j])
                                      : hist[(int64_t)s * hs + (int64_t)(hrows + tp - start) * W + c0 + j];
          acc = add_rn(acc, mul_rn(v, wt[j][tap]));
        }
      }
      o[j] = silu_hw(acc);
    }
    store(t, o);
  }
}

// Ragged batch, any layout: one (token, channel) per thread, the same tap
// order and roundings as conv_silu_kernel over [its sequence's history; its
// tokens].
__global__ __launch_bounds__(256) void conv_silu_varlen_scalar(const void* x, int64_t ldx, int dti,
                                                               const float* hist, int hrows, int64_t hs,
                                                               const int* __restrict__ cu, int nseq,
                                                               const float* w, int taps, void* y, int64_t ldy,
                                                               int dto, int T, int W) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * W) return;
  const int t = static_cast<int>(idx / W), c = static_cast<int>(idx % W);
  const int s = seq_of(cu, nseq, t);
  const int start = min(max(cu[s], 0), t);  // seq_start: as in the vectorised kernel
  float acc = 0.0f;
  for (int tap = 0; tap < taps; ++tap) {
    const int tp = t - (taps - 1 - tap);  // packed row of this delay
    const int hr = hrows + (tp - start);  // its row in [history; tokens]
    if (hr < 0) continue;
    float v;
    if (tp >= start && tp >= 0)
      v = ld(x, (int64_t)tp * ldx + c, dti);
    else if (hist)
      v = hist[(int64_t)s * hs + (int64_t)hr * W + c];
    else
      continue;
    acc = add_rn(acc, mul_rn(v, w[(int64_t)c * taps + tap]));
  }
  st(y, (int64_t)t * ldy + c, dto, acc / (1.0f + expf(-acc)));
}

// Row RMSNorm with the row held in registers: one wave per row, VPL values
// per lane at columns (i * 64 + lane) * 4 + j (width == 4 * 64 * (VPL/4)
// exactly).  rms_row_out reduces and writes a row that a kernel has loaded.
template <int VPL, class TO>
__device__ __forceinline__ void rms_row_out(const float* v, int lane, const float* __restrict__ w, TO* dst,
                                            float eps, float inv_width) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) s += v[i] * v[i];
  s = wave_sum(s);
  const float inverse = 1.0f / sqrtf(add_rn(mul_rn(s, inv_width), eps));
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) {
    const int c = (i * 64 + lane) * 4;
    const float4_t ww = *reinterpret_cast<const float4_t*>(w + c);
    float4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = mul_rn(mul_rn(v[i * 4 + j], inverse), ww[j]);
    if constexpr (sizeof(TO) == 2) {  // one 8-byte store of the four rounded values
      half4 h;
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = to_f16(o[j]);
      *reinterpret_cast<half4*>(dst + c) = h;
    } else {
      *reinterpret_cast<float4_t*>(dst + c) = o;
    }
  }
}

template <int VPL, class TO>
__global__ __launch_bounds__(256) void rms_f32_rows_kernel(const float* __restrict__ x, int64_t ldx,
                                                           const float* __restrict__ w, TO* __restrict__ y,
                                                           int64_t ldy, int rows, int width, float eps,
                                                           float inv_width) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float v[VPL];
  const float* src = x + (int64_t)row * ldx;
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) {
    const float4_t a = *reinterpret_cast<const float4_t*>(src + (i * 64 + lane) * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[i * 4 + j] = a[j];
  }
  rms_row_out<VPL, TO>(v, lane, w, y + (int64_t)row * ldy, eps, inv_width);
}

// Token embedding and the first layer's input norm in one pass (the rows of
// embed_vec_kernel, then rms_f32_rows_kernel's arithmetic on the same
// values): one wave per token writes its f32 residual row and its normalised
// row, so the residual is not read back.
template <int VPL, class TT, class TO>
__global__ __launch_bounds__(256) void embed_rms_kernel(const int32_t* __restrict__ ids, int T,
                                                        const TT* __restrict__ table, int vocab,
                                                        float* __restrict__ h, const float* __restrict__ w,
                                                        TO* __restrict__ y, int64_t ldy, float eps, float inv_width) {
  constexpr int H = VPL * 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T) return;
  const int id = min(max(ids[row], 0), vocab - 1);
  const TT* src = table + (int64_t)id * H;
  float* hrow = h + (int64_t)row * H;
  float v[VPL];
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) {
    const int c = (i * 64 + lane) * 4;
    float4_t a;
    if constexpr (sizeof(TT) == 2) {
      const half4 q = *reinterpret_cast<const half4*>(src + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = static_cast<float>(q[j]);
    } else {
      a = *reinterpret_cast<const float4_t*>(src + c);
    }
    *reinterpret_cast<float4_t*>(hrow + c) = a;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[i * 4 + j] = a[j];
  }
  rms_row_out<VPL, TO>(v, lane, w, y + (int64_t)row * ldy, eps, inv_width);
}

// Gated output norm for rows of 128: 16 lanes per row, 8 values per lane,
// kGatedRows rows per 16-lane group (rows g, g + 16, ... of the work-group's
// block; their o and z loads are requested before the first row is reduced).
// The kernel is bound by vector ALU work rather than bytes (16.8M elements
// per DeltaNet layer at T = 4096), so SiLU uses the hardware exp2 and
// reciprocal (silu_hw) instead of expf and an IEEE division.
constexpr int kGatedRows = 1;

template <class T8>
__device__ __forceinline__ void load8_f32(const T8* src, float* v) {
  if constexpr (sizeof(T8) == 2) {
    const half8 h = *reinterpret_cast<const half8*>(src);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(h[j]);
  } else {
    const float4_t a = *reinterpret_cast<const float4_t*>(src);
    const float4_t b = *reinterpret_cast<const float4_t*>(src + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = a[j], v[4 + j] = b[j];
  }
}

template <class TOI, class TZ, class TO>
__global__ __launch_bounds__(256) void gated_rms128_kernel(const TOI* __restrict__ o, const TZ* __restrict__ z,
                                                           int64_t ldz, const float* __restrict__ w,
                                                           TO* __restrict__ y, int T, int Hv, float eps) {
  const int rows = T * Hv;
  const int row0 = blockIdx.x * (16 * kGatedRows) + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const int c = sub * 8;
  const bool half_out = sizeof(TO) == 2;
  // a 16-lane group shares its row, so a group is active or inactive as a
  // whole and the shuffles below stay inside active groups
  float v[kGatedRows][8], zf[kGatedRows][8];
#pragma unroll
  for (int k = 0; k < kGatedRows; ++k) {
    const int row = row0 + 16 * k;
    if (row < rows) {
      const int t = row / Hv, h = row % Hv;
      load8_f32(o + (int64_t)row * 128 + c, v[k]);
      load8_f32(z + (int64_t)t * ldz + (int64_t)h * 128 + c, zf[k]);
    }
  }
  float wv[8];
  load8_f32(w + c, wv);
#pragma unroll
  for (int k = 0; k < kGatedRows; ++k) {
    const int row = row0 + 16 * k;
    if (row >= rows) break;
    if (half_out) {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[k][j] = static_cast<float>(to_f16(v[k][j]));
    }
    // explicit fused steps: the compiler would otherwise contract some
    // products into their sums, differently for f16 and f32 o
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s = __builtin_fmaf(v[k][j], v[k][j], s);
    s = sum16(s);
    const float inverse = 1.0f / sqrtf(add_rn(mul_rn(s, 1.0f / 128.0f), eps));
    TO out[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float n = mul_rn(mul_rn(v[k][j], inverse), wv[j]);
      if (half_out) n = static_cast<float>(to_f16(n));
      out[j] = cvt_out<TO>(mul_rn(n, silu_hw(zf[k][j])));
    }
    TO* dst = y + (int64_t)row * 128 + c;
#pragma unroll
    for (int j = 0; j < 8; ++j) dst[j] = out[j];
  }
}

// ---- SwiGLU product, the unfused form of the f16 GEMM epilogue ---------------
// f16: y = half(half(silu(g)) * u) with g, u f16 values (the product of two
// f16 values is exact in f32, so y is rounded once); f32: silu(g) * u with
// expf and an IEEE division, as the f32 epilogue.
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* g, const void* u, void* y, int64_t n, int dt) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float gv = ld(g, i, dt), uv = ld(u, i, dt);
  if (dt == CLEF_F16)
    st(y, i, dt, static_cast<float>(to_f16(silu_hw(gv))) * uv);
  else
    st(y, i, dt, (gv / (1.0f + expf(-gv))) * uv);
}

// ---- decay and write strength (qwen.rs:619-627) -----------------------------
__global__ __launch_bounds__(256) void gates_kernel(const void* a, int64_t lda, const void* b,
                                                    int64_t ldb, int dti, const float* dt,
                                                    const float* alog, float* g, float* beta, int T,
                                                    int Hv) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= T * Hv) return;
  const int t = idx / Hv, h = idx % Hv;
  g[idx] = delta_decay(ld(a, (int64_t)t * lda + h, dti), dt[h], alog[h]);
  beta[idx] = delta_strength(ld(b, (int64_t)t * ldb + h, dti));
}

// ---- gated output norm (qwen.rs:671-676): one wave per (token, head) row ----
__global__ __launch_bounds__(256) void gated_rms_kernel(const void* o, int dto_in, const void* z, int64_t ldz,
                                                        int dtz, const float* w, void* y, int dto,
                                                        int T, int Hv, int width, float eps,
                                                        float inv_width) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= T * Hv) return;
  const int t = row / Hv, h = row % Hv;
  float s = 0.0f;
  for (int i = lane; i < width; i += 64) {
    const float v = rnd(ld(o, (int64_t)row * width + i, dto_in), dto);
    s = __builtin_fmaf(v, v, s);
  }
  s = wave_sum(s);
  const float inverse = 1.0f / sqrtf(add_rn(mul_rn(s, inv_width), eps));
  for (int i = lane; i < width; i += 64) {
    const float v = rnd(ld(o, (int64_t)row * width + i, dto_in), dto);
    const float n = rnd(mul_rn(mul_rn(v, inverse), w[i]), dto);
    const float zv = ld(z, (int64_t)t * ldz + (int64_t)h * width + i, dtz);
    st(y, (int64_t)row * width + i, dto, mul_rn(n, silu_hw(zv)));
  }
}

// ---- q/k head norm + rotary, head-major output (qwen.rs:437-470) ------------
struct RotaryTable {
  float inv_freq[128];
};

// cos and sin of position p times one inverse frequency (ops.rs:165-188):
// the angle rounded once in f32, then the library cosf / sinf
__device__ __forceinline__ void rotary_angle(float p, float inv_freq, float& c, float& s) {
  const float ang = mul_rn(p, inv_freq);
  c = cosf(ang);
  s = sinf(ang);
}

__global__ __launch_bounds__(256) void qk_norm_rotary_kernel(const void* x, int64_t ldx, int64_t hs,
                                                             int dti, const float* w, void* y,
                                                             int64_t ldy_tok, int dto, int T,
                                                             int heads, int d, int rot, int pos0,
                                                             int dst_offset, float eps,
                                                             float inv_width, RotaryTable tab,
                                                             const int* __restrict__ cu, int nseq) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);  // (t, head)
  const int lane = threadIdx.x & 63;
  if (row >= T * heads) return;
  const int t = row / heads, h = row % heads;
  const int64_t src = (int64_t)t * ldx + (int64_t)h * hs;
  float s = 0.0f;
  for (int i = lane; i < d; i += 64) {
    const float v = ld(x, src + i, dti);
    s += v * v;
  }
  s = wave_sum(s);
  const float inverse = 1.0f / sqrtf(add_rn(mul_rn(s, inv_width), eps));
  const int half = rot / 2;
  // position: pos0 + t, or pos0 + (t - first token of t's sequence)
  const float p = static_cast<float>(pos0 + (cu ? t - seq_start(cu, nseq, t) : t));
  const int64_t dst = ((int64_t)h * ldy_tok + dst_offset + t) * d;
  for (int i = lane; i < d; i += 64) {
    const float v = rnd(mul_rn(mul_rn(ld(x, src + i, dti), inverse), w[i]), dto);
    float out = v;
    if (i < rot) {
      const int j = i < half ? i + half : i - half;
      const float vj = rnd(mul_rn(mul_rn(ld(x, src + j, dti), inverse), w[j]), dto);
      const float r = i < half ? -vj : vj;
      const float ang = mul_rn(p, tab.inv_freq[i % half]);
      out = add_rn(mul_rn(v, cosf(ang)), mul_rn(r, sinf(ang)));
    }
    st(y, dst + i, dto, out);
  }
}

// One token per work-group (four waves, heads h = wave, wave + 4, ...), each
// lane holding EPL = d / 64 consecutive features: the rotation's cos and sin
// are computed once per token and frequency (shared by every head, as the
// pair i, i + rot/2 shares its angle), rows are read and written as vectors,
// and a rotated feature's partner comes from the lane rot / (2 EPL) away.
// Same per-element roundings as qk_norm_rotary_kernel; the squares are
// summed per lane over consecutive features, then across the wave.
template <int EPL, class TI, class TO>
__global__ __launch_bounds__(256) void qk_norm_rotary_tok(const TI* __restrict__ x, int64_t ldx, int64_t hs,
                                                          const float* __restrict__ w, TO* __restrict__ y,
                                                          int64_t ldy_tok, int heads, int rot, int pos0,
                                                          int dst_offset, float eps, float inv_width, int vec,
                                                          RotaryTable tab, const int* __restrict__ cu, int nseq,
                                                          float2* __restrict__ tab_out, int T) {
  constexpr int D = 64 * EPL;
  // one token per wave (four per work-group): its angles, then all its heads
  __shared__ float cs_all[4][128], sn_all[4][128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = 4 * blockIdx.x + wave;
  if (t >= T) return;  // whole waves; no barrier below
  float* const cs = cs_all[wave];
  float* const sn = sn_all[wave];
  const int half = rot / 2;
  // position: pos0 + t, or pos0 + (t - first token of t's sequence)
  const float p = static_cast<float>(pos0 + (cu ? t - seq_start(cu, nseq, t) : t));
  for (int f = lane; f < half; f += 64) {
    rotary_angle(p, tab.inv_freq[f], cs[f], sn[f]);
    if (tab_out) tab_out[(int64_t)t * half + f] = make_float2(cs[f], sn[f]);
  }
  // the wave's own LDS writes complete before its reads below (in order)
  __builtin_amdgcn_wave_barrier();
  const int i0 = lane * EPL;
  const int pd = half / EPL;  // partner lane distance
  float wv[EPL], cw[EPL], sw[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int i = i0 + e;
    wv[e] = w[i];
    const int f = i < half ? i : i - half;
    cw[e] = i < rot ? cs[f] : 1.0f;
    sw[e] = i < rot ? (i < half ? -sn[f] : sn[f]) : 0.0f;  // r = -v[i + half] below half, v[i - half] above
  }
  for (int h = 0; h < heads; ++h) {
    const TI* src = x + (int64_t)t * ldx + (int64_t)h * hs + i0;
    float v[EPL];
    bool got = false;
    if constexpr (EPL == 4) {
      if (vec) {
        if constexpr (sizeof(TI) == 2) {
          const half4 q = *reinterpret_cast<const half4*>(src);
#pragma unroll
          for (int e = 0; e < EPL; ++e) v[e] = static_cast<float>(q[e]);
        } else {
          const float4_t q = *reinterpret_cast<const float4_t*>(src);
#pragma unroll
          for (int e = 0; e < EPL; ++e) v[e] = q[e];
        }
        got = true;
      }
    }
    if (!got)
#pragma unroll
      for (int e = 0; e < EPL; ++e) v[e] = static_cast<float>(src[e]);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss += v[e] * v[e];
    ss = wave_sum(ss);
    const float inverse = 1.0f / sqrtf(add_rn(mul_rn(ss, inv_width), eps));
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      v[e] = static_cast<float>(cvt_out<TO>(mul_rn(mul_rn(v[e], inverse), wv[e])));
    const int plane = i0 < half ? lane + pd : (i0 < rot ? lane - pd : lane);
    TO out[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float vj = __shfl(v[e], plane, 64);
      out[e] = cvt_out<TO>(i0 + e < rot ? add_rn(mul_rn(v[e], cw[e]), mul_rn(vj, sw[e])) : v[e]);
    }
    TO* dst = y + ((int64_t)h * ldy_tok + dst_offset + t) * D + i0;
    bool done = false;
    if constexpr (EPL == 4) {
      if (vec) {
        if constexpr (sizeof(TO) == 2)
          *reinterpret_cast<half4*>(dst) = half4{out[0], out[1], out[2], out[3]};
        else
          *reinterpret_cast<float4_t*>(dst) = float4_t{out[0], out[1], out[2], out[3]};
        done = true;
      }
    }
    if (!done)
#pragma unroll
      for (int e = 0; e < EPL; ++e) dst[e] = out[e];
  }
}

// ---- values to [heads, d, tokens] --------------------------------------------
__global__ __launch_bounds__(256) void values_t_kernel(const void* x, int64_t ldx, int dti, void* y,
                                                       int64_t ldy_tok, int dto, int T, int heads,
                                                       int d, int dst_offset) {
  // tile of 64 tokens x 64 features per block, transposed through LDS
  __shared__ float tile[64][65];
  const int h = blockIdx.z, t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int t = t0 + r, e = e0 + tx;
    tile[r][tx] = (t < T && e < d) ? ld(x, (int64_t)t * ldx + (int64_t)h * d + e, dti) : 0.0f;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int e = e0 + r, t = t0 + tx;
    if (t < T && e < d) st(y, ((int64_t)h * d + e) * ldy_tok + dst_offset + t, dto, tile[tx][r]);
  }
}

// f16 in and out, d a multiple of 64, 16-byte aligned rows: a 64-token x
// 64-feature tile moves as 16-byte vectors (8 features of a token in, 8
// tokens of a feature out) through an LDS tile; the last group of a partial
// tile is stored element by element.
__global__ __launch_bounds__(256) void values_t_f16_kernel(const half_t* __restrict__ x, int64_t ldx,
                                                           half_t* __restrict__ y, int64_t ldy_tok, int T, int d,
                                                           int dst_offset) {
  __shared__ __attribute__((aligned(16))) half_t tile[64][72];  // [token][feature], padded rows
  const int h = blockIdx.z, t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = threadIdx.x + 256 * k;
    const int r = i >> 3, c = (i & 7) * 8;
    const int t = min(t0 + r, T - 1);
    *reinterpret_cast<half8*>(&tile[r][c]) = *reinterpret_cast<const half8*>(x + (int64_t)t * ldx + (int64_t)h * d + e0 + c);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = threadIdx.x + 256 * k;
    const int e = i >> 3, t8 = (i & 7) * 8;
    if (t0 + t8 >= T) continue;
    half8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = tile[t8 + j][e];
    half_t* dst = y + ((int64_t)h * d + e0 + e) * ldy_tok + dst_offset + t0 + t8;
    if (t0 + t8 + 8 <= T) {
      *reinterpret_cast<half8*>(dst) = v;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (t0 + t8 + j < T) dst[j] = v[j];
    }
  }
}

// ---- embedding gather and pooled head ---------------------------------------
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* ids, int T, const void* table, int dt,
                                                    int vocab, int H, float* h) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * H) return;
  const int t = static_cast<int>(idx / H), c = static_cast<int>(idx % H);
  const int id = min(max(ids[t], 0), vocab - 1);  // ids are validated by the caller
  h[idx] = ld(table, (int64_t)id * H + c, dt);
}

// 8 consecutive features per thread: one 16-byte (f16) or two 16-byte (f32)
// row loads and two 16-byte stores
template <class TT>
__global__ __launch_bounds__(256) void embed_vec_kernel(const int32_t* __restrict__ ids, int T,
                                                        const TT* __restrict__ table, int vocab, int H,
                                                        float* __restrict__ h) {
  const int per_row = H / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * per_row) return;
  const int t = static_cast<int>(idx / per_row), c = static_cast<int>(idx % per_row) * 8;
  const int id = min(max(ids[t], 0), vocab - 1);
  const TT* src = table + (int64_t)id * H + c;
  float4_t a, b;
  if constexpr (sizeof(TT) == 2) {
    const half8 v = *reinterpret_cast<const half8*>(src);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = static_cast<float>(v[j]), b[j] = static_cast<float>(v[4 + j]);
  } else {
    a = *reinterpret_cast<const float4_t*>(src);
    b = *reinterpret_cast<const float4_t*>(src + 4);
  }
  float* dst = h + (int64_t)t * H + c;
  *reinterpret_cast<float4_t*>(dst) = a;
  *reinterpret_cast<float4_t*>(dst + 4) = b;
}

__global__ __launch_bounds__(64) void head_kernel(const float* x, int H, const float* w, float* logits) {
  const int j = blockIdx.x, lane = threadIdx.x;
  float s = 0.0f;
  for (int i = lane; i < H; i += 64) s += x[i] * w[(int64_t)j * H + i];
  s = wave_sum(s);
  if (lane == 0) logits[j] = s;
}

bool dtype_ok(int d) { return d == CLEF_F32 || d == CLEF_F16; }

}  // namespace
}  // namespace clef

using namespace clef;

extern "C" int clef_rms_norm(const void* x, int64_t ldx, int dtype_in, const float* w, void* y,
                             int64_t ldy, int dtype_out, int rows, int width, float eps,
                             void* stream) {
  if (ldx == 0) ldx = width;
  if (ldy == 0) ldy = width;
  CLEF_REQUIRE(x && w && y, "RMS: null pointer");
  CLEF_REQUIRE(rows >= 1 && width >= 1 && ldx >= width && ldy >= width, "RMS: dimensions");
  CLEF_REQUIRE(dtype_ok(dtype_in) && dtype_ok(dtype_out), "RMS: dtype");
  CLEF_REQUIRE(eps > 0.0f && eps <= 1.0f, "RMS: epsilon");
  const float inv_w = static_cast<float>(1.0 / static_cast<double>(width));
  // (4-element vector loads of x and w, 4-element stores of y)
  const bool vec = dtype_in == CLEF_F32 && ldx % 4 == 0 && ldy % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                     reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  if (vec && (width == 2048 || width == 1024)) {
    const dim3 g((rows + 3) / 4);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float* xf = static_cast<const float*>(x);
    if (width == 2048) {
      if (dtype_out == CLEF_F16)
        hipLaunchKernelGGL((rms_f32_rows_kernel<32, half_t>), g, dim3(256), 0, st, xf, ldx, w,
                           static_cast<half_t*>(y), ldy, rows, width, eps, inv_w);
      else
        hipLaunchKernelGGL((rms_f32_rows_kernel<32, float>), g, dim3(256), 0, st, xf, ldx, w,
                           static_cast<float*>(y), ldy, rows, width, eps, inv_w);
    } else {
      if (dtype_out == CLEF_F16)
        hipLaunchKernelGGL((rms_f32_rows_kernel<16, half_t>), g, dim3(256), 0, st, xf, ldx, w,
                           static_cast<half_t*>(y), ldy, rows, width, eps, inv_w);
      else
        hipLaunchKernelGGL((rms_f32_rows_kernel<16, float>), g, dim3(256), 0, st, xf, ldx, w,
                           static_cast<float*>(y), ldy, rows, width, eps, inv_w);
    }
    return check_launch("rms_norm");
  }
  hipLaunchKernelGGL(rms_kernel, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, x, ldx,
                     dtype_in, w, y, ldy, dtype_out, rows, width, eps,
                     static_cast<float>(1.0 / static_cast<double>(width)));
  return check_launch("rms_norm");
}

extern "C" int clef_conv_silu(const void* x, int64_t ldx, int dtype_in, const float* history,
                              int history_rows, const float* w, int taps, void* y, int64_t ldy,
                              int dtype_out, int T, int W, void* stream) {
  if (ldx == 0) ldx = W;
  if (ldy == 0) ldy = W;
  CLEF_REQUIRE(x && w && y, "conv: null pointer");
  CLEF_REQUIRE(T >= 1 && W >= 1 && ldx >= W && ldy >= W, "conv: dimensions");
  CLEF_REQUIRE(taps >= 1 && taps <= 8 && history_rows >= 0 && history_rows <= taps - 1 &&
                   (history_rows == 0 || history),
               "conv: taps or history");
  CLEF_REQUIRE(dtype_ok(dtype_in) && dtype_ok(dtype_out), "conv: dtype");
  const bool vec = taps <= 4 && W % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  if (vec) {
    const dim3 g((W / 8 + 255) / 256, (T + kConvRun - 1) / kConvRun);
    hipStream_t st = static_cast<hipStream_t>(stream);
#define CLEF_CONV_VEC(TI, TO, T4)                                                                       \
  hipLaunchKernelGGL((conv_silu_vec_kernel<TI, TO, T4>), g, dim3(256), 0, st, static_cast<const TI*>(x), ldx, \
                     history, history_rows, w, taps, static_cast<TO*>(y), ldy, T, W)
#define CLEF_CONV_VEC_T(TI, TO)    \
  if (taps == 4)                   \
    CLEF_CONV_VEC(TI, TO, true);   \
  else                             \
    CLEF_CONV_VEC(TI, TO, false)
    if (dtype_in == CLEF_F16 && dtype_out == CLEF_F16) {
      CLEF_CONV_VEC_T(half_t, half_t);
    } else if (dtype_in == CLEF_F16) {
      CLEF_CONV_VEC_T(half_t, float);
    } else if (dtype_out == CLEF_F16) {
      CLEF_CONV_VEC_T(float, half_t);
    } else {
      CLEF_CONV_VEC_T(float, float);
    }
#undef CLEF_CONV_VEC_T
#undef CLEF_CONV_VEC
    return check_launch("conv_silu");
  }
  const int64_t n = (int64_t)T * W;
  hipLaunchKernelGGL(conv_silu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, dtype_in, history, history_rows, w, taps, y, ldy,
                     dtype_out, T, W);
  return check_launch("conv_silu");
}

extern "C" int clef_conv_silu_varlen(const void* x, int64_t ldx, int dtype_in, const float* history,
                                     int history_rows, int64_t history_stride, const int32_t* cu_seqlens,
                                     int nseq, const float* w, int taps, void* y, int64_t ldy, int dtype_out,
                                     int T, int W, void* stream) {
  if (ldx == 0) ldx = W;
  if (ldy == 0) ldy = W;
  CLEF_REQUIRE(x && w && y && cu_seqlens && nseq >= 1, "conv: null pointer or no sequences");
  CLEF_REQUIRE(T >= 1 && W >= 1 && ldx >= W && ldy >= W, "conv: dimensions");
  CLEF_REQUIRE(taps >= 1 && taps <= 8 && history_rows >= 0 && history_rows <= taps - 1 &&
                   (history_rows == 0 || history) && history_stride >= 0,
               "conv: taps or history");
  CLEF_REQUIRE(dtype_ok(dtype_in) && dtype_ok(dtype_out), "conv: dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!(taps <= 4 && W % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(y) & 15) == 0)) {
    const int64_t n = (int64_t)T * W;
    hipLaunchKernelGGL(conv_silu_varlen_scalar, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, ldx,
                       dtype_in, history, history_rows, history_stride, cu_seqlens, nseq, w, taps, y, ldy, dtype_out,
                       T, W);
    return check_launch("conv_silu_varlen");
  }
  const dim3 g((W / 8 + 255) / 256, (T + kConvRun - 1) / kConvRun);
#define CLEF_CONV_VL4(TI, TO, T4)                                                                              \
  hipLaunchKernelGGL((conv_silu_varlen_kernel<TI, TO, T4>), g, dim3(256), 0, st, static_cast<const TI*>(x), ldx, \
                     history, history_rows, history_stride, cu_seqlens, nseq, w, taps, static_cast<TO*>(y), ldy,     \
                     T, W)
#define CLEF_CONV_VL(TI, TO)      \
  if (taps == 4)                  \
    CLEF_CONV_VL4(TI, TO, true);  \
  else                            \
    CLEF_CONV_VL4(TI, TO, false)
  if (dtype_in == CLEF_F16 && dtype_out == CLEF_F16) {
    CLEF_CONV_VL(half_t, half_t);
  } else if (dtype_in == CLEF_F16) {
    CLEF_CONV_VL(half_t, float);
  } else if (dtype_out == CLEF_F16) {
    CLEF_CONV_VL(float, half_t);
  } else {
    CLEF_CONV_VL(float, float);
  }
#undef CLEF_CONV_VL
#undef CLEF_CONV_VL4
  return check_launch("conv_silu_varlen");
}

extern "C" int clef_delta_gates(const void* a, int64_t lda, const void* b, int64_t ldb, int dtype_in,
                                const float* dt, const float* a_log, float* g, float* beta, int T,
                                int Hv, void* stream) {
  if (lda == 0) lda = Hv;
  if (ldb == 0) ldb = Hv;
  CLEF_REQUIRE(a && b && dt && a_log && g && beta, "gates: null pointer");
  CLEF_REQUIRE(T >= 1 && Hv >= 1 && lda >= Hv && ldb >= Hv, "gates: dimensions");
  CLEF_REQUIRE(dtype_ok(dtype_in), "gates: dtype");
  hipLaunchKernelGGL(gates_kernel, dim3((T * Hv + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     a, lda, b, ldb, dtype_in, dt, a_log, g, beta, T, Hv);
  return check_launch("delta_gates");
}

extern "C" int clef_silu_mul(const void* gate, const void* up, void* y, int64_t n, int dtype, void* stream) {
  CLEF_REQUIRE(gate && up && y, "silu_mul: null pointer");
  // (one element per thread: at most 2^31 - 1 work-groups of 256)
  CLEF_REQUIRE(n >= 1 && n <= int64_t(0x7fffffff) * 256 && dtype_ok(dtype), "silu_mul: size or dtype");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, gate, up,
                     y, n, dtype);
  return check_launch("silu_mul");
}

extern "C" int clef_gated_rms_silu(const void* o, int dtype_o, const void* z, int64_t ldz, int dtype_z,
                                   const float* w, void* y, int dtype_out, int T, int Hv, int width,
                                   float eps, void* stream) {
  if (ldz == 0) ldz = (int64_t)Hv * width;
  CLEF_REQUIRE(o && z && w && y, "gated norm: null pointer");
  CLEF_REQUIRE(T >= 1 && Hv >= 1 && width >= 1 && ldz >= (int64_t)Hv * width, "gated norm: dimensions");
  CLEF_REQUIRE(dtype_ok(dtype_o) && dtype_ok(dtype_z) && dtype_ok(dtype_out), "gated norm: dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (width == 128 && ldz % 8 == 0 &&
      ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(w)) & 15) == 0) {
    const dim3 g((T * Hv + 16 * kGatedRows - 1) / (16 * kGatedRows));
#define CLEF_GRMS(TOI, TZ, TO)                                                                                   \
  hipLaunchKernelGGL((gated_rms128_kernel<TOI, TZ, TO>), g, dim3(256), 0, st, static_cast<const TOI*>(o),      \
                     static_cast<const TZ*>(z), ldz, w, static_cast<TO*>(y), T, Hv, eps)
#define CLEF_GRMS_O(TZ, TO)        \
  if (dtype_o == CLEF_F16)         \
    CLEF_GRMS(half_t, TZ, TO);     \
  else                             \
    CLEF_GRMS(float, TZ, TO)
    if (dtype_z == CLEF_F16 && dtype_out == CLEF_F16) {
      CLEF_GRMS_O(half_t, half_t);
    } else if (dtype_z == CLEF_F16) {
      CLEF_GRMS_O(half_t, float);
    } else if (dtype_out == CLEF_F16) {
      CLEF_GRMS_O(float, half_t);
    } else {
      CLEF_GRMS_O(float, float);
    }
#undef CLEF_GRMS_O
#undef CLEF_GRMS
    return check_launch("gated_rms_silu");
  }
  hipLaunchKernelGGL(gated_rms_kernel, dim3((T * Hv + 3) / 4), dim3(256), 0, st, o, dtype_o, z, ldz, dtype_z, w,
                     y, dtype_out, T, Hv, width, eps, static_cast<float>(1.0 / static_cast<double>(width)));
  return check_launch("gated_rms_silu");
}

// per-token kernel when d is 64, 128 or 256 and the rotary half splits into
// whole lanes; false if not taken (nothing launched)
static bool qk_norm_rotary_tok_launch(const void* x, int64_t ldx, int64_t hs, int dti, const float* w, void* y,
                                      int64_t ldy_tok, int dto, int T, int heads, int d, int rot, int pos0,
                                      int dst_offset, float eps, const RotaryTable& tab, const int* cu, int nseq,
                                      hipStream_t st, float2* tab_out = nullptr) {
  const int epl = d / 64;
  if (d % 64 != 0 || !(epl == 1 || epl == 2 || epl == 4) || (rot / 2) % epl != 0) return false;
  const int es_in = dti == CLEF_F16 ? 2 : 4, es_out = dto == CLEF_F16 ? 2 : 4;
  const int vec = (reinterpret_cast<uintptr_t>(x) % (es_in * epl) == 0 && (ldx * es_in) % (es_in * epl) == 0 &&
                   (hs * es_in) % (es_in * epl) == 0 && reinterpret_cast<uintptr_t>(y) % (es_out * epl) == 0)
                      ? 1
                      : 0;
  const float inv = static_cast<float>(1.0 / static_cast<double>(d));
#define CLEF_QKR(E, TI, TO)                                                                                     \
  hipLaunchKernelGGL((qk_norm_rotary_tok<E, TI, TO>), dim3((T + 3) / 4), dim3(256), 0, st,                     \
                     static_cast<const TI*>(x), ldx, hs, w, static_cast<TO*>(y), ldy_tok, heads, rot, pos0, dst_offset, \
                     eps, inv, vec, tab, cu, nseq, tab_out, T)
#define CLEF_QKR_E(TI, TO)      \
  if (epl == 4)                 \
    CLEF_QKR(4, TI, TO);        \
  else if (epl == 2)            \
    CLEF_QKR(2, TI, TO);        \
  else                          \
    CLEF_QKR(1, TI, TO)
  if (dti == CLEF_F16 && dto == CLEF_F16) {
    CLEF_QKR_E(half_t, half_t);
  } else if (dti == CLEF_F16) {
    CLEF_QKR_E(half_t, float);
  } else if (dto == CLEF_F16) {
    CLEF_QKR_E(float, half_t);
  } else {
    CLEF_QKR_E(float, float);
  }
#undef CLEF_QKR_E
#undef CLEF_QKR
  return true;
}

extern "C" int clef_qk_norm_rotary(const void* x, int64_t ldx, int64_t hs, int dtype_in, const float* w,
                                   void* y, int64_t ldy_tok, int dtype_out, int T, int heads, int d,
                                   int rot_dim, double theta, int pos0, int dst_offset, float eps,
                                   void* stream) {
  if (hs == 0) hs = d;
  if (ldx == 0) ldx = (int64_t)heads * hs;
  CLEF_REQUIRE(x && w && y, "q/k norm: null pointer");
  CLEF_REQUIRE(T >= 1 && heads >= 1 && d >= 1 && hs >= d && ldx >= (int64_t)(heads - 1) * hs + d,
               "q/k norm: dimensions");
  CLEF_REQUIRE(rot_dim >= 0 && rot_dim <= d && rot_dim % 2 == 0 && rot_dim / 2 <= 128,
               "q/k norm: rotary width");
  CLEF_REQUIRE(dst_offset >= 0 && ldy_tok >= (int64_t)dst_offset + T && pos0 >= 0, "q/k norm: destination");
  CLEF_REQUIRE(dtype_ok(dtype_in) && dtype_ok(dtype_out), "q/k norm: dtype");
  RotaryTable tab{};
  for (int i = 0; i < rot_dim / 2; ++i)  // ops.rs:165: theta.powf(-(2i)/dim) in f64, then f32
    tab.inv_freq[i] = static_cast<float>(std::pow(theta, -static_cast<double>(2 * i) / rot_dim));
  if (qk_norm_rotary_tok_launch(x, ldx, hs, dtype_in, w, y, ldy_tok, dtype_out, T, heads, d, rot_dim, pos0,
                                dst_offset, eps, tab, nullptr, 0, static_cast<hipStream_t>(stream)))
    return check_launch("qk_norm_rotary");
  hipLaunchKernelGGL(qk_norm_rotary_kernel, dim3((T * heads + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, hs, dtype_in, w, y, ldy_tok, dtype_out, T, heads, d,
                     rot_dim, pos0, dst_offset, eps, static_cast<float>(1.0 / static_cast<double>(d)),
                     tab, nullptr, 0);
  return check_launch("qk_norm_rotary");
}

extern "C" int clef_qk_norm_rotary_varlen(const void* x, int64_t ldx, int64_t hs, int dtype_in, const float* w,
                                          void* y, int64_t ldy_tok, int dtype_out, int T, int heads, int d,
                                          int rot_dim, double theta, int pos0, const int32_t* cu_seqlens,
                                          int nseq, int dst_offset, float eps, void* stream) {
  if (hs == 0) hs = d;
  if (ldx == 0) ldx = (int64_t)heads * hs;
  CLEF_REQUIRE(x && w && y && cu_seqlens && nseq >= 1, "q/k norm: null pointer or no sequences");
  CLEF_REQUIRE(T >= 1 && heads >= 1 && d >= 1 && hs >= d && ldx >= (int64_t)(heads - 1) * hs + d,
               "q/k norm: dimensions");
  CLEF_REQUIRE(rot_dim >= 0 && rot_dim <= d && rot_dim % 2 == 0 && rot_dim / 2 <= 128,
               "q/k norm: rotary width");
  CLEF_REQUIRE(dst_offset >= 0 && ldy_tok >= (int64_t)dst_offset + T && pos0 >= 0, "q/k norm: destination");
  CLEF_REQUIRE(dtype_ok(dtype_in) && dtype_ok(dtype_out), "q/k norm: dtype");
  RotaryTable tab{};
  for (int i = 0; i < rot_dim / 2; ++i)
    tab.inv_freq[i] = static_cast<float>(std::pow(theta, -static_cast<double>(2 * i) / rot_dim));
  if (qk_norm_rotary_tok_launch(x, ldx, hs, dtype_in, w, y, ldy_tok, dtype_out, T, heads, d, rot_dim, pos0,
                                dst_offset, eps, tab, cu_seqlens, nseq, static_cast<hipStream_t>(stream)))
    return check_launch("qk_norm_rotary");
  hipLaunchKernelGGL(qk_norm_rotary_kernel, dim3((T * heads + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, hs, dtype_in, w, y, ldy_tok, dtype_out, T, heads, d,
                     rot_dim, pos0, dst_offset, eps, static_cast<float>(1.0 / static_cast<double>(d)),
                     tab, cu_seqlens, nseq);
  return check_launch("qk_norm_rotary");
}

// (cos, sin) of positions pos0 + t for the rot / 2 rotary frequencies, as
// float2 rows [T][rot / 2]: the values the per-token q/k kernel rotates by.
__global__ __launch_bounds__(64) void rotary_table_kernel(RotaryTable tab, int half, int pos0, float2* __restrict__ out) {
  const int t = blockIdx.x;
  const float p = static_cast<float>(pos0 + t);
  for (int f = threadIdx.x; f < half; f += 64) {
    float c, s;
    rotary_angle(p, tab.inv_freq[f], c, s);
    out[(int64_t)t * half + f] = make_float2(c, s);
  }
}

namespace clef {
// The key norm + rotary of the single-sequence attention layer, also writing
// the (cos, sin) rows of its positions to tab_out ([T][rot / 2] float2) for
// the attention core's fused query preparation (f16 in and out; the
// per-token kernel's shapes: an error, before any launch, elsewhere).
int qk_norm_rotary_table_launch(const void* x, int64_t ldx, int64_t hs, const float* w, void* y, int64_t ldy_tok,
                                int T, int heads, int d, int rot, double theta, int pos0, int dst_offset, float eps,
                                float* tab_out, hipStream_t st) {
  CLEF_REQUIRE(x && w && y && tab_out && T >= 1 && heads >= 1 && rot >= 2 && rot <= d && rot % 2 == 0 &&
                   rot / 2 <= 128 && hs >= d && ldy_tok >= (int64_t)dst_offset + T && pos0 >= 0,
               "q/k norm with rotary table: arguments");
  RotaryTable tab{};
  for (int i = 0; i < rot / 2; ++i)  // ops.rs:165, as clef_qk_norm_rotary
    tab.inv_freq[i] = static_cast<float>(std::pow(theta, -static_cast<double>(2 * i) / rot));
  if (!qk_norm_rotary_tok_launch(x, ldx, hs, CLEF_F16, w, y, ldy_tok, CLEF_F16, T, heads, d, rot, pos0, dst_offset,
                                 eps, tab, nullptr, 0, st, reinterpret_cast<float2*>(tab_out)))
    return fail(-1, "q/k norm with rotary table: d must be 64, 128 or 256 with whole lanes of the rotary half");
  return check_launch("qk_norm_rotary");
}
}  // namespace clef

extern "C" int clef_rotary_table(int T, int rot_dim, double theta, int pos0, float* out, void* stream) {
  CLEF_REQUIRE(out, "rotary table: null pointer");
  CLEF_REQUIRE(T >= 1 && rot_dim >= 2 && rot_dim % 2 == 0 && rot_dim / 2 <= 128 && pos0 >= 0,
               "rotary table: dimensions");
  RotaryTable tab{};
  for (int i = 0; i < rot_dim / 2; ++i)  // ops.rs:165, as clef_qk_norm_rotary
    tab.inv_freq[i] = static_cast<float>(std::pow(theta, -static_cast<double>(2 * i) / rot_dim));
  hipLaunchKernelGGL(rotary_table_kernel, dim3(T), dim3(64), 0, (hipStream_t)stream, tab, rot_dim / 2, pos0,
                     reinterpret_cast<float2*>(out));
  return check_launch("rotary_table");
}

extern "C" int clef_values_transposed(const void* x, int64_t ldx, int dtype_in, void* y, int64_t ldy_tok,
                                      int dtype_out, int T, int heads, int d, int dst_offset,
                                      void* stream) {
  if (ldx == 0) ldx = (int64_t)heads * d;
  CLEF_REQUIRE(x && y, "values: null pointer");
  CLEF_REQUIRE(T >= 1 && heads >= 1 && d >= 1 && ldx >= (int64_t)heads * d, "values: dimensions");
  CLEF_REQUIRE(dst_offset >= 0 && ldy_tok >= (int64_t)dst_offset + T, "values: destination");
  CLEF_REQUIRE(dtype_ok(dtype_in) && dtype_ok(dtype_out), "values: dtype");
  const bool vec = dtype_in == CLEF_F16 && dtype_out == CLEF_F16 && d % 64 == 0 && ldx % 8 == 0 &&
                   ldy_tok % 8 == 0 && dst_offset % 8 == 0 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(values_t_f16_kernel, dim3((T + 63) / 64, d / 64, heads), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const half_t*>(x), ldx, static_cast<half_t*>(y), ldy_tok, T, d, dst_offset);
  else
    hipLaunchKernelGGL(values_t_kernel, dim3((T + 63) / 64, (d + 63) / 64, heads), dim3(256), 0,
                       (hipStream_t)stream, x, ldx, dtype_in, y, ldy_tok, dtype_out, T, heads, d, dst_offset);
  return check_launch("values_transposed");
}

extern "C" int clef_embed(const int32_t* ids, int T, const void* table, int dtype, int vocab, int H,
                          float* h, void* stream) {
  CLEF_REQUIRE(ids && table && h, "embed: null pointer");
  CLEF_REQUIRE(T >= 1 && vocab >= 1 && H >= 1 && dtype_ok(dtype), "embed: dimensions");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (H % 8 == 0 && ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(h)) & 15) == 0) {
    const int64_t n = (int64_t)T * (H / 8);
    const dim3 g((unsigned)((n + 255) / 256));
    if (dtype == CLEF_F16)
      hipLaunchKernelGGL(embed_vec_kernel<half_t>, g, dim3(256), 0, st, ids, T, static_cast<const half_t*>(table),
                         vocab, H, h);
    else
      hipLaunchKernelGGL(embed_vec_kernel<float>, g, dim3(256), 0, st, ids, T, static_cast<const float*>(table),
                         vocab, H, h);
    return check_launch("embed");
  }
  const int64_t n = (int64_t)T * H;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, ids, T, table, dtype,
                     vocab, H, h);
  return check_launch("embed");
}

namespace clef {
bool embed_rms_applies(const void* table, int H, const float* h, const float* w, const void* y, int64_t ldy) {
  return (H == 2048 || H == 1024) && ldy >= H && ldy % 4 == 0 &&
         ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(w) |
           reinterpret_cast<uintptr_t>(y)) & 15) == 0;
}

// Embedding + first input norm (embed_rms_kernel), for the shapes
// embed_rms_applies accepts.
int embed_rms_launch(const int32_t* ids, int T, const void* table, int dtype_table, int vocab, int H, float* h,
                     const float* w, void* y, int64_t ldy, int dtype_out, float eps, hipStream_t st) {
  CLEF_REQUIRE(ids && table && h && w && y && T >= 1 && vocab >= 1, "embed+norm: arguments");
  CLEF_REQUIRE(embed_rms_applies(table, H, h, w, y, ldy), "embed+norm: shape or alignment");
  CLEF_REQUIRE(dtype_ok(dtype_table) && dtype_ok(dtype_out), "embed+norm: dtype");
  const float inv_w = static_cast<float>(1.0 / static_cast<double>(H));
  const dim3 g((T + 3) / 4);
#define CLEF_EMBED_RMS(VPL, TT, TO)                                                                       \
  hipLaunchKernelGGL((embed_rms_kernel<VPL, TT, TO>), g, dim3(256), 0, st, ids, T, static_cast<const TT*>(table), \
                     vocab, h, w, static_cast<TO*>(y), ldy, eps, inv_w)
#define CLEF_EMBED_RMS_T(VPL)                                              \
  if (dtype_table == CLEF_F16 && dtype_out == CLEF_F16) {                  \
    CLEF_EMBED_RMS(VPL, half_t, half_t);                                   \
  } else if (dtype_table == CLEF_F16) {                                    \
    CLEF_EMBED_RMS(VPL, half_t, float);                                    \
  } else if (dtype_out == CLEF_F16) {                                      \
    CLEF_EMBED_RMS(VPL, float, half_t);                                    \
  } else {                                                                 \
    CLEF_EMBED_RMS(VPL, float, float);                                     \
  }
  if (H == 2048) {
    CLEF_EMBED_RMS_T(32)
  } else {
    CLEF_EMBED_RMS_T(16)
  }
#undef CLEF_EMBED_RMS_T
#undef CLEF_EMBED_RMS
  return check_launch("embed_rms");
}
}  // namespace clef

extern "C" int clef_head_logits(const float* x, int H, const float* w, int n_logits, float* logits,
                                void* stream) {
  CLEF_REQUIRE(x && w && logits && H >= 1 && n_logits >= 1 && n_logits <= 65536, "head: arguments");
  hipLaunchKernelGGL(head_kernel, dim3(n_logits), dim3(64), 0, (hipStream_t)stream, x, H, w, logits);
  return check_launch("head_logits");
}
