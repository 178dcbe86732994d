// Projection GEMMs y = x . W^T for gfx950 (x [M,K], W [N,K], both K-contiguous).
//
// Replaces the reference's tile GEMM (crates/core/src/models/neural.metal:7-125,
// dispatch neural.rs:201-280) and candle_nn::Linear (projection.rs:82-95).
//
// Design: one work-group of 4 waves (2 x 2) computes a BM x BN tile with
// v_mfma_f32_32x32x16_f16 (f16 operands) or v_mfma_f32_32x32x2_f32 (f32
// operands), accumulating in f32.  K advances in BK steps through a double
// buffered LDS stage (rows padded by 16 bytes so the 16-byte fragment reads of
// 32 consecutive rows hit distinct bank groups); the next stage's global loads
// are issued before the current stage's MFMAs so they overlap.  The tile
// index is remapped so that each XCD (blockIdx % 8) works on a compact band of
// tiles, which keeps the shared x rows and W rows in that XCD's L2.
//
// f32 operands: each BK = 32 stage is accumulated in a fresh accumulator and
// then added to the running sum, which cuts the rounding error of a K = 6144
// dot product roughly fourfold against one accumulator chain over all of K
// (that is what keeps the f32 profile within 1e-5 of an exactly accumulated
// product at the block shape); the second accumulator set caps f32 tiles at
// 256 x 128.
//
// Epilogues: store (f16 rounded once from the f32 accumulator, or f32);
// residual (h += to_f32(round(acc)), the residual add of qwen.rs:399-410);
// SwiGLU (silu(gate) * up with the half roundings of neural.metal:29-44).
#include "common.hpp"
#include "gemm.hpp"

namespace clef {
namespace {

template <class T> struct Mma32;
template <> struct Mma32<half_t> {
  typedef half8 frag;
  static constexpr int kBlock = 16;
  static __device__ __forceinline__ void mma(float16_t& c, const frag& a, const frag& b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mma32<float> {
  typedef float4_t frag;
  static constexpr int kBlock = 8;
  static __device__ __forceinline__ void mma(float16_t& c, const frag& a, const frag& b) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[3], b[3], c, 0, 0, 0);
  }
};

template <class T> struct V16;
template <> struct V16<half_t> { typedef half8 type; };
template <> struct V16<float> { typedef float4_t type; };

__device__ __forceinline__ float round_to(float v, int dtype) {
  return dtype == 1 ? static_cast<float>(static_cast<half_t>(v)) : v;
}

// EPI: 0 store, 1 residual add into f32 y, 2 SwiGLU (B rows = [gate tile | up tile]).
template <class T, int BM, int BN, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
  constexpr int BK = 128 / sizeof(T);          // 64 halves or 32 floats: 128-byte rows
  constexpr int VE = 16 / sizeof(T);           // elements per 16-byte vector
  constexpr int LDS_ROW = BK + VE;             // padded row (elements)
  constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
  constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 MFMA tiles per wave
  constexpr int KB = Mma32<T>::kBlock;
  constexpr int NKB = BK / KB;
  constexpr int ROWS_PER_PASS = 256 / (BK / VE);  // 32 rows per 256-thread pass
  constexpr int PA = BM / ROWS_PER_PASS, PB = BN / ROWS_PER_PASS;
  typedef typename Mma32<T>::frag frag;
  typedef typename V16<T>::type vec;

  __shared__ __attribute__((aligned(16))) T sA[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) T sB[2][BN * LDS_ROW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- tile index with XCD-compact placement
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (EPI == 2 ? (p.N + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN);
  const int ntiles = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
  // walk groups of 4 tile-rows so consecutive t share W columns and x rows
  const int group = 4;
  const int gsize = group * tiles_n;
  const int gid = t / gsize;
  const int first_m = gid * group;
  const int gm = min(group, tiles_m - first_m);
  const int tm = first_m + (t % gsize) % gm;
  const int tn = (t % gsize) / gm;
  const int m0 = tm * BM;
  const int n0 = tn * (EPI == 2 ? BN / 2 : BN);

  const T* X = static_cast<const T*>(p.x);
  const T* W = static_cast<const T*>(p.w);
  const T* W2 = static_cast<const T*>(p.w2);

  // global -> register staging for one BK slice
  vec ra[PA], rb[PB];
  const int lrow = tid / (BK / VE);        // row within a pass
  const int lcol = (tid % (BK / VE)) * VE;  // element column within BK
  // Rows are clamped into the matrices (results of clamped rows are never
  // stored); columns beyond K are zeroed when staged.  With p.vec the rows
  // are 16-byte aligned and K % VE == 0, otherwise elements load one by one.
  auto load_vec = [&](const T* row, int k) -> vec {
    if (p.vec) return *reinterpret_cast<const vec*>(row + min(k, p.K - VE));
    vec v;
#pragma unroll
    for (int e = 0; e < VE; ++e) v[e] = row[min(k + e, p.K - 1)];
    return v;
  };
  auto load_stage = [&](int k0) {
    const int kc = k0 + lcol;
#pragma unroll
    for (int i = 0; i < PA; ++i) {
      const int r = min(m0 + i * ROWS_PER_PASS + lrow, p.M - 1);
      ra[i] = load_vec(X + (int64_t)r * p.ldx, kc);
    }
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const int br = i * ROWS_PER_PASS + lrow;
      const T* src;
      if (EPI == 2) {  // wave column wb holds [gate | up] rows of the same outputs
        const int wb = br / WN, within = br % WN;
        const int nr = min(n0 + wb * (WN / 2) + (within % (WN / 2)), p.N - 1);
        src = (within >= WN / 2 ? W2 : W) + (int64_t)nr * p.ldw;
      } else {
        src = W + (int64_t)min(n0 + br, p.N - 1) * p.ldw;
      }
      rb[i] = load_vec(src, kc);
    }
  };
  auto mask_k = [&](vec v, int k) -> vec {
    if (k + VE <= p.K) return v;
#pragma unroll
    for (int e = 0; e < VE; ++e)
      if (k + e >= p.K) v[e] = T(0);
    return v;
  };
  auto store_stage = [&](int buf, int k0) {
    const int kc = k0 + lcol;
#pragma unroll
    for (int i = 0; i < PA; ++i)
      *reinterpret_cast<vec*>(&sA[buf][(i * ROWS_PER_PASS + lrow) * LDS_ROW + lcol]) = mask_k(ra[i], kc);
#pragma unroll
    for (int i = 0; i < PB; ++i)
      *reinterpret_cast<vec*>(&sB[buf][(i * ROWS_PER_PASS + lrow) * LDS_ROW + lcol]) = mask_k(rb[i], kc);
  };

  constexpr bool kSplit = sizeof(T) == 4;  // per-stage accumulation (f32 operands)
  static_assert(!kSplit || TM * TN <= 8, "f32 tiles of at most 256 x 128: two accumulator sets");
  float16_t acc[TM][TN], tot[kSplit ? TM : 1][kSplit ? TN : 1];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  if constexpr (kSplit)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) tot[i][j][e] = 0.0f;

  const int nk = (p.K + BK - 1) / BK;
  load_stage(0);
  store_stage(0, 0);
  lds_barrier();
  const int frow = lane & 31, fk = (lane >> 5) * VE;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_stage((kt + 1) * BK);
    const T* a_base = &sA[buf][(wm * WM + frow) * LDS_ROW + fk];
    const T* b_base = &sB[buf][(wn * WN + frow) * LDS_ROW + fk];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      frag af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const frag*>(a_base + i * 32 * LDS_ROW + kb * KB);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const frag*>(b_base + j * 32 * LDS_ROW + kb * KB);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) Mma32<T>::mma(acc[i][j], af[i], bf[j]);
    }
    if constexpr (kSplit) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          tot[i][j] += acc[i][j];
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        }
    }
    if (kt + 1 < nk) {
      store_stage(buf ^ 1, (kt + 1) * BK);
      lds_barrier();
    }
  }
  if constexpr (kSplit)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = tot[i][j];

  // ---- epilogue.  acc[i][j][e]: row (e/4)*8 + (lane/32)*4 + e%4, col lane%32
  const int ccol = lane & 31, rgrp = (lane >> 5) * 4;
  if (EPI == 2) {
    // wave column wn: gate cols wn*WN/2 .. +WN/2 (tiles j < TN/2), up cols in j >= TN/2
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN / 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = m0 + wm * WM + i * 32 + (e >> 2) * 8 + rgrp + (e & 3);
          const int c = n0 + wn * (WN / 2) + j * 32 + ccol;
          if (r < p.M && c < p.N) {
            float out;
            if (p.dtype_out == 1) {  // half roundings of neural.metal:35-42 (SiLU as gemm_f16.hip's)
              const float g = static_cast<float>(to_f16(acc[i][j][e]));
              const float s = static_cast<float>(to_f16(silu_hw(g)));
              out = s * static_cast<float>(to_f16(acc[i][j + TN / 2][e]));
            } else {
              const float g = acc[i][j][e];
              out = (g / (1.0f + expf(-g))) * acc[i][j + TN / 2][e];
            }
            const int64_t o = (int64_t)r * p.ldy + c;
            if (p.dtype_out == 1)
              static_cast<half_t*>(p.y)[o] = static_cast<half_t>(out);
            else
              static_cast<float*>(p.y)[o] = out;
          }
        }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = m0 + wm * WM + i * 32 + (e >> 2) * 8 + rgrp + (e & 3);
        const int c = n0 + wn * WN + j * 32 + ccol;
        if (r < p.M && c < p.N) {
          const int64_t o = (int64_t)r * p.ldy + c;
          const float v = acc[i][j][e];
          if (EPI == 1) {
            float* y = static_cast<float*>(p.y);
            y[o] = y[o] + round_to(v, p.dtype_out);
          } else if (p.dtype_out == 1) {
            static_cast<half_t*>(p.y)[o] = static_cast<half_t>(v);
          } else {
            static_cast<float*>(p.y)[o] = v;
          }
        }
      }
}

template <class T, int BM, int BN, int EPI>
int launch_tile(const GemmParams& p, hipStream_t s) {
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = EPI == 2 ? (p.N + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_kernel<T, BM, BN, EPI>), dim3(tiles_m * tiles_n), dim3(256), 0, s, p);
  return check_launch("gemm");
}

// Tile choice: minimise (waves of 256 work-groups) x (tile area), preferring
// the larger tile on ties (more reuse per byte).
template <class T, int EPI>
int launch_epi(const GemmParams& p, hipStream_t s) {
  const int ncu = 256;
  const int n_eff = EPI == 2 ? 2 * p.N : p.N;
  auto cost = [&](int bm, int bn) {
    const long tiles = (long)((p.M + bm - 1) / bm) * ((n_eff + bn - 1) / bn);
    return ((tiles + ncu - 1) / ncu) * (long)bm * bn;
  };
  const long c256 = cost(256, 256), c128 = cost(128, 128), c_mid = cost(256, 128);
  if constexpr (sizeof(T) == 2)
    if (c256 <= c128 && c256 <= c_mid) return launch_tile<T, 256, 256, EPI>(p, s);
  if (c_mid <= c128) return launch_tile<T, 256, 128, EPI>(p, s);
  return launch_tile<T, 128, 128, EPI>(p, s);
}

}  // namespace

int gemm_launch(const GemmParams& p, int epilogue, hipStream_t s) {
  if (gemm_f16_dma_ok(p)) return gemm_f16_dma_launch(p, epilogue, s);
  if (p.dtype_in == 1) {
    if (epilogue == 0) return launch_epi<half_t, 0>(p, s);
    if (epilogue == 1) return launch_epi<half_t, 1>(p, s);
    return launch_epi<half_t, 2>(p, s);
  }
  if (epilogue == 0) return launch_epi<float, 0>(p, s);
  if (epilogue == 1) return launch_epi<float, 1>(p, s);
  return launch_epi<float, 2>(p, s);
}

}  // namespace clef
