// Shared device helpers for the gfx950 kernels: element conversion, MFMA
// fragments, error plumbing.  Wavefronts are 64 lanes.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace clef {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ---- scalar conversions --------------------------------------------------
template <class T> __device__ __forceinline__ float to_f32(T x) { return static_cast<float>(x); }
template <class T> __device__ __forceinline__ T from_f32(float x) { return static_cast<T>(x); }

// ---- MFMA fragments ------------------------------------------------------
// A fragment is 16 bytes per lane covering one "k-block" of a 16x16 tile:
//   f16: 8 halves, k-block of 32, one v_mfma_f32_16x16x32_f16;
//   f32: 4 floats, k-block of 16, four v_mfma_f32_16x16x4_f32.
// Operands are stored K-contiguous ([rows][K]).  Lane l supplies row l%16
// and the 16 bytes at byte offset 16*(l/16) of the k-block, for both A and B
// (B given as [N][K]); for f32 the four floats of a lane feed four MFMAs
// whose k index is 4*(l/16)+s, a permutation of k applied to both operands.
// The accumulator layout is that of the hardware: lane l holds rows
// 4*(l/16)+i (i = 0..3) of column l%16.
template <class T> struct Mma;

template <> struct Mma<half_t> {
  typedef half8 frag;
  static constexpr int kBlock = 32;
  static __device__ __forceinline__ void mma(float4_t& c, const frag& a, const frag& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mma<float> {
  typedef float4_t frag;
  static constexpr int kBlock = 16;
  static __device__ __forceinline__ void mma(float4_t& c, const frag& a, const frag& b) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  }
};

template <class T>
__device__ __forceinline__ typename Mma<T>::frag load_frag(const T* p) {
  return *reinterpret_cast<const typename Mma<T>::frag*>(p);
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over each row of 16 lanes with DPP moves (no LDS round trips): lane
// partners xor 1 and xor 2 (quad permutes), then the half-row and row
// mirrors, which pair the same quads and halves as xor 4 and xor 8.  Each
// step adds a value to its partner's, so every lane of a row ends with the
// same bits, summed in the association of an xor butterfly.
template <int CTRL>
__device__ __forceinline__ float dpp_partner(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// The same over groups of N = 2, 4, 8, 16 or 32 consecutive lanes (32: the
// two rows meet through one lane shuffle).
template <int N>
__device__ __forceinline__ float lane_sum(float v) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32, "2..32 lanes");
  if constexpr (N >= 2) v += dpp_partner<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v += dpp_partner<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp_partner<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp_partner<0x140>(v);  // row_mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
  return v;
}
__device__ __forceinline__ float sum16(float v) { return lane_sum<16>(v); }
// Maximum over groups of N = 2, 4, 8 or 16 consecutive lanes, by the same moves.
template <int N>
__device__ __forceinline__ float lane_max(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "2..16 lanes");
  if constexpr (N >= 2) v = fmaxf(v, dpp_partner<0xB1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp_partner<0x4E>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp_partner<0x141>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp_partner<0x140>(v));
  return v;
}

// Work-group barrier for LDS producer/consumer hand-offs only.  Unlike
// __syncthreads() it does not wait for outstanding global loads, so register
// prefetches issued before it stay in flight across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// f32 multiply and add, each rounded on its own.  HIP's __fmul_rn and
// __fadd_rn are plain operators, which the compiler still contracts into an
// FMA or folds into a following f16 conversion (v_fma_mixlo_f16: one rounding
// where the reference rounds twice); contraction is off inside these.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// f32 -> f16, round to nearest even, of the f32 value as rounded.  The empty
// asm keeps the compiler from folding a producing multiply into the
// conversion (v_fma_mixlo_f16 rounds the exact product once).
__device__ __forceinline__ half_t to_f16(float x) {
  asm("" : "+v"(x));
  return static_cast<half_t>(x);
}
template <class T>
__device__ __forceinline__ T cvt_out(float x) {
  if constexpr (sizeof(T) == 2)
    return to_f16(x);
  else
    return x;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
// SiLU with the hardware exp2 and reciprocal: x / (1 + e^-x) to a relative
// error of about 1e-6 (the argument's rounding, |x| log2(e) ulp, dominates);
// a few instructions where expf and an IEEE division take about thirty.
__device__ __forceinline__ float silu_hw(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
// sigmoid on the same hardware exp2 and reciprocal
__device__ __forceinline__ float sigmoid_hw(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// DeltaNet gates (qwen.rs:615-623): decay g = softplus(a + dt) * -exp(A_log)
// with the stable softplus max(x, 0) + log(1 + exp(-|x|)), strength
// beta = sigmoid(b); f32 throughout, each step rounded as written.
__device__ __forceinline__ float delta_decay(float a, float dt, float alog) {
  const float av = add_rn(a, dt);
  const float sp = add_rn(fmaxf(av, 0.0f), logf(add_rn(expf(-fabsf(av)), 1.0f)));
  return mul_rn(sp, -expf(alog));
}
__device__ __forceinline__ float delta_strength(float b) { return 1.0f / (1.0f + expf(-b)); }

// ---- host-side error plumbing ---------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);  // records msg, returns code
int check_launch(const char* what);          // hipGetLastError -> 0 or >0

// Token embedding fused with the first layer's input RMSNorm (pointwise.hip):
// writes the f32 residual rows h [T, H] and the normalised rows y (ldy apart).
// embed_rms_applies: whether the shape and alignment are on its path (H 1024
// or 2048, 16-byte aligned rows); elsewhere callers run clef_embed and
// clef_rms_norm.
bool embed_rms_applies(const void* table, int H, const float* h, const float* w, const void* y, int64_t ldy);
int embed_rms_launch(const int32_t* ids, int T, const void* table, int dtype_table, int vocab, int H, float* h,
                     const float* w, void* y, int64_t ldy, int dtype_out, float eps, hipStream_t st);

// Key norm + rotary (f16) that also writes the (cos, sin) rows of positions
// pos0 .. pos0 + T - 1 to tab_out ([T][rot / 2] float2) for the attention
// core's fused query path (pointwise.hip); an error, nothing launched, off
// the per-token kernel's shapes.
int qk_norm_rotary_table_launch(const void* x, int64_t ldx, int64_t hs, const float* w, void* y, int64_t ldy_tok,
                                int T, int heads, int d, int rot, double theta, int pos0, int dst_offset, float eps,
                                float* tab_out, hipStream_t st);

}  // namespace clef

#define CLEF_REQUIRE(cond, msg)                              \
  do {                                                       \
    if (!(cond)) return ::clef::fail(-1, std::string(msg));  \
  } while (0)
