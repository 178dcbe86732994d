// Chunked gated-DeltaNet scan for gfx950: kernels and launchers.
//
// Semantics: delta_recurrence_prefill (crates/core/src/models/qwen.rs:826-882)
// with repeat-interleave GQA (qwen.rs:727-738); chunkwise algebra as in
// crates/core/src/models/chunk.metal:10-164, restated for C = 64.
//
// For one v-head and a chunk of C tokens with in-chunk cumulative log-decay
// gam_r = sum_{j<=r} g_j (padding rows have g = 0, beta = 0, k = q = 0),
// with k^, q^ the normalised keys and scaled normalised queries:
//   A[r][c] = beta_r (k^_r.k^_c) exp(gam_r - gam_c)  (c < r);  Tm = (I + A)^-1
//   M[r][c] = (q^_r.k^_c) exp(gam_r - gam_c)          (c <= r)
//   W       = diag(exp(gam_last - gam))
//   U       = K^^T W Tm diag(beta) (dk x C)
//   N       = M Tm diag(beta)      (C x C)
//   Y       = V - diag(exp gam) K^ S
//   O       = diag(exp gam) Q^ S + N Y
//   S'      = exp(gam_last) S + U Y
// Decay ratios are only formed for c <= r, so g = -1000 underflows to exact
// zeros instead of dividing by an underflowed prefix product.
//
// scan_prepare (grid chunks x Hk, fully parallel) does everything that does
// not depend on the state and writes it as MFMA operand blocks (64 lanes x
// 16 bytes, in the order the consumer's lanes read them): K^ and Q^ of the
// k-head, then per v-head the scalars, U and N.  (I + A)^-1 is formed in f32:
// 16x16 diagonal blocks by forward substitution, the rest by block forward
// substitution on MFMA.
//
// scan_carry (grid Hv x ceil(dv/16)) runs the chunks in order for one v-head
// and 16 value columns (the columns of S evolve independently):
//   wave 0  the recurrence X = K^ S, Y, S' = el S + U Y.  S stays in MFMA
//           accumulators and re-enters the next product as an operand
//           without leaving the registers (see slot_index);
//   wave 1  loads K^, U and the scalars of chunk i+2 into a 3-slot LDS ring
//           with global->LDS DMA (2 slots for f32 operands);
//   waves 2-3  O of chunk i-1 from the S and Y wave 0 hands over in LDS.
// One barrier per chunk.  Work-groups sharing a k-head are placed on one XCD
// so its rows come from that XCD's L2.
#pragma once
#include "common.hpp"
#include "scan.hpp"

namespace clef {
namespace {

constexpr int kC = 64;   // chunk length
constexpr int kVT = 16;  // value columns per carry work-group

template <class T> struct Vec16;  // 16-byte vector of T
template <> struct Vec16<float> { typedef float4_t type; static constexpr int n = 4; };
template <> struct Vec16<half_t> { typedef half8 type; static constexpr int n = 8; };

// Tile geometry for compute dtype CT and padded key width DK.
template <class CT, int DK> struct Geo {
  static constexpr int EPF = 16 / sizeof(CT);   // elements per lane fragment
  static constexpr int KB = Mma<CT>::kBlock;    // k-block of one fragment
  static constexpr int TPK = KB / 16;           // accumulator tiles per k-block
  static constexpr int NKX = DK / KB;           // k-blocks over dk
  static constexpr int NKT = kC / KB;           // k-blocks over the chunk
  static constexpr int NST = DK / 16;           // 16-row tiles of the state
  static constexpr int NBK = 4 * NKX;           // blocks of K^ (or Q^) per chunk
  static constexpr int NBU = NST * NKT;         // blocks of U per chunk
  static constexpr int NBN = 4 * NKT;           // blocks of N per chunk
};

// Index held by row slot m (0..15) of 16-row tile t of a dimension.  f32
// fragments (k-block 16): 16t + m.  f16 fragments (k-block 32): tiles pair
// up and slot m of tile 2b+u is 32b + 8(m/4) + 4u + m%4, so the slots
// 4g..4g+3 of tiles 2b and 2b+1 that one lane holds in an accumulator are
// the 8 consecutive indices 32b+8g.. of the k-block fragment of lane group
// g.  Accumulator tiles therefore become MFMA operands in place.
template <class CT>
__device__ __forceinline__ int slot_index(int t, int m) {
  if constexpr (sizeof(CT) == 4)
    return 16 * t + m;
  else
    return 32 * (t >> 1) + 8 * (m >> 2) + 4 * (t & 1) + (m & 3);
}

// k-block fragment kb from accumulator tiles (the view slot_index sets up).
__device__ __forceinline__ float4_t pack_frag(const float4_t* acc, int kb, float) { return acc[kb]; }
__device__ __forceinline__ half8 pack_frag(const float4_t* acc, int kb, half_t) {
  const float4_t a = acc[2 * kb], b = acc[2 * kb + 1];
  half8 f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = static_cast<half_t>(a[i]);
    f[4 + i] = static_cast<half_t>(b[i]);
  }
  return f;
}

// EPF consecutive f32 values times a scale (and optional per-element
// weights) as a CT fragment.
__device__ __forceinline__ float4_t frag_from_f32(const float* x, const float* w, float scale, float) {
  float4_t a = *reinterpret_cast<const float4_t*>(x) * scale;
  if (w) a = a * *reinterpret_cast<const float4_t*>(w);
  return a;
}
__device__ __forceinline__ half8 frag_from_f32(const float* x, const float* w, float scale, half_t) {
  float4_t a = *reinterpret_cast<const float4_t*>(x) * scale;
  float4_t b = *reinterpret_cast<const float4_t*>(x + 4) * scale;
  if (w) {
    a = a * *reinterpret_cast<const float4_t*>(w);
    b = b * *reinterpret_cast<const float4_t*>(w + 4);
  }
  half8 f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = static_cast<half_t>(a[i]);
    f[4 + i] = static_cast<half_t>(b[i]);
  }
  return f;
}

// Branch-free row loader: VI elements e0..e0+VI-1 of a row, addresses clamped
// into the row (so every access is valid), in the input dtype.
template <class IT>
__device__ __forceinline__ typename Vec16<IT>::type load_row_raw(const IT* row, int e0, int dk,
                                                                bool vec_ok) {
  constexpr int VI = Vec16<IT>::n;
  typename Vec16<IT>::type v;
  if (vec_ok) {  // dk % VI == 0 and 16-byte aligned rows
    v = *reinterpret_cast<const typename Vec16<IT>::type*>(row + min(e0, dk - VI));
  } else {
#pragma unroll
    for (int i = 0; i < VI; ++i) v[i] = row[min(e0 + i, dk - 1)];
  }
  return v;
}

__device__ __forceinline__ uint32_t load_bits(const void* p, int64_t i, int dtype) {
  return dtype == 0 ? static_cast<const uint32_t*>(p)[i] : static_cast<const uint16_t*>(p)[i];
}

__device__ __forceinline__ float bits_to_f32(uint32_t b, int dtype) {
  if (dtype == 0) return __uint_as_float(b);
  const uint16_t h = static_cast<uint16_t>(b);
  return static_cast<float>(*reinterpret_cast<const half_t*>(&h));
}

// e^x for decay factors: hardware 2^x (1 ulp) of x log2(e).  Callers pass
// differences of cumulative log-decays, formed before scaling so they keep
// full precision; results below the normal range may flush to zero.
__device__ __forceinline__ float decay_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Raw buffer access with out-of-range offsets: a load at kOOB returns 0 and a
// store there is dropped, so masked rows and columns need no branches.
constexpr int kOOB = 0x7ffffff0;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// 32-bit register holding one element's bits (f16 in the low half), so the
// compiler never packs two prefetched halves into one register.
template <class T> __device__ __forceinline__ uint32_t buffer_load_bits(__amdgpu_buffer_rsrc_t r, int off);
template <> __device__ __forceinline__ uint32_t buffer_load_bits<float>(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
template <> __device__ __forceinline__ uint32_t buffer_load_bits<half_t>(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <class T> __device__ __forceinline__ float bits_value(uint32_t b);
template <> __device__ __forceinline__ float bits_value<float>(uint32_t b) { return __uint_as_float(b); }
template <> __device__ __forceinline__ float bits_value<half_t>(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(b)));
}
__device__ __forceinline__ void buffer_store(__amdgpu_buffer_rsrc_t r, int off, float v, float) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
}
__device__ __forceinline__ void buffer_store(__amdgpu_buffer_rsrc_t r, int off, float v, half_t) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, static_cast<half_t>(v)), r, off, 0, 0);
}

// One 1 KiB operand block global -> LDS: lane l copies the 16 bytes at
// src + 16 l to lds + 16 l (lds is the wave-uniform block base).
__device__ __forceinline__ void dma_block(const void* src_lane, void* lds_block) {
  __builtin_amdgcn_global_load_lds(src_lane, lds_block, 16, 0, 0);
}

// ---------------------------------------------------------------------------
// Token span of chunk c (ragged batches: from the chunk table; false past
// its last chunk).
__device__ __forceinline__ bool chunk_span(const ScanParams& p, int c, int& t0, int& n) {
  if (p.chunk_tab) {
    if (c >= *p.nchunk_total) return false;
    const int2 e = p.chunk_tab[c];
    t0 = e.x;
    n = e.y;
  } else {
    t0 = c * kC;
    n = min(kC, p.T - t0);
  }
  return true;
}

// Token span of chunk c in the carry, with the batch kind known at compile
// time (one sequence: no table lookups on the recurrence's path).
template <bool VL>
__device__ __forceinline__ void chunk_at(const ScanParams& p, int c, int& t0, int& n) {
  if constexpr (VL) {
    const int2 e = p.chunk_tab[c];
    t0 = e.x;
    n = e.y;
  } else {
    t0 = c * kC;
    n = min(kC, p.T - t0);
  }
}

// ---------------------------------------------------------------------------
// Conv prologue (ScanParams::mixed): the mixer's causal conv + SiLU computed
// where its outputs are consumed, in the separate conv kernel's order and
// roundings (taps oldest -> newest, each product and sum rounded, hardware
// SiLU, the result rounded to the input dtype), so the scan sees the same q,
// k and v values.

// Sequence of token t and its first token (one sequence: 0 and 0).
__device__ __forceinline__ void conv_sequence(const ScanParams& p, int t, int& seq, int& start) {
  seq = 0;
  start = 0;
  if (!p.cu_seqlens) return;
  int lo = 0, hi = p.nseq - 1;  // the last s with cu_seqlens[s] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.cu_seqlens[mid] <= t)
      lo = mid;
    else
      hi = mid - 1;
  }
  seq = lo;
  start = p.cu_seqlens[lo];
}

// Channels ch .. ch+VI-1 of token tp: a row of `mixed` (clamped to `last`,
// the chunk's last token) from the sequence start on, before it the
// sequence's history rows, before those zero (a zero product added to the
// running sum leaves it unchanged, as skipping the tap does).
template <class IT>
__device__ __forceinline__ void conv_load(const ScanParams& p, int tp, int last, int seq, int start, int ch,
                                          float* x) {
  constexpr int VI = Vec16<IT>::n;
  if (tp >= start) {
    const IT* row = static_cast<const IT*>(p.mixed) + (int64_t)min(tp, last) * p.ld_mixed + ch;
    const typename Vec16<IT>::type v = *reinterpret_cast<const typename Vec16<IT>::type*>(row);
#pragma unroll
    for (int i = 0; i < VI; ++i) x[i] = static_cast<float>(v[i]);
    return;
  }
  const int hr = p.hist_rows + (tp - start);
  if (p.conv_hist && hr >= 0) {
    const float* h = p.conv_hist + (int64_t)seq * p.hist_stride + (int64_t)hr * p.conv_channels + ch;
#pragma unroll
    for (int i = 0; i < VI; ++i) x[i] = h[i];
  } else {
#pragma unroll
    for (int i = 0; i < VI; ++i) x[i] = 0.0f;
  }
}

// RPT consecutive rows (chunk rows r0 .. r0+RPT-1) of VI channels from ch:
// y[j][i] = round_IT(silu(sum_tap x[t-3+tap] w[tap])); rows past the chunk's
// n tokens and inactive lanes give 0.
template <class IT, int RPT>
__device__ __forceinline__ void conv_rows(const ScanParams& p, int t0, int n, int r0, int seq, int start, int ch,
                                          bool active, float (*y)[Vec16<IT>::n]) {
  constexpr int VI = Vec16<IT>::n;
  float w[VI][4];
  float xr[RPT + 3][VI];
  if (active) {
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const float4_t w4 = *reinterpret_cast<const float4_t*>(p.conv_w + (int64_t)(ch + i) * 4);
#pragma unroll
      for (int tap = 0; tap < 4; ++tap) w[i][tap] = w4[tap];
    }
#pragma unroll
    for (int k = 0; k < RPT + 3; ++k) conv_load<IT>(p, t0 + r0 + k - 3, t0 + n - 1, seq, start, ch, xr[k]);
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      float acc = 0.0f;
#pragma unroll
      for (int tap = 0; tap < 4; ++tap) acc = add_rn(acc, mul_rn(xr[j + tap][i], w[i][tap]));
      const float v = silu_hw(acc);
      y[j][i] = (active && r0 + j < n) ? (sizeof(IT) == 2 ? static_cast<float>(to_f16(v)) : v) : 0.0f;
    }
  }
}

// l2 normalisation of one row held by TPR consecutive lanes (VI values each),
// eps inside the sqrt (qwen.rs:837-840), times the query scale for q; the
// explicit fmaf steps fix the association for every caller.
template <class CT, int VI, int TPR>
__device__ __forceinline__ void l2norm_row(const float* x, float extra, CT* dst) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < VI; ++i) s = fmaf(x[i], x[i], s);
#pragma unroll
  for (int off = 1; off < TPR; off <<= 1) s += __shfl_xor(s, off, 64);
  const float inv = 1.0f / sqrtf(s + 1e-6f);
  const float scale = inv * extra;
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const float v = x[i] * scale;
    if constexpr (sizeof(CT) == 2)
      dst[i] = to_f16(v);
    else
      dst[i] = v;
  }
}

// Kernel 1: per (chunk, k-head) preparation of every state-independent
// operand of the chunk, for all v-heads of the k-head.
// ---------------------------------------------------------------------------
template <class CT, class IT, int DK, bool CONV>
__global__ __launch_bounds__(256) void scan_prepare(ScanParams p) {
  typedef Geo<CT, DK> G;
  constexpr int EPF = G::EPF, KB = G::KB, TPK = G::TPK, NKX = G::NKX, NKT = G::NKT, NST = G::NST;
  constexpr int VI = Vec16<IT>::n;       // input elements per 16-byte vector
  constexpr int TPR = DK / VI;           // threads per row
  constexpr int RPP = 256 / TPR;         // rows per pass
  constexpr int NPASS = (2 * kC) / RPP;
  constexpr int LDR = DK + EPF;          // sK / sQ pitch (CT)
  constexpr int LDT = kC + EPF;          // sKT / sM pitch (CT)
  constexpr int LDF = kC + 4;            // f32 64x64 pitch
  static_assert(TPR <= 64 && (TPR & (TPR - 1)) == 0, "row group must fit a wave");
  typedef typename Mma<CT>::frag frag;

  // sKT lives throughout; region R holds sK, sQ (phases 1-2), then sA, sTT, sM.
  constexpr int kBytesKQ = 2 * kC * LDR * (int)sizeof(CT);
  constexpr int kBytes3 = 2 * kC * LDF * 4 + kC * LDT * (int)sizeof(CT);
  constexpr int kBytesR = kBytesKQ > kBytes3 ? kBytesKQ : kBytes3;
  __shared__ __attribute__((aligned(16))) CT sKT[DK * LDT];  // K^ transposed [e][token]
  __shared__ __attribute__((aligned(16))) char sR[kBytesR];
  __shared__ __attribute__((aligned(16))) float sGam[kC];
  __shared__ __attribute__((aligned(16))) float sBeta[kC];
  __shared__ __attribute__((aligned(16))) float sW[kC];   // exp(gam_last - gam)
  __shared__ __attribute__((aligned(16))) float sWc[kC];  // capture weights
  CT* sK = reinterpret_cast<CT*>(sR);
  CT* sQ = sK + kC * LDR;
  float* sA = reinterpret_cast<float*>(sR);   // A, row-major [r][c]
  float* sTT = sA + kC * LDF;                 // (I+A)^-1 transposed: sTT[c][r] = Tm[r][c]
  CT* sM = reinterpret_cast<CT*>(sTT + kC * LDF);  // M row-major [r][c]

  const int chunk = blockIdx.x, hk = blockIdx.y;
  const int rep = p.Hv / p.Hk;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int col = lane & 15, grp = lane >> 4;
  int t0, n;
  if (!chunk_span(p, chunk, t0, n)) return;  // grid sized for the most chunks a batch can have
  const int dk = p.dk;
  const int64_t ck = (int64_t)chunk * p.Hk + hk;
  const int cap_chunk = p.capture > 0 ? (p.capture - 1) / kC : -1;
  const int cap_row = p.capture > 0 ? (p.capture - 1) % kC : 0;

  // ---- 1. loads: q/k rows (clamped), g and beta of the first v-head
  uint32_t gbits = 0, bbits = 0;
  if (wave == 0) {
    const int64_t gi = (int64_t)(t0 + min(lane, n - 1)) * p.sgb + (int64_t)hk * rep;
    gbits = load_bits(p.g, gi, p.dtype_gb);
    bbits = load_bits(p.beta, gi, p.dtype_gb);
  }
  if constexpr (CONV) {
    // the conv prologue: lane group g (TPR lanes) holds chunk rows
    // RPT g .. RPT g + RPT - 1 of k, then of q, VI channels per lane
    constexpr int RPT = TPR / 4;
    const int g = tid / TPR, e0 = (tid % TPR) * VI;
    int seq, start;
    conv_sequence(p, t0, seq, start);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const bool isq = m == 1;
      const int ch = (isq ? 0 : p.Hk * dk) + hk * dk + e0;  // [q | k | v] channels
      float y[RPT][VI];
      conv_rows<IT, RPT>(p, t0, n, RPT * g, seq, start, ch, e0 < dk, y);
#pragma unroll
      for (int j = 0; j < RPT; ++j)
        l2norm_row<CT, VI, TPR>(y[j], isq ? p.qscale : 1.0f, (isq ? sQ : sK) + (RPT * g + j) * LDR + e0);
    }
  } else {
    const IT* qbase = static_cast<const IT*>(p.q);
    const IT* kbase = static_cast<const IT*>(p.k);
    typename Vec16<IT>::type raw[NPASS];
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int rr = ps * RPP + tid / TPR;
      const bool isq = rr >= kC;
      const int r = isq ? rr - kC : rr;
      const IT* row = (isq ? qbase : kbase) + (int64_t)(t0 + min(r, n - 1)) * p.sqk + (int64_t)hk * dk;
      raw[ps] = load_row_raw<IT>(row, (tid % TPR) * VI, dk, p.vec_qk);
    }
    // l2-normalise rows into LDS; zero padding rows and columns dk..DK-1
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int rr = ps * RPP + tid / TPR;
      const bool isq = rr >= kC;
      const int r = isq ? rr - kC : rr;
      const int e0 = (tid % TPR) * VI;
      float x[VI];
#pragma unroll
      for (int i = 0; i < VI; ++i) x[i] = (r < n && e0 + i < dk) ? static_cast<float>(raw[ps][i]) : 0.0f;
      l2norm_row<CT, VI, TPR>(x, isq ? p.qscale : 1.0f, (isq ? sQ : sK) + r * LDR + e0);
    }
  }
  lds_barrier();

  // ---- 2. K^ / Q^ operand blocks, K^ transposed, Gram tiles
  {
    frag* kf = static_cast<frag*>(p.Kf) + ck * G::NBK * 64 + lane;
    frag* qf = static_cast<frag*>(p.Qf) + ck * G::NBK * 64 + lane;
    for (int blk = wave; blk < 2 * G::NBK; blk += 4) {
      const bool isq = blk >= G::NBK;
      const int b = isq ? blk - G::NBK : blk;
      const int t = b / NKX, kb = b % NKX;
      // K^ rows in slot order (rows of X = K^ S), Q^ rows in token order
      const int row = isq ? 16 * t + col : slot_index<CT>(t, col);
      const frag f = load_frag<CT>((isq ? sQ : sK) + row * LDR + kb * KB + grp * EPF);
      (isq ? qf : kf)[b * 64] = f;
    }
    for (int it = tid; it < DK * (kC / EPF); it += 256) {
      const int e = it / (kC / EPF), tok0 = (it % (kC / EPF)) * EPF;
      frag f;
#pragma unroll
      for (int j = 0; j < EPF; ++j) f[j] = sK[(tok0 + j) * LDR + e];
      *reinterpret_cast<frag*>(sKT + e * LDT + tok0) = f;
    }
  }
  // 20 lower 16x16 tiles: K^K^T (jobs 0-9) and Q^K^T (jobs 10-19), 5 per wave
  float4_t gram[5];
#pragma unroll
  for (int s = 0; s < 5; ++s) {
    const int job = wave + 4 * s;
    const bool isqk = job >= 10;
    const int idx = isqk ? job - 10 : job;
    const int tr = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
    const int tc = idx - tr * (tr + 1) / 2;
    const CT* a_src = (isqk ? sQ : sK) + (16 * tr + col) * LDR + grp * EPF;
    const CT* b_src = sK + (16 * tc + col) * LDR + grp * EPF;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) Mma<CT>::mma(acc, load_frag<CT>(a_src + kb * KB), load_frag<CT>(b_src + kb * KB));
    gram[s] = acc;
  }
  lds_barrier();  // sK / sQ are dead from here on
  // zeros that no v-head rewrites: the six 16x16 blocks of sTT below its
  // diagonal blocks (Tm above them) and the six tiles of sM above its diagonal
  for (int e = tid; e < 6 * 256; e += 256) {
    const int blk = e >> 8, ra = (e >> 4) & 15, cb = e & 15;
    const int hi = blk >= 3 ? 3 : blk >= 1 ? 2 : 1;  // (hi, lo): (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
    const int lo = blk - hi * (hi - 1) / 2;
    sTT[(16 * hi + ra) * LDF + 16 * lo + cb] = 0.0f;
    sM[(16 * lo + ra) * LDT + 16 * hi + cb] = CT(0);
  }

  // ---- 3. per v-head
  for (int v = 0; v < rep; ++v) {
    const int h = hk * rep + v;
    const int64_t cv = (int64_t)chunk * p.Hv + h;
    // 3a. cumulative decay and the per-row factors (wave 0, lane = token)
    if (wave == 0) {
      const float gv = lane < n ? bits_to_f32(gbits, p.dtype_gb) : 0.0f;
      const float bv = lane < n ? bits_to_f32(bbits, p.dtype_gb) : 0.0f;
      if (v + 1 < rep) {  // next v-head's g and beta
        const int64_t gi = (int64_t)(t0 + min(lane, n - 1)) * p.sgb + h + 1;
        gbits = load_bits(p.g, gi, p.dtype_gb);
        bbits = load_bits(p.beta, gi, p.dtype_gb);
      }
      float cs = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(cs, off, 64);
        if (lane >= off) cs += o;
      }
      const float gl = __shfl(cs, kC - 1, 64);
      const float gcap = __shfl(cs, cap_row, 64);
      sGam[lane] = cs;
      sBeta[lane] = bv;
      sW[lane] = decay_exp(gl - cs);
      if (chunk == cap_chunk) sWc[lane] = lane <= cap_row ? decay_exp(gcap - cs) : 0.0f;
      float* sc = p.sc + cv * 256;
      sc[lane] = bv;
      sc[64 + lane] = decay_exp(cs);
      sc[128 + lane] = cs;
      sc[192 + lane] = 0.0f;
    }
    lds_barrier();
    // 3b. A (f32) and M (CT) from the Gram tiles
#pragma unroll
    for (int s = 0; s < 5; ++s) {
      const int job = wave + 4 * s;
      const bool isqk = job >= 10;
      const int idx = isqk ? job - 10 : job;
      const int tr = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
      const int tc = idx - tr * (tr + 1) / 2;
      const int c = 16 * tc + col;
      const float gc = sGam[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * tr + 4 * grp + i;
        const float d = (c <= r) ? decay_exp(sGam[r] - gc) : 0.0f;
        if (!isqk)
          sA[r * LDF + c] = (c < r) ? (sBeta[r] * gram[s][i]) * d : 0.0f;
        else
          sM[r * LDT + c] = static_cast<CT>((c <= r) ? gram[s][i] * d : 0.0f);
      }
    }
    lds_barrier();
    // 3c. Tm = (I + A)^-1.  Diagonal 16x16 blocks: wave 0, lane = (block,
    //     column j), rows by forward substitution.
    if (wave == 0) {
      const int b = lane >> 4, j = lane & 15;
      float t[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float* arow = sA + (16 * b + r) * LDF + 16 * b;
        float s = (r == j) ? 1.0f : 0.0f;
#pragma unroll
        for (int c = 0; c < r; ++c) s = fmaf(-arow[c], t[c], s);
        t[r] = s;
      }
      float* dst = sTT + (16 * b + j) * LDF + 16 * b;
#pragma unroll
      for (int r4 = 0; r4 < 16; r4 += 4)
        *reinterpret_cast<float4_t*>(dst + r4) = float4_t{t[r4], t[r4 + 1], t[r4 + 2], t[r4 + 3]};
    }
    lds_barrier();
    //     Off-diagonal blocks, block row by block row:
    //     T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj   (wave j computes T_ij)
#pragma unroll
    for (int i = 1; i < 4; ++i) {
      if (wave < i) {
        const int j = wave;
        float4_t R = {0.f, 0.f, 0.f, 0.f};
        for (int k = j; k < i; ++k) {
          const float4_t a = *reinterpret_cast<const float4_t*>(sA + (16 * i + col) * LDF + 16 * k + 4 * grp);
          const float4_t bt = *reinterpret_cast<const float4_t*>(sTT + (16 * j + col) * LDF + 16 * k + 4 * grp);
          Mma<float>::mma(R, a, bt);
        }
        float4_t ti;
#pragma unroll
        for (int s = 0; s < 4; ++s) ti[s] = sTT[(16 * i + 4 * grp + s) * LDF + 16 * i + col];
        float4_t tij = {0.f, 0.f, 0.f, 0.f};
        Mma<float>::mma(tij, ti, R);  // R's accumulator layout is the B operand layout
        *reinterpret_cast<float4_t*>(sTT + (16 * j + col) * LDF + 16 * i + 4 * grp) = -tij;
      }
      lds_barrier();
    }
    // 3d. U blocks (s, b): U[slot(s, m)][token block b], as U^T = (W Tm B)^T K^
    //     on MFMA; token tiles of block b are TPK*b + u.  Tm[r][c] = 0 for
    //     r < c, so token blocks kr < b contribute nothing.
    auto u_blocks = [&](const float* wts, frag* dst) {
      constexpr int WPB = 4 / NKT;     // waves per token block
      constexpr int SPW = NST / WPB;   // state tiles per wave
      const int b = wave / WPB;
      const int s0 = (wave % WPB) * SPW;
      frag af[TPK][NKT];
#pragma unroll
      for (int u = 0; u < TPK; ++u)
#pragma unroll
        for (int kr = 0; kr < NKT; ++kr)
          if (kr >= b) {
            const int c = slot_index<CT>(TPK * b + u, col);
            af[u][kr] = frag_from_f32(sTT + c * LDF + kr * KB + grp * EPF, wts + kr * KB + grp * EPF, sBeta[c], CT(0));
          }
#pragma unroll
      for (int ss = 0; ss < SPW; ++ss) {
        const int s = s0 + ss;
        const CT* bsrc = sKT + slot_index<CT>(s, col) * LDT + grp * EPF;
        float4_t acc[TPK];
#pragma unroll
        for (int u = 0; u < TPK; ++u) acc[u] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kr = 0; kr < NKT; ++kr)
          if (kr >= b) {
            const frag bf = load_frag<CT>(bsrc + kr * KB);
#pragma unroll
            for (int u = 0; u < TPK; ++u) Mma<CT>::mma(acc[u], af[u][kr], bf);
          }
        dst[(s * NKT + b) * 64 + lane] = pack_frag(acc, 0, CT(0));
      }
    };
    u_blocks(sW, static_cast<frag*>(p.Uf) + cv * G::NBU * 64);
    if (chunk == cap_chunk) u_blocks(sWc, static_cast<frag*>(p.Ucf) + (int64_t)h * G::NBU * 64);
    // 3e. N blocks (t, b): N[16t + m][token block b], as N^T = (Tm B)^T M^T;
    //     wave t.  Nonzero terms need c' <= k <= r.
    {
      const int t = wave;
      const int kmax = (16 * t + 15) / KB;
      frag bm[NKT];
#pragma unroll
      for (int kb = 0; kb < NKT; ++kb) bm[kb] = load_frag<CT>(sM + (16 * t + col) * LDT + kb * KB + grp * EPF);
      frag* dst = static_cast<frag*>(p.Nf) + cv * G::NBN * 64;
#pragma unroll
      for (int b = 0; b < NKT; ++b) {
        float4_t acc[TPK];
#pragma unroll
        for (int u = 0; u < TPK; ++u) {
          acc[u] = float4_t{0.f, 0.f, 0.f, 0.f};
          const int c = slot_index<CT>(TPK * b + u, col);
#pragma unroll
          for (int kb = 0; kb < NKT; ++kb)
            if (kb >= b && kb <= kmax)
              Mma<CT>::mma(acc[u], frag_from_f32(sTT + c * LDF + kb * KB + grp * EPF, nullptr, sBeta[c], CT(0)), bm[kb]);
        }
        dst[(t * NKT + b) * 64 + lane] = pack_frag(acc, 0, CT(0));
      }
    }
    lds_barrier();  // before the next v-head rewrites sA, sTT, sM, sGam
  }

  if constexpr (CONV) {
    // ---- 4. the convolved v of this k-head's v-heads, for the carry
    // (rows of this chunk only; p.v has token stride p.sv, dv == dk)
    constexpr int RPT = TPR / 4;
    const int g = tid / TPR, e0 = (tid % TPR) * VI;
    int seq, start;
    conv_sequence(p, t0, seq, start);
    IT* vout = static_cast<IT*>(const_cast<void*>(p.v));
    for (int v = 0; v < rep; ++v) {
      const int h = hk * rep + v;
      const int ch = 2 * p.Hk * dk + h * p.dv + e0;
      float y[RPT][VI];
      conv_rows<IT, RPT>(p, t0, n, RPT * g, seq, start, ch, e0 < p.dv, y);
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int r = RPT * g + j;
        if (r < n && e0 < p.dv) {
          typename Vec16<IT>::type o;
#pragma unroll
          for (int i = 0; i < VI; ++i) o[i] = static_cast<IT>(y[j][i]);  // exact: y holds IT values
          *reinterpret_cast<typename Vec16<IT>::type*>(vout + (int64_t)(t0 + r) * p.sv + (int64_t)h * p.dv + e0) = o;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential chunk carry for one (v-head, 16 value columns).
// ---------------------------------------------------------------------------
template <class CT, int DK>
struct Carry {
  typedef Geo<CT, DK> G;
  typedef typename Mma<CT>::frag frag;
  static constexpr int D0 = sizeof(CT) == 2 ? 3 : 2;   // ring slots
  static constexpr int NL = G::NBK + G::NBU + 1;       // blocks per slot (+ scalars)
  static constexpr int NH = G::NKX + G::NKT;           // hand-off blocks: S, Y
  static constexpr int SLOT = NL * 64;                 // ring slot, 16-byte units
  static_assert((D0 - 2) * NL < 64, "ring wait count must fit vmcnt");
};

struct CarryCtx {
  int h, hk, j0, jc, jcc;
  bool col_ok;
  int lane, col, grp;
  int nchunks, cap_chunk, cap_row;
  int c0;             // the sequence's first chunk
  const float* init;  // the sequence's initial state [Hv][dk][dv] or null
  float* fin;         // its final state or null
};

// wave 1: K^, U and scalars of chunk i+D0-1 into the ring during chunk i.
template <class CT, int DK, bool VL>
__device__ __forceinline__ void carry_loader(const ScanParams& p, const CarryCtx& x,
                                             typename Carry<CT, DK>::frag* ring) {
  typedef Carry<CT, DK> K;
  typedef typename K::G G;
  auto issue = [&](int c) {
    typename K::frag* slot = ring + (c % K::D0) * K::SLOT;
    const int64_t cg = (VL ? x.c0 : 0) + c;
    const char* kf = static_cast<const char*>(p.Kf) + ((cg * p.Hk + x.hk) * G::NBK * 64 + x.lane) * 16;
    const char* uf = static_cast<const char*>(p.Uf) + ((cg * p.Hv + x.h) * G::NBU * 64 + x.lane) * 16;
    const char* sc = reinterpret_cast<const char*>(p.sc + (cg * p.Hv + x.h) * 256) + x.lane * 16;
#pragma unroll
    for (int b = 0; b < G::NBK; ++b) dma_block(kf + b * 1024, slot + b * 64);
#pragma unroll
    for (int b = 0; b < G::NBU; ++b) dma_block(uf + b * 1024, slot + (G::NBK + b) * 64);
    dma_block(sc, slot + (G::NBK + G::NBU) * 64);
  };
  for (int c = 0; c < K::D0 - 1; ++c)
    if (c < x.nchunks) issue(c);
  wait_vmcnt<0>();
  lds_barrier();  // prologue
  for (int i = 0; i < x.nchunks; ++i) {
    if (i + K::D0 - 1 < x.nchunks) {
      issue(i + K::D0 - 1);
      wait_vmcnt<(K::D0 - 2) * K::NL>();  // chunk i+1 has landed
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();  // end of chunk i
  }
  lds_barrier();  // outputs of the last chunk
}

// wave 0: the recurrence.  IT = dtype of v.
template <class CT, int DK, class IT, bool VL>
__device__ __forceinline__ void carry_recurrence(const ScanParams& p, const CarryCtx& x,
                                                 const typename Carry<CT, DK>::frag* ring,
                                                 typename Carry<CT, DK>::frag* hand) {
  typedef Carry<CT, DK> K;
  typedef typename K::G G;
  typedef typename K::frag frag;
  constexpr int NST = G::NST, NKX = G::NKX, NKT = G::NKT, NBK = G::NBK, NBU = G::NBU, TPK = G::TPK;
  const int lane = x.lane, grp = x.grp;
  const int dk = p.dk, dv = p.dv;
  const float* init = VL ? x.init : p.initial;
  float* fin = VL ? x.fin : p.final_state;

  float4_t S[NST];
#pragma unroll
  for (int s = 0; s < NST; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = slot_index<CT>(s, 4 * grp + i);
      float v = 0.0f;
      if (init && row < dk && x.col_ok) v = init[((int64_t)x.h * dk + row) * dv + x.jc];
      S[s][i] = v;
    }
  frag Sf[NKX];
#pragma unroll
  for (int kb = 0; kb < NKX; ++kb) Sf[kb] = pack_frag(S, kb, CT(0));

  const IT* vbase = static_cast<const IT*>(p.v) + (int64_t)x.h * dv + x.j0;
  // byte offsets of this lane's 16 X-rows within a chunk of v; rows past the
  // end of the sequence fall outside the chunk's buffer range and read 0
  int voff[16];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      voff[4 * t + i] = x.col_ok ? (slot_index<CT>(t, 4 * grp + i) * (int)p.sv + x.col) * (int)sizeof(IT) : kOOB;
  auto load_v = [&](uint32_t* vb, int c) {
    int t0, n;
    chunk_at<VL>(p, (VL ? x.c0 : 0) + min(c, x.nchunks - 1), t0, n);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(vbase + (int64_t)t0 * p.sv, n * (int)p.sv * (int)sizeof(IT));
#pragma unroll
    for (int k = 0; k < 16; ++k) vb[k] = buffer_load_bits<IT>(r, voff[k]);
  };
  uint32_t va[16], vb[16];
  load_v(va, 0);
  load_v(vb, 1);
  lds_barrier();  // prologue

  auto step = [&](int i, uint32_t* vbuf) {
    const frag* slot = ring + (i % K::D0) * K::SLOT;
    const float* scs = reinterpret_cast<const float*>(slot + (NBK + NBU) * 64);  // beta, eg, gam
    // every LDS operand of the chunk is requested before the first product,
    // so the reads overlap each other and the MFMAs instead of serialising
    frag kfr[4][NKX], ufr[NST][NKT];
    float4_t eg[4];
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb)
#pragma unroll
      for (int t = 0; t < 4; ++t) kfr[t][kb] = slot[(t * NKX + kb) * 64 + lane];
#pragma unroll
    for (int t = 0; t < 4; ++t) eg[t] = *reinterpret_cast<const float4_t*>(scs + 64 + slot_index<CT>(t, 4 * grp));
    const float el = scs[64 + kC - 1];
    // hand S_i to the output waves
    frag* hs = hand + (i & 1) * K::NH * 64;
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) hs[kb * 64 + lane] = Sf[kb];
    __builtin_amdgcn_sched_barrier(0);
    // X = K^ S (token rows in slot order)
    float4_t X[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) X[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    // (rounds of 4 independent accumulators, fenced so the scheduler cannot
    // turn them into dependent chains)
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) {
#pragma unroll
      for (int t = 0; t < 4; ++t) Mma<CT>::mma(X[t], kfr[t][kb], Sf[kb]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // U is requested while the products run (its registers replace K^'s)
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
      for (int b = 0; b < NKT; ++b) ufr[s][b] = slot[(NBK + s * NKT + b) * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
    // Y = V - exp(gam) X (beta is folded into U and N) for token block b
    frag Yf[NKT];
    auto y_block = [&](int b) {
#pragma unroll
      for (int u = 0; u < TPK; ++u) {
        const int t = TPK * b + u;
#pragma unroll
        for (int j = 0; j < 4; ++j) X[t][j] = bits_value<IT>(vbuf[4 * t + j]) - eg[t][j] * X[t][j];
      }
      Yf[b] = pack_frag(X, b, CT(0));
    };
    if (i != x.cap_chunk) {
      // S <- exp(gam_last) S + U Y: the scaling runs under the X products, and
      // each token block's update starts as soon as its Y is packed
#pragma unroll
      for (int s = 0; s < NST; ++s) S[s] = S[s] * el;
#pragma unroll
      for (int b = 0; b < NKT; ++b) {
        y_block(b);
#pragma unroll
        for (int s = 0; s < NST; ++s) Mma<CT>::mma(S[s], ufr[s][b], Yf[b]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // capture chunk: the state after token `capture` is
      // exp(gam_r*) S_i + Ucap Y_i, formed before S_i is updated
#pragma unroll
      for (int b = 0; b < NKT; ++b) y_block(b);
      const float ec = decay_exp(scs[128 + x.cap_row]);
      const frag* uc = static_cast<const frag*>(p.Ucf) + (int64_t)x.h * NBU * 64 + lane;
#pragma unroll
      for (int s = 0; s < NST; ++s) {
        float4_t acc = S[s] * ec;
#pragma unroll
        for (int b = 0; b < NKT; ++b) Mma<CT>::mma(acc, uc[(s * NKT + b) * 64], Yf[b]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = slot_index<CT>(s, 4 * grp + j);
          if (row < dk && x.col_ok) p.captured[((int64_t)x.h * dk + row) * dv + x.jc] = acc[j];
        }
      }
#pragma unroll
      for (int s = 0; s < NST; ++s) {
        S[s] = S[s] * el;
#pragma unroll
        for (int b = 0; b < NKT; ++b) Mma<CT>::mma(S[s], ufr[s][b], Yf[b]);
      }
    }
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) Sf[kb] = pack_frag(S, kb, CT(0));
    // hand Y_i to the output waves
#pragma unroll
    for (int b = 0; b < NKT; ++b) hs[(NKX + b) * 64 + lane] = Yf[b];
    load_v(vbuf, i + 2);
    lds_barrier();  // end of chunk i
  };
  int i = 0;
  for (; i + 1 < x.nchunks; i += 2) {
    step(i, va);
    step(i + 1, vb);
  }
  if (i < x.nchunks) step(i, va);
  lds_barrier();  // outputs of the last chunk

  if (fin) {
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = slot_index<CT>(s, 4 * grp + j);
        if (row < dk && x.col_ok) fin[((int64_t)x.h * dk + row) * dv + x.jc] = S[s][j];
      }
  }
}

// wave 0, f16 operands: the recurrence with the LDS reads of each round
// interleaved with the MFMAs of the previous one (a wave issues one 1 KiB
// read per ~14 cycles, an MFMA per 18).  IT = dtype of v.
template <class CT, int DK, class IT, bool VL>
__device__ __forceinline__ void carry_recurrence_f16(const ScanParams& p, const CarryCtx& x,
                                                     const typename Carry<CT, DK>::frag* ring,
                                                     typename Carry<CT, DK>::frag* hand) {
  typedef Carry<CT, DK> K;
  typedef typename K::G G;
  typedef typename K::frag frag;
  constexpr int NST = G::NST, NKX = G::NKX, NBK = G::NBK, NBU = G::NBU;
  static_assert(G::NKT == 2 && G::TPK == 2, "f16 geometry");
  const int lane = x.lane, grp = x.grp;
  const int dk = p.dk, dv = p.dv;
  const float* init = VL ? x.init : p.initial;
  float* fin = VL ? x.fin : p.final_state;

  float4_t S[NST];
#pragma unroll
  for (int s = 0; s < NST; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = slot_index<CT>(s, 4 * grp + i);
      float v = 0.0f;
      if (init && row < dk && x.col_ok) v = init[((int64_t)x.h * dk + row) * dv + x.jc];
      S[s][i] = v;
    }
  frag Sf[NKX];
#pragma unroll
  for (int kb = 0; kb < NKX; ++kb) Sf[kb] = pack_frag(S, kb, CT(0));

  // v two chunks ahead in registers: byte offsets of this lane's 16 X-rows;
  // rows past the end of the sequence fall outside the buffer range (read 0)
  const IT* vbase = static_cast<const IT*>(p.v) + (int64_t)x.h * dv + x.j0;
  int voff[16];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      voff[4 * q + j] = x.col_ok ? (slot_index<CT>(q, 4 * grp + j) * (int)p.sv + x.col) * (int)sizeof(IT) : kOOB;
  auto load_v = [&](uint32_t* vb, int c) {
    int t0, n;
    chunk_at<VL>(p, (VL ? x.c0 : 0) + min(c, x.nchunks - 1), t0, n);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(vbase + (int64_t)t0 * p.sv, n * (int)p.sv * (int)sizeof(IT));
#pragma unroll
    for (int k = 0; k < 16; ++k) vb[k] = buffer_load_bits<IT>(r, voff[k]);
  };
  uint32_t va[16], vb[16];
  load_v(va, 0);
  load_v(vb, 1);
  lds_barrier();  // prologue

  auto step = [&](int i, uint32_t* vbuf) {
    const frag* slot = ring + (i % K::D0) * K::SLOT;
    const float* scs = reinterpret_cast<const float*>(slot + (NBK + NBU) * 64);  // beta, eg, gam
    frag* hs = hand + (i & 1) * K::NH * 64;
    frag kf[4][NKX], uf[NST][2];
    float4_t eg[4], X[4];
    float el;
#pragma unroll
    for (int t = 0; t < 4; ++t) kf[t][0] = slot[(t * NKX) * 64 + lane];
#pragma unroll
    for (int t = 0; t < 4; ++t) X[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_sched_barrier(0);
    // X = K^ S in rounds of 4 independent products; each round also requests
    // the next round's operands
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) {
      if (kb + 1 < NKX) {
#pragma unroll
        for (int t = 0; t < 4; ++t) kf[t][kb + 1] = slot[(t * NKX + kb + 1) * 64 + lane];
      }
      if (kb == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) eg[t] = *reinterpret_cast<const float4_t*>(scs + 64 + slot_index<CT>(t, 4 * grp));
        el = scs[64 + kC - 1];
      }
      if (kb == NKX - 1) {
#pragma unroll
        for (int s = 0; s < NST; ++s) uf[s][0] = slot[(NBK + 2 * s) * 64 + lane];
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) Mma<CT>::mma(X[t], kf[t][kb], Sf[kb]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Y = V - exp(gam) X for token block b (beta is folded into U and N)
    frag Yf[2];
    auto y_block = [&](int b) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          X[2 * b + u][j] = bits_value<IT>(vbuf[4 * (2 * b + u) + j]) - eg[2 * b + u][j] * X[2 * b + u][j];
      Yf[b] = pack_frag(X, b, CT(0));
    };
    y_block(0);
    if (i == x.cap_chunk) {
      // state after token `capture`: exp(gam_r*) S_i + Ucap Y_i
      y_block(1);
      const float ec = decay_exp(scs[128 + x.cap_row]);
      const frag* uc = static_cast<const frag*>(p.Ucf) + (int64_t)x.h * NBU * 64 + lane;
#pragma unroll
      for (int s = 0; s < NST; ++s) {
        float4_t acc = S[s] * ec;
#pragma unroll
        for (int b = 0; b < 2; ++b) Mma<CT>::mma(acc, uc[(2 * s + b) * 64], Yf[b]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = slot_index<CT>(s, 4 * grp + j);
          if (row < dk && x.col_ok) p.captured[((int64_t)x.h * dk + row) * dv + x.jc] = acc[j];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // S <- exp(gam_last) S + U Y, token block 0 (requests U of block 1)
#pragma unroll
    for (int s = 0; s < NST; ++s) uf[s][1] = slot[(NBK + 2 * s + 1) * 64 + lane];
#pragma unroll
    for (int s = 0; s < NST; ++s) {
      S[s] = S[s] * el;
      Mma<CT>::mma(S[s], uf[s][0], Yf[0]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i != x.cap_chunk) y_block(1);
    // token block 1; S_i goes to the output waves meanwhile
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) hs[kb * 64 + lane] = Sf[kb];
#pragma unroll
    for (int s = 0; s < NST; ++s) Mma<CT>::mma(S[s], uf[s][1], Yf[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) Sf[kb] = pack_frag(S, kb, CT(0));
#pragma unroll
    for (int b = 0; b < 2; ++b) hs[(NKX + b) * 64 + lane] = Yf[b];
    load_v(vbuf, i + 2);
    lds_barrier();  // end of chunk i
  };
  int i = 0;
  for (; i + 1 < x.nchunks; i += 2) {
    step(i, va);
    step(i + 1, vb);
  }
  if (i < x.nchunks) step(i, va);
  lds_barrier();  // outputs of the last chunk

  if (fin) {
#pragma unroll
    for (int s = 0; s < NST; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = slot_index<CT>(s, 4 * grp + j);
        if (row < dk && x.col_ok) fin[((int64_t)x.h * dk + row) * dv + x.jc] = S[s][j];
      }
  }
}

// waves 2-3: O of chunk c during chunk c+1, rows 16t.. for t = 2(wave-2)+{0,1}.
template <class CT, int DK, class OT, bool VL>
__device__ __forceinline__ void carry_outputs(const ScanParams& p, const CarryCtx& x, int ow,
                                              const typename Carry<CT, DK>::frag* hand) {
  typedef Carry<CT, DK> K;
  typedef typename K::G G;
  typedef typename K::frag frag;
  constexpr int NKX = G::NKX, NKT = G::NKT;
  const int lane = x.lane, grp = x.grp;
  struct Ops {
    frag q[2][NKX];
    frag nn[2][NKT];
    float4_t eg[2];
  };
  auto load_o = [&](Ops& o, int c) {
    const int64_t cc = (VL ? x.c0 : 0) + min(c, x.nchunks - 1);
    const frag* qf = static_cast<const frag*>(p.Qf) + (cc * p.Hk + x.hk) * G::NBK * 64 + lane;
    const frag* nf = static_cast<const frag*>(p.Nf) + (cc * p.Hv + x.h) * G::NBN * 64 + lane;
    const float* scs = p.sc + (cc * p.Hv + x.h) * 256;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int t = 2 * ow + tt;
#pragma unroll
      for (int kb = 0; kb < NKX; ++kb) o.q[tt][kb] = qf[(t * NKX + kb) * 64];
#pragma unroll
      for (int b = 0; b < NKT; ++b) o.nn[tt][b] = nf[(t * NKT + b) * 64];
      o.eg[tt] = *reinterpret_cast<const float4_t*>(scs + 64 + 16 * t + 4 * grp);
    }
  };
  Ops oa, ob;
  load_o(oa, 0);
  load_o(ob, 1);
  const OT* out = static_cast<const OT*>(p.out) + (int64_t)x.h * p.dv + x.j0;
  int ooff[2][4];  // byte offsets of this lane's output rows within a chunk
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ooff[tt][j] = x.col_ok ? ((16 * (2 * ow + tt) + 4 * grp + j) * (int)p.so + x.col) * (int)sizeof(OT) : kOOB;
  lds_barrier();  // prologue
  lds_barrier();  // chunk 0 (no outputs yet)
  auto ostep = [&](int c, Ops& o) {
    const frag* hs = hand + (c & 1) * K::NH * 64;
    frag sf[NKX], yf[NKT];
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) sf[kb] = hs[kb * 64 + lane];
#pragma unroll
    for (int b = 0; b < NKT; ++b) yf[b] = hs[(NKX + b) * 64 + lane];
    int t0, n;
    chunk_at<VL>(p, (VL ? x.c0 : 0) + c, t0, n);
    // rows past the end of the sequence fall outside the buffer range: dropped
    const __amdgpu_buffer_rsrc_t r = make_rsrc(out + (int64_t)t0 * p.so, n * (int)p.so * (int)sizeof(OT));
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < NKX; ++kb) Mma<CT>::mma(acc, o.q[tt][kb], sf[kb]);
      acc = acc * o.eg[tt];
#pragma unroll
      for (int b = 0; b < NKT; ++b) Mma<CT>::mma(acc, o.nn[tt][b], yf[b]);
#pragma unroll
      for (int j = 0; j < 4; ++j) buffer_store(r, ooff[tt][j], acc[j], OT(0));
    }
    load_o(o, c + 2);
    lds_barrier();  // end of chunk c+1
  };
  int c = 0;
  for (; c + 1 < x.nchunks; c += 2) {
    ostep(c, oa);
    ostep(c + 1, ob);
  }
  if (c < x.nchunks) ostep(c, oa);
}

template <class CT, int DK, bool VL>
__global__ __launch_bounds__(256) void scan_carry(ScanParams p) {
  typedef Carry<CT, DK> K;
  __shared__ __attribute__((aligned(16))) typename K::frag ring[K::D0 * K::SLOT];
  __shared__ __attribute__((aligned(16))) typename K::frag hand[2 * K::NH * 64];

  CarryCtx x;
  x.lane = threadIdx.x & 63;
  x.col = x.lane & 15;
  x.grp = x.lane >> 4;
  const int wave = wave_id();
  // XCD-aware placement for one sequence: logical work-group L -> consecutive
  // L share a k-head.  A ragged batch keeps the launch order (sequences with
  // the most chunks first) across all XCDs instead.
  const int nwg = gridDim.x;
  int L = blockIdx.x;
  if (!VL && (nwg & 7) == 0) L = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int ntiles = (p.dv + kVT - 1) / kVT;
  const int rep = p.Hv / p.Hk;
  const int slot = L / (p.Hv * ntiles);
  L -= slot * p.Hv * ntiles;
  int seq = 0;
  x.c0 = 0;
  x.nchunks = p.nchunks;
  if (VL) {
    const int4 e = p.seq_tab[slot];
    seq = e.x;
    x.c0 = e.y;
    x.nchunks = e.z;
  }
  x.h = L / ntiles;
  x.hk = x.h / rep;
  x.j0 = (L % ntiles) * kVT;
  x.jc = x.j0 + x.col;
  x.col_ok = x.jc < p.dv;
  x.jcc = min(x.jc, p.dv - 1);
  x.init = p.initial ? p.initial + seq * p.init_stride : nullptr;
  x.fin = p.final_state ? p.final_state + (int64_t)seq * p.Hv * p.dk * p.dv : nullptr;
  x.cap_chunk = p.capture > 0 ? (p.capture - 1) / kC : -1;
  x.cap_row = p.capture > 0 ? (p.capture - 1) % kC : 0;

  if (VL && x.nchunks == 0) {  // empty sequence: the final state is the initial one
    if (wave == 0 && x.fin && x.col_ok)
      for (int r = x.grp; r < p.dk; r += 4) {
        const int64_t o = ((int64_t)x.h * p.dk + r) * p.dv + x.jc;
        x.fin[o] = x.init ? x.init[o] : 0.0f;
      }
    return;
  }
  if (wave == 1) {
    carry_loader<CT, DK, VL>(p, x, ring);
  } else if (wave == 0) {
    if constexpr (sizeof(CT) == 2) {
      if (p.dtype_qkv == 0)
        carry_recurrence_f16<CT, DK, float, VL>(p, x, ring, hand);
      else
        carry_recurrence_f16<CT, DK, half_t, VL>(p, x, ring, hand);
    } else {
      if (p.dtype_qkv == 0)
        carry_recurrence<CT, DK, float, VL>(p, x, ring, hand);
      else
        carry_recurrence<CT, DK, half_t, VL>(p, x, ring, hand);
    }
  } else {
    if (p.dtype_out == 0)
      carry_outputs<CT, DK, float, VL>(p, x, wave - 2, hand);
    else
      carry_outputs<CT, DK, half_t, VL>(p, x, wave - 2, hand);
  }
}

template <class CT, class IT, int DK>
int launch_dk(const ScanParams& p, hipStream_t stream) {
  if (p.mixed)
    hipLaunchKernelGGL((scan_prepare<CT, IT, DK, true>), dim3(p.nchunks, p.Hk), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((scan_prepare<CT, IT, DK, false>), dim3(p.nchunks, p.Hk), dim3(256), 0, stream, p);
  int rc = check_launch("scan_prepare");
  if (rc) return rc;
  const int ntiles = (p.dv + kVT - 1) / kVT;
  const int nseq = p.seq_tab ? p.nseq : 1;
  if (p.seq_tab)
    hipLaunchKernelGGL((scan_carry<CT, DK, true>), dim3(nseq * p.Hv * ntiles), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((scan_carry<CT, DK, false>), dim3(p.Hv * ntiles), dim3(256), 0, stream, p);
  return check_launch("scan_carry");
}

template <class CT, class IT>
int launch_it(const ScanParams& p, hipStream_t stream) {
  if (p.dk <= 32) return launch_dk<CT, IT, 32>(p, stream);
  if (p.dk <= 64) return launch_dk<CT, IT, 64>(p, stream);
  return launch_dk<CT, IT, 128>(p, stream);
}

}  // namespace
}  // namespace clef
