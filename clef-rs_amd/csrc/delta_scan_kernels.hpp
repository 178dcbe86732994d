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
// not depend on the state and writes U and N as MFMA operand blocks (64
// lanes x 16 bytes, in the order the consumer's lanes read them) plus the
// per-row scalars.  (I + A)^-1 is formed in f32: 16x16 diagonal blocks by
// forward substitution, the rest by block forward substitution on MFMA.
//
// scan_carry (grid Hv x ceil(dv/16)) runs the chunks in order for one v-head
// and 16 value columns (the columns of S evolve independently), reading the
// raw key and query rows: K^ S and Q^ S are the raw products times per-row
// factors (see the carry below).
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



// l2 normalisation of one row held by TPR consecutive lanes (VI values each),
// eps inside the sqrt (qwen.rs:837-840), times the query scale for q; the
// explicit fmaf steps fix the association for every caller.  Returns the
// factor the row was multiplied by.
template <class CT, int VI, int TPR>
__device__ __forceinline__ float l2norm_row(const float* x, float extra, CT* dst) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < VI; ++i) s = fmaf(x[i], x[i], s);
  s = lane_sum<TPR>(s);  // DPP moves, the association of an xor butterfly
  const float inv = 1.0f / sqrtf(s + 1e-6f);
  const float scale = inv * extra;
  CT out[VI];
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const float v = x[i] * scale;
    if constexpr (sizeof(CT) == 2)
      out[i] = to_f16(v);
    else
      out[i] = v;
  }
  __builtin_memcpy(dst, out, sizeof(out));  // one vector store (dst is 16-byte aligned)
  return scale;
}

// ---------------------------------------------------------------------------
// Kernel 1: per (chunk, k-head) preparation of the state-independent operands
// of the chunk, for all v-heads of the k-head: U and N blocks and the per-row
// scalars (the normalised keys and queries themselves are not stored: the
// carry multiplies the raw rows and applies the norms as row factors).
// ---------------------------------------------------------------------------
constexpr int kPW = 8;  // waves of a scan_prepare work-group

// Two work-groups per CU (16 waves, 128 registers each) where the LDS holds
// two; f32 products with 128-wide keys need more LDS than half a CU.
template <class CT, class IT, int DK>
__global__ __launch_bounds__(64 * kPW, (sizeof(CT) == 4 && DK > 64) ? 2 : 4) void scan_prepare(ScanParams p) {
  typedef Geo<CT, DK> G;
  constexpr int EPF = G::EPF, KB = G::KB, TPK = G::TPK, NKX = G::NKX, NKT = G::NKT, NST = G::NST;
  constexpr int VI = Vec16<IT>::n;       // input elements per 16-byte vector
  constexpr int TPR = DK / VI;           // threads per row
  constexpr int NT = 64 * kPW;           // threads
  constexpr int RPP = NT / TPR;          // rows per pass
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
  __shared__ __attribute__((aligned(16))) float sInv[2][kC];  // row factors: keys 1/|k|, queries qscale/|q|
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
  const int cap_chunk = p.capture > 0 ? (p.capture - 1) / kC : -1;
  const int cap_row = p.capture > 0 ? (p.capture - 1) % kC : 0;

  // ---- 1. loads: q/k rows (clamped), g and beta of the first v-head
  uint32_t gbits = 0, bbits = 0;
  if (wave == 0) {
    const int64_t gi = (int64_t)(t0 + min(lane, n - 1)) * p.sgb + (int64_t)hk * rep;
    gbits = load_bits(p.g, gi, p.dtype_gb);
    bbits = load_bits(p.beta, gi, p.dtype_gb);
  }
  {
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
      const float f = l2norm_row<CT, VI, TPR>(x, isq ? p.qscale : 1.0f, (isq ? sQ : sK) + r * LDR + e0);
      if (tid % TPR == 0) sInv[isq][r] = r < n ? f : 0.0f;
    }
  }
  lds_barrier();

  // ---- 2. K^ transposed, Gram tiles
  // (consecutive lanes take consecutive columns e: their element reads share
  // a row and hit distinct banks)
  for (int it = tid; it < DK * (kC / EPF); it += NT) {
    const int e = it % DK, tok0 = (it / DK) * EPF;
    frag f;
#pragma unroll
    for (int j = 0; j < EPF; ++j) f[j] = sK[(tok0 + j) * LDR + e];
    *reinterpret_cast<frag*>(sKT + e * LDT + tok0) = f;
  }
  // 20 lower 16x16 tiles: K^K^T (jobs 0-9) and Q^K^T (jobs 10-19); wave w
  // takes the jobs w, w + kPW, ...
  constexpr int JPW = (20 + kPW - 1) / kPW;
  float4_t gram[JPW];
#pragma unroll
  for (int s = 0; s < JPW; ++s) {
    const int job = wave + kPW * s;
    if (job >= 20) break;
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
  for (int e = tid; e < 6 * 256; e += NT) {
    const int blk = e >> 8, ra = (e >> 4) & 15, cb = e & 15;
    const int hi = blk >= 3 ? 3 : blk >= 1 ? 2 : 1;  // (hi, lo): (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
    const int lo = blk - hi * (hi - 1) / 2;
    sTT[(16 * hi + ra) * LDF + 16 * lo + cb] = 0.0f;
    sM[(16 * lo + ra) * LDT + 16 * hi + cb] = CT(0);
  }

  // ---- 3. per v-head
  for (int v = 0; v < rep; ++v) {
    const int h = hk * rep + v;
    uint32_t gnext = 0, bnext = 0;
    const int64_t cv = (int64_t)chunk * p.Hv + h;
    // 3a. cumulative decay and the per-row factors (wave 0, lane = token):
    //     the carry's row factors 1/|k| e^gam (for V - e^gam K^ S) and
    //     qscale/|q| e^gam (for e^gam Q^ S), gam (capture) and e^gam
    if (wave == 0) {
      const float gv = lane < n ? bits_to_f32(gbits, p.dtype_gb) : 0.0f;
      const float bv = lane < n ? bits_to_f32(bbits, p.dtype_gb) : 0.0f;
      if (v + 1 < rep) {  // next v-head's g and beta, awaited at the end of this one
        const int64_t gi = (int64_t)(t0 + min(lane, n - 1)) * p.sgb + h + 1;
        gnext = load_bits(p.g, gi, p.dtype_gb);
        bnext = load_bits(p.beta, gi, p.dtype_gb);
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
      const float eg = decay_exp(cs);
      float* sc = p.sc + cv * 256;
      sc[lane] = sInv[0][lane] * eg;
      sc[64 + lane] = sInv[1][lane] * eg;
      sc[128 + lane] = cs;
      sc[192 + lane] = eg;
    }
    lds_barrier();
    // 3b. A (f32) and M (CT) from the Gram tiles
#pragma unroll
    for (int s = 0; s < JPW; ++s) {
      const int job = wave + kPW * s;
      if (job >= 20) break;
      const bool isqk = job >= 10;
      const int idx = isqk ? job - 10 : job;
      const int tr = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
      const int tc = idx - tr * (tr + 1) / 2;
      const int c = 16 * tc + col;
      const float gc = sGam[c];
      // the four rows' gam and beta as vectors; the ratio is exponentiated for
      // every element and masked afterwards (above the diagonal it may be
      // inf, and the select keeps it out), so the block has no branches
      const float4_t gr = *reinterpret_cast<const float4_t*>(sGam + 16 * tr + 4 * grp);
      const float4_t br = *reinterpret_cast<const float4_t*>(sBeta + 16 * tr + 4 * grp);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * tr + 4 * grp + i;
        const float e = decay_exp(gr[i] - gc);
        const float d = c <= r ? e : 0.0f;
        if (!isqk)
          sA[r * LDF + c] = c < r ? (br[i] * gram[s][i]) * d : 0.0f;
        else
          sM[r * LDT + c] = static_cast<CT>(c <= r ? gram[s][i] * d : 0.0f);
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
      constexpr int WPB = kPW / NKT < NST ? kPW / NKT : NST;  // waves per token block
      constexpr int SPW = NST / WPB;                           // state tiles per wave
      static_assert(WPB >= 1 && NST % WPB == 0, "whole state tiles per wave");
      const int b = wave / WPB;
      if (b >= NKT) return;  // (narrow keys: more waves than blocks)
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
    //     wave w: t = w % 4, token blocks [b0, b0 + BPW).  Nonzero terms need
    //     c' <= k <= r.
    {
      constexpr int BPW = NKT * 4 / kPW;  // token blocks per wave
      static_assert(BPW >= 1 && NKT * 4 % kPW == 0, "whole token blocks per wave");
      const int t = wave & 3, b0 = (wave >> 2) * BPW;
      const int kmax = (16 * t + 15) / KB;
      frag bm[NKT];
#pragma unroll
      for (int kb = 0; kb < NKT; ++kb) bm[kb] = load_frag<CT>(sM + (16 * t + col) * LDT + kb * KB + grp * EPF);
      frag* dst = static_cast<frag*>(p.Nf) + cv * G::NBN * 64;
#pragma unroll
      for (int bb = 0; bb < BPW; ++bb) {
        const int b = b0 + bb;
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
    gbits = gnext;  // the loads were issued a whole v-head ago
    bbits = bnext;
    lds_barrier();  // before the next v-head rewrites sA, sTT, sM, sGam
  }

}

// ---------------------------------------------------------------------------
// Kernel 2: sequential chunk carry for one (v-head, 16 value columns).
//
// Wave 0 runs the recurrence; loader waves fill a ring of LDS slots, D0 - 1
// chunks ahead, with global->LDS DMA (f16: wave 1 the chunk's raw key rows,
// wave 2 its U blocks and row scalars; f32: wave 1 both); output waves form
// the outputs of the previous chunk (f16: four waves of one 16-row tile, f32:
// two of two) from the S and Y that wave 0 hands over in LDS and from query
// rows and N blocks they load into registers a few chunks ahead.  One
// barrier per chunk.
//
// Norms as row factors: with a_r = 1/|k_r| and b_r = qscale/|q_r|,
//   e^gam (K^ S) = diag(a e^gam) (K S),   e^gam (Q^ S) = diag(b e^gam) (Q S),
// so the raw key and query rows (the conv output, as stored) are the MFMA
// operands and nothing normalised is written to memory.
// ---------------------------------------------------------------------------

// XOR swizzle of the 16-byte chunk index of a raw key row in LDS, so that the
// 16 rows one MFMA fragment read touches (slot-ordered rows for f16, which
// differ in row bits 0, 1, 3, 4; consecutive rows for f32) hit distinct banks
// for every row width (NCH chunks of 16 bytes per row).
template <class CT, int NCH>
__device__ __forceinline__ int kswz(int r) {
  if constexpr (sizeof(CT) == 2) {
    if constexpr (NCH >= 16) return (r & 3) | ((r >> 1) & 12);
    else if constexpr (NCH == 8) return ((r >> 1) & 1) | ((r >> 2) & 6);
    else return (r >> 3) & 3;
  } else {
    if constexpr (NCH >= 16) return r & 15;
    else if constexpr (NCH == 8) return (r >> 1) & 7;
    else return (r >> 2) & 3;
  }
}

template <class CT, class IT, int DK>
struct Carry {
  typedef Geo<CT, DK> G;
  typedef typename Mma<CT>::frag frag;
  static constexpr int RB = DK * (int)sizeof(IT);        // bytes of a raw key row
  static constexpr int NCH = RB / 16;                     // its 16-byte chunks
  static constexpr int KBYTES = kC * RB;                  // a chunk's raw keys
  static constexpr int NDK = KBYTES / 1024;               // 1 KiB DMA instructions for them
  static constexpr int UOFF = KBYTES;                     // U blocks within a slot
  static constexpr int SOFF = KBYTES + G::NBU * 1024;     // row scalars within a slot
  static constexpr int SLOT = SOFF + 1024;
  static constexpr int HAND = 2 * (G::NKX + G::NKT) * 1024;  // S and Y hand-off, double buffered
  static constexpr int LDS = 160 * 1024 - 64;             // less the exchange flags
  // recurrence waves: f16 one (its chunk takes ~16 cycles per product; an LDS
  // exchange of partial products between two waves costs more than it
  // saves), f32 four (each a quarter of the products, 32 cycles each), as far
  // as the k-blocks go and as long as two ring slots and their 4 KiB partial
  // products still fit the LDS
  static constexpr int rec_waves() {
    int n = sizeof(CT) == 2 ? 1 : 4;
    if (n > G::NKX) n = G::NKX;
    while (n > 1 && 2 * SLOT + HAND + n * 4096 > LDS) n /= 2;
    return n;
  }
  static constexpr int NREC = rec_waves();
  static constexpr int KPR = G::NKX / NREC;               // k-blocks of the state per recurrence wave
  static constexpr int SPR = G::NST / NREC;               // its 16-row tiles
  static constexpr int XCH = NREC > 1 ? NREC * 4096 : 0;  // partial products Y_r
  // waves: NREC recurrence, NLOAD loaders, NOUT output waves of TPW 16-row tiles
  // (one f32 recurrence wave leaves room for two output waves of 512 registers).
  // (f16 with three loaders, eight waves, takes the same time: the chunk's
  // DMA costs the products it shares the CU with, not its own issue rate or
  // latency; f32 already has nine waves.)
  static constexpr int NLOAD = sizeof(CT) == 2 ? 2 : 1;
  static constexpr int NOUT = (sizeof(CT) == 4 && NREC == 1) ? 2 : 4;
  static constexpr int TPW = 4 / NOUT;
  static constexpr int OD = (sizeof(CT) == 4 && NOUT == 4) ? 1 : 2;  // chunks of output operands in registers
  // a chunk's DMA items: NDK key blocks, NBU U blocks, one block of row
  // scalars; loader w issues items [w PERW, (w + 1) PERW)
  static constexpr int NITEM = NDK + G::NBU + 1;
  static constexpr int PERW = (NITEM + NLOAD - 1) / NLOAD;
  // ring slots: at most 4, as many as the LDS holds, and few enough that the
  // DMA instructions a loader keeps in flight fit the 6-bit vmcnt
  static constexpr int DL = (LDS - HAND - XCH) / SLOT, DV = 2 + 63 / PERW;
  static constexpr int D0 = DL < DV ? (DL < 4 ? DL : 4) : (DV < 4 ? DV : 4);
  static constexpr int THREADS = 64 * (NREC + NLOAD + NOUT);
  // with three or more slots the loaders land chunk i+1 before chunk i
  // starts, so the recurrence reads the next chunk's keys during this one
  // (not with f32 keys under f16 products: their conversion needs the room)
  static constexpr bool PREF = D0 >= 3 && sizeof(IT) == sizeof(CT);
  static_assert(D0 >= 2 && D0 * SLOT + HAND + XCH <= LDS, "two ring slots fit the LDS");
  static_assert(G::NKX % NREC == 0 && G::NST % NREC == 0, "whole k-blocks per recurrence wave");
  static_assert((D0 - 2) * PERW < 64, "ring wait counts fit vmcnt");
  static_assert(KBYTES % 1024 == 0, "whole DMA instructions per chunk of keys");
};

// LDS hand-off between the recurrence waves of a work-group: wave r sets byte
// r of one flag word to the chunk count mod 256 once its partial product is
// in LDS (the waves are never a whole chunk apart: they meet at the barrier
// that ends each chunk), and a single read of the word sees every wave.  The
// word is accessed through an LDS-space pointer: a volatile access through a
// generic pointer becomes a system-coherent flat access that waits for every
// outstanding global load.
typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) unsigned lds_u32;
// Every earlier LDS access of the wave has completed before its byte changes.
__device__ __forceinline__ void lds_publish(unsigned* flags, int r, unsigned v) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  *((volatile lds_u8*)flags + r) = (unsigned char)v;
}
// Waits until the low n bytes of the word all read v.  Bounded: after 2^22
// polls the wave goes on, so every wave reaches the end of the kernel.
__device__ __forceinline__ void lds_wait_all(const unsigned* flags, int n, unsigned v) {
  const unsigned mask = n >= 4 ? 0xffffffffu : (1u << (8 * n)) - 1u;
  const unsigned want = (v & 0xffu) * 0x01010101u & mask;
  const volatile lds_u32* f = (const volatile lds_u32*)flags;
  for (int k = 0; k < (1 << 22); ++k)
    if ((*f & mask) == want) break;
  asm volatile("" ::: "memory");
}

// Token span of chunk c of the work-group's sequence: a sequence's chunks
// are 64-token steps from its first token (the chunk table holds exactly
// these spans), so no table is read on the carry's paths; a lookup there
// makes each step wait for it, and in-order vmcnt then drains every load
// in flight behind it.
struct CarryCtx;
__device__ __forceinline__ void chunk_of(const CarryCtx& x, int c, int& t0, int& n);

struct CarryCtx {
  int h, hk, j0, jc;
  bool col_ok;
  int lane, col, grp;
  int nchunks, cap_chunk, cap_row;
  int c0;             // the sequence's first chunk
  int t0s, lens;      // the sequence's first token and length
  const float* init;  // the sequence's initial state [Hv][dk][dv] or null
  float* fin;         // its final state or null
};

__device__ __forceinline__ void chunk_of(const CarryCtx& x, int c, int& t0, int& n) {
  t0 = x.t0s + c * kC;
  n = min(kC, x.lens - c * kC);
}

// EPF elements k.. of raw key row r in a slot's key region, as a CT fragment.
template <class CT, class IT, int DK>
__device__ __forceinline__ typename Mma<CT>::frag key_frag(const char* keys, int r, int k) {
  constexpr int RB = DK * (int)sizeof(IT), NCH = RB / 16;
  const char* row = keys + r * RB;
  const int key = kswz<CT, NCH>(r);
  if constexpr (sizeof(CT) == sizeof(IT)) {
    const int c = (k * (int)sizeof(IT)) >> 4;
    return *reinterpret_cast<const typename Mma<CT>::frag*>(row + ((c ^ key) << 4));
  } else if constexpr (sizeof(IT) == 2) {  // f16 keys, f32 fragment of 4
    const int b = k * 2, c = b >> 4;
    const half4 v = *reinterpret_cast<const half4*>(row + ((c ^ key) << 4) + (b & 15));
    return float4_t{static_cast<float>(v[0]), static_cast<float>(v[1]), static_cast<float>(v[2]),
                    static_cast<float>(v[3])};
  } else {  // f32 keys, f16 fragment of 8 (two chunks)
    const int c = (k * 4) >> 4;
    const float4_t a = *reinterpret_cast<const float4_t*>(row + ((c ^ key) << 4));
    const float4_t b = *reinterpret_cast<const float4_t*>(row + (((c + 1) ^ key) << 4));
    half8 f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = static_cast<half_t>(a[i]);
      f[4 + i] = static_cast<half_t>(b[i]);
    }
    return f;
  }
}

// EPF elements k.. of a raw query row in global memory as a CT fragment;
// elements past dk read as zero (VEC: dk == DK and 16-byte rows).  VEC is a
// template parameter: a run-time choice inside the prefetching loop makes the
// compiler wait for every load where the two paths join.
template <class CT, class IT, bool VEC>
__device__ __forceinline__ typename Mma<CT>::frag query_frag(const IT* row, int k, int dk) {
  constexpr int EPF = 16 / (int)sizeof(CT);
  typename Mma<CT>::frag f;
  if constexpr (VEC) {
    if constexpr (sizeof(CT) == sizeof(IT)) {
      return *reinterpret_cast<const typename Mma<CT>::frag*>(row + k);
    } else if constexpr (sizeof(IT) == 2) {
      const half4 v = *reinterpret_cast<const half4*>(row + k);
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = static_cast<float>(v[i]);
      return f;
    } else {
      const float4_t a = *reinterpret_cast<const float4_t*>(row + k);
      const float4_t b = *reinterpret_cast<const float4_t*>(row + k + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[i] = static_cast<half_t>(a[i]);
        f[4 + i] = static_cast<half_t>(b[i]);
      }
      return f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPF; ++i) f[i] = static_cast<CT>(k + i < dk ? static_cast<float>(row[k + i]) : 0.0f);
    return f;
  }
}

// The raw key rows of chunk c element by element, for rows that are not
// whole 16-byte vectors (dk < DK or unaligned rows): stored in the layout the
// key DMA produces (below), with zeros past dk.
template <class CT, class IT, int DK, bool VL>
__device__ __forceinline__ void carry_keys_slow(const ScanParams& p, const CarryCtx& x, char* keys, int c) {
  typedef Carry<CT, IT, DK> K;
  int t0, n;
  chunk_of(x, c, t0, n);
  const char* base = reinterpret_cast<const char*>(static_cast<const IT*>(p.k) + (int64_t)t0 * p.sqk +
                                                   (int64_t)x.hk * p.dk);
  const int64_t rowb = p.sqk * (int64_t)sizeof(IT);
  constexpr int VI = 16 / (int)sizeof(IT);
  for (int q = 0; q < K::NDK; ++q) {
    const int o = 1024 * q + 16 * x.lane, r = o / K::RB, pc = (o % K::RB) >> 4;
    const int e0 = (pc ^ kswz<CT, K::NCH>(r)) * VI;
    const IT* row = reinterpret_cast<const IT*>(base + min(r, n - 1) * rowb);
    typename Vec16<IT>::type v;
#pragma unroll
    for (int i = 0; i < VI; ++i) v[i] = e0 + i < p.dk ? row[e0 + i] : IT(0);
    *reinterpret_cast<typename Vec16<IT>::type*>(keys + o) = v;
  }
}

// Loader LW: DMA items [LW PERW, (LW + 1) PERW) of each chunk into its ring
// slot.  Items: the raw key rows' 1 KiB blocks q < NDK, then the U blocks,
// then the row scalars.  Key block q, lane l writes slot bytes 1024 q + 16 l,
// i.e. row r = (1024 q + 16 l) / RB at swizzled chunk pc, and reads logical
// chunk pc ^ kswz(r) of that row (rows past the chunk's end repeat its last
// row, whose results are multiplied by a zero row factor).  Without whole
// 16-byte key rows (FAST false) loader 0 writes the keys with carry_keys_slow
// instead: chunk i + 1 + PREF during chunk i (the recurrence reads chunk
// i + 1's keys during chunk i when it prefetches), so they are published by
// the barrier that ends chunk i - PREF.
template <class CT, class IT, int DK, bool VL, int LW, bool FAST>
__device__ __forceinline__ void carry_loader_w(const ScanParams& p, const CarryCtx& x, char* ring) {
  typedef Carry<CT, IT, DK> K;
  constexpr int NDK = K::NDK, NU = K::G::NBU;
  constexpr int Q0 = LW * K::PERW < K::NITEM ? LW * K::PERW : K::NITEM;
  constexpr int Q1 = Q0 + K::PERW < K::NITEM ? Q0 + K::PERW : K::NITEM;
  constexpr int KQ0 = Q0 < NDK ? Q0 : NDK, KQ1 = Q1 < NDK ? Q1 : NDK;
  // DMA instructions this wave issues per chunk (what its vmcnt waits count)
  constexpr int PER = (Q1 - Q0) - (FAST ? 0 : KQ1 - KQ0);
  constexpr int PREF = K::PREF ? 1 : 0;
  auto slot = [&](int c) { return ring + (c % K::D0) * K::SLOT; };
  auto issue = [&](int c) {
    char* s = slot(c);
    const int64_t cg = (VL ? x.c0 : 0) + c;
    if constexpr (FAST && KQ1 > KQ0) {
      int t0, n;
      chunk_of(x, c, t0, n);
      const char* base = reinterpret_cast<const char*>(static_cast<const IT*>(p.k) + (int64_t)t0 * p.sqk +
                                                       (int64_t)x.hk * p.dk);
      const int64_t rowb = p.sqk * (int64_t)sizeof(IT);
#pragma unroll
      for (int q = KQ0; q < KQ1; ++q) {
        const int o = 1024 * q + 16 * x.lane, r = o / K::RB, pc = (o % K::RB) >> 4;
        const int lc = pc ^ kswz<CT, K::NCH>(r);
        dma_block(base + min(r, n - 1) * rowb + (lc << 4), s + 1024 * q);
      }
    }
    if constexpr (Q1 > NDK) {
      const char* uf = static_cast<const char*>(p.Uf) + ((cg * p.Hv + x.h) * NU * 64 + x.lane) * 16;
#pragma unroll
      for (int q = (Q0 > NDK ? Q0 : NDK); q < Q1; ++q) {
        if (q < NDK + NU)
          dma_block(uf + (q - NDK) * 1024, s + K::UOFF + (q - NDK) * 1024);
        else
          dma_block(reinterpret_cast<const char*>(p.sc + (cg * p.Hv + x.h) * 256) + x.lane * 16, s + K::SOFF);
      }
    }
  };
  for (int c = 0; c < K::D0 - 1; ++c)
    if (c < x.nchunks) issue(c);
  if constexpr (!FAST && LW == 0)
    for (int c = 0; c <= PREF && c < x.nchunks; ++c) carry_keys_slow<CT, IT, DK, VL>(p, x, slot(c), c);
  wait_vmcnt<0>();
  lds_barrier();  // prologue
  for (int i = 0; i < x.nchunks; ++i) {
    if (i + K::D0 - 1 < x.nchunks) {
      issue(i + K::D0 - 1);
      // chunk i+1 (prefetching recurrence: i+2) has landed: what may still
      // be in flight is this wave's requests for the chunks after it
      constexpr int AHEAD = K::D0 - 2 - PREF;
      wait_vmcnt<AHEAD * PER>();
    } else {
      wait_vmcnt<0>();
    }
    if constexpr (!FAST && LW == 0)
      if (i + 1 + PREF < x.nchunks) carry_keys_slow<CT, IT, DK, VL>(p, x, slot(i + 1 + PREF), i + 1 + PREF);
    lds_barrier();  // end of chunk i
  }
  lds_barrier();  // outputs of the last chunk
}

template <class CT, class IT, int DK, bool VL, int LW>
__device__ __forceinline__ void carry_loader_fs(const ScanParams& p, const CarryCtx& x, char* ring) {
  if (p.vec_qk && p.dk == DK)
    carry_loader_w<CT, IT, DK, VL, LW, true>(p, x, ring);
  else
    carry_loader_w<CT, IT, DK, VL, LW, false>(p, x, ring);
}

template <class CT, class IT, int DK, bool VL>
__device__ __forceinline__ void carry_loader(const ScanParams& p, const CarryCtx& x, int lw, char* ring) {
  typedef Carry<CT, IT, DK> K;
  static_assert(K::NLOAD >= 1 && K::NLOAD <= 3, "one to three loader waves");
  static_assert(K::PERW * K::NLOAD >= K::NITEM && K::PERW * (K::NLOAD - 1) < K::NITEM, "items dealt to every loader");
  if (lw == 0) carry_loader_fs<CT, IT, DK, VL, 0>(p, x, ring);
  if constexpr (K::NLOAD > 1) {
    if (lw == 1) carry_loader_fs<CT, IT, DK, VL, 1>(p, x, ring);
  }
  if constexpr (K::NLOAD > 2) {
    if (lw == 2) carry_loader_fs<CT, IT, DK, VL, 2>(p, x, ring);
  }
}

// Recurrence wave R of NREC: it holds the KPR k-blocks KB0 = R KPR.. of the
// state (its 16-row tiles S0 = R SPR..).  Per chunk i (slot i % D0):
//   X_R = K_R S_R (raw key columns of those k-blocks),
//   P_R = -(a e^gam) X_R, plus V in wave 0 (beta is folded into U and N),
//   Y = P_0 + P_1 + ... (exchanged in LDS, summed in the same order by all),
//   S_R <- e^gam_last S_R + U_R Y (the wave's rows of U).
// With one wave this is Y = V - (a e^gam) K S.  S_i and Y_i go to the output
// waves through `hand`.
template <class CT, class IT, int DK, bool VL, bool CAP, int R>
__device__ __forceinline__ void carry_recurrence(const ScanParams& p, const CarryCtx& x, const char* ring,
                                                 typename Mma<CT>::frag* hand, float4_t* xch, unsigned* xflag) {
  typedef Carry<CT, IT, DK> K;
  typedef typename K::G G;
  typedef typename K::frag frag;
  constexpr int NKX = G::NKX, NKT = G::NKT, NBU = G::NBU, KB = G::KB, EPF = G::EPF;
  constexpr int NREC = K::NREC, KPR = K::KPR, SPR = K::SPR, KB0 = R * KPR, S0 = R * SPR;
  const int lane = x.lane, grp = x.grp, col = x.col;
  const int dk = p.dk, dv = p.dv;
  const float* init = VL ? x.init : p.initial;
  float* fin = VL ? x.fin : p.final_state;

  float4_t S[SPR];
#pragma unroll
  for (int s = 0; s < SPR; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = slot_index<CT>(S0 + s, 4 * grp + i);
      float v = 0.0f;
      if (init && row < dk && x.col_ok) v = init[((int64_t)x.h * dk + row) * dv + x.jc];
      S[s][i] = v;
    }
  frag Sf[KPR];
#pragma unroll
  for (int k = 0; k < KPR; ++k) Sf[k] = pack_frag(S, k, CT(0));

  // wave 0: v two chunks ahead in registers (this lane's 16 X-rows); rows
  // past the end of the sequence fall outside the buffer range (read 0), and
  // so do columns past dv: their lanes add 2^31 to every offset (a chunk's
  // range is at most 64 rows of 2^22 four-byte elements, 2^30 bytes, so the
  // sum stays in 32 bits and past the range).  Branch-free offsets keep the
  // loads unconditional, so they stay in flight across the loop.
  const IT* vbase = static_cast<const IT*>(p.v) + (int64_t)x.h * dv + x.j0;
  const uint32_t vlane = (uint32_t)col * (uint32_t)sizeof(IT) + (x.col_ok ? 0u : 0x80000000u);
  const uint32_t vrow = (uint32_t)p.sv * (uint32_t)sizeof(IT);
  auto load_v = [&](uint32_t* vb, int c) {
    int t0, n;
    chunk_of(x, min(c, x.nchunks - 1), t0, n);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(vbase + (int64_t)t0 * p.sv, n * (int)p.sv * (int)sizeof(IT));
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        vb[4 * t + j] = buffer_load_bits<IT>(r, (int)((uint32_t)slot_index<CT>(t, 4 * grp + j) * vrow + vlane));
  };
  constexpr int NV = R == 0 ? 16 : 1;
  uint32_t va[NV], vb[NV];
  if constexpr (R == 0) {
    load_v(va, 0);
    load_v(vb, 1);
  }
  // this lane's key rows (slot order) and k offset within each k-block
  int krow[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) krow[t] = slot_index<CT>(t, col);
  frag kf[4][KPR];
  auto load_k = [&](int c) {
    const char* slot = ring + (c % K::D0) * K::SLOT;
#pragma unroll
    for (int k = 0; k < KPR; ++k)
#pragma unroll
      for (int t = 0; t < 4; ++t) kf[t][k] = key_frag<CT, IT, DK>(slot, krow[t], (KB0 + k) * KB + grp * EPF);
  };
  lds_barrier();  // prologue
  if constexpr (K::PREF) load_k(0);

  auto step = [&](int i, uint32_t* vbuf) {
    const char* slot = ring + (i % K::D0) * K::SLOT;
    const frag* uslot = reinterpret_cast<const frag*>(slot + K::UOFF);
    const float* scs = reinterpret_cast<const float*>(slot + K::SOFF);  // a e^gam, b e^gam, gam, e^gam
    frag* hs = hand + (i & 1) * (NKX + NKT) * 64;
    // the chunk's keys: read during the previous chunk, or up front
    if constexpr (!K::PREF) load_k(i);
    float4_t ya[4], X[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) ya[t] = *reinterpret_cast<const float4_t*>(scs + slot_index<CT>(t, 4 * grp));
    // the wave's U rows: into the key registers once the last product has
    // taken its operands (f32, four recurrence waves: after its partial
    // product is published, for want of registers)
    constexpr bool EARLY_U = NREC <= 2;
    frag uf[SPR][NKT];
    auto load_u = [&]() {
#pragma unroll
      for (int s = 0; s < SPR; ++s)
#pragma unroll
        for (int b = 0; b < NKT; ++b) uf[s][b] = uslot[((S0 + s) * NKT + b) * 64 + lane];
    };
    const float el = scs[192 + kC - 1];
    // S_i goes to the output waves
#pragma unroll
    for (int k = 0; k < KPR; ++k) hs[(KB0 + k) * 64 + lane] = Sf[k];
#pragma unroll
    for (int t = 0; t < 4; ++t) X[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < KPR; ++k) {
#pragma unroll
      for (int t = 0; t < 4; ++t) Mma<CT>::mma(X[t], kf[t][k], Sf[k]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EARLY_U) {
      load_u();
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (R == 0)
          X[t][j] = bits_value<IT>(vbuf[4 * t + j]) - ya[t][j] * X[t][j];
        else
          X[t][j] = -(ya[t][j] * X[t][j]);
      }
    if constexpr (NREC > 1) {
      float4_t* mine = xch + R * 4 * 64;
#pragma unroll
      for (int t = 0; t < 4; ++t) mine[t * 64 + lane] = X[t];
      lds_publish(xflag, R, i + 1);
      if constexpr (!EARLY_U) load_u();
      lds_wait_all(xflag, NREC, i + 1);
      if constexpr (EARLY_U) {
        // the other waves' partials, all requested before the first sum
        float4_t px[NREC][4];
#pragma unroll
        for (int r = 0; r < NREC; ++r)
#pragma unroll
          for (int t = 0; t < 4; ++t) px[r][t] = r == R ? X[t] : xch[(r * 4 + t) * 64 + lane];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float4_t acc = px[0][t];
#pragma unroll
          for (int r = 1; r < NREC; ++r) acc = acc + px[r][t];
          X[t] = acc;
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float4_t acc = R == 0 ? X[t] : xch[t * 64 + lane];
#pragma unroll
          for (int r = 1; r < NREC; ++r) acc = acc + (r == R ? X[t] : xch[(r * 4 + t) * 64 + lane]);
          X[t] = acc;
        }
      }
    }
    frag Yf[NKT];
#pragma unroll
    for (int b = 0; b < NKT; ++b) Yf[b] = pack_frag(X, b, CT(0));
    if (CAP && i == x.cap_chunk) {
      // state after token `capture`: exp(gam_r*) S_i + Ucap Y_i
      const float ec = decay_exp(scs[128 + x.cap_row]);
      const frag* uc = static_cast<const frag*>(p.Ucf) + (int64_t)x.h * NBU * 64 + lane;
#pragma unroll
      for (int s = 0; s < SPR; ++s) {
        float4_t acc = S[s] * ec;
#pragma unroll
        for (int b = 0; b < NKT; ++b) Mma<CT>::mma(acc, uc[((S0 + s) * NKT + b) * 64], Yf[b]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = slot_index<CT>(S0 + s, 4 * grp + j);
          if (row < dk && x.col_ok) p.captured[((int64_t)x.h * dk + row) * dv + x.jc] = acc[j];
        }
      }
    }
    // Y_i goes to the output waves
    if constexpr (R == 0) {
#pragma unroll
      for (int b = 0; b < NKT; ++b) hs[(NKX + b) * 64 + lane] = Yf[b];
    }
    __builtin_amdgcn_sched_barrier(0);
    // S <- exp(gam_last) S + U Y: each tile's rescale is issued while the
    // previous tile's product runs, and the next chunk's keys are requested
    // once the U operands are in
#pragma unroll
    for (int s = 0; s < SPR; ++s) {
      S[s] = S[s] * el;
      Mma<CT>::mma(S[s], uf[s][0], Yf[0]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 1; b < NKT; ++b) {
#pragma unroll
      for (int s = 0; s < SPR; ++s) Mma<CT>::mma(S[s], uf[s][b], Yf[b]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (K::PREF) load_k(i + 1);
#pragma unroll
    for (int k = 0; k < KPR; ++k) Sf[k] = pack_frag(S, k, CT(0));
    if constexpr (R == 0) load_v(vbuf, i + 2);
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
    for (int s = 0; s < SPR; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = slot_index<CT>(S0 + s, 4 * grp + j);
        if (row < dk && x.col_ok) fin[((int64_t)x.h * dk + row) * dv + x.jc] = S[s][j];
      }
  }
}

// Output waves: O of chunk c during chunk c+1, TPW tiles of 16 rows (token
// order) from row 16 TPW ow: O = diag(b e^gam) (Q S) + N Y.  Query rows, N
// blocks and the row factors are loaded into registers OD chunks ahead.
template <class CT, class IT, int DK, class OT, bool VL, bool VEC>
__device__ __forceinline__ void carry_outputs(const ScanParams& p, const CarryCtx& x, int ow,
                                              const typename Mma<CT>::frag* hand) {
  typedef Carry<CT, IT, DK> K;
  typedef typename K::G G;
  typedef typename K::frag frag;
  constexpr int NKX = G::NKX, NKT = G::NKT, KB = G::KB, EPF = G::EPF, OD = K::OD, TPW = K::TPW;
  const int lane = x.lane, grp = x.grp, col = x.col;
  struct Ops {
    frag q[TPW][NKX];
    frag nn[TPW][NKT];
    float4_t yo[TPW];
  };
  auto load_o = [&](Ops& o, int c) {
    const int cc = min(c, x.nchunks - 1);
    int t0, n;
    chunk_of(x, cc, t0, n);
    const int64_t cg = (VL ? x.c0 : 0) + cc;
    const frag* nf = static_cast<const frag*>(p.Nf) + (cg * p.Hv + x.h) * G::NBN * 64 + lane;
    const float* scs = p.sc + (cg * p.Hv + x.h) * 256;
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      const int t = TPW * ow + tt;
      const IT* qrow = static_cast<const IT*>(p.q) + (int64_t)(t0 + min(16 * t + col, n - 1)) * p.sqk +
                       (int64_t)x.hk * p.dk;
#pragma unroll
      for (int kb = 0; kb < NKX; ++kb) o.q[tt][kb] = query_frag<CT, IT, VEC>(qrow, kb * KB + grp * EPF, p.dk);
#pragma unroll
      for (int b = 0; b < NKT; ++b) o.nn[tt][b] = nf[(t * NKT + b) * 64];
      o.yo[tt] = *reinterpret_cast<const float4_t*>(scs + 64 + 16 * t + 4 * grp);
    }
  };
  Ops ops[OD];
#pragma unroll
  for (int d = 0; d < OD; ++d) load_o(ops[d], d);
  const OT* out = static_cast<const OT*>(p.out) + (int64_t)x.h * p.dv + x.j0;
  // branch-free store offsets: columns past dv add 2^31 (past the range)
  const uint32_t olane = (uint32_t)col * (uint32_t)sizeof(OT) + (x.col_ok ? 0u : 0x80000000u);
  const uint32_t orow = (uint32_t)p.so * (uint32_t)sizeof(OT);
  lds_barrier();  // prologue
  lds_barrier();  // chunk 0 (no outputs yet)
  auto ostep = [&](int c, Ops& o) {
    const frag* hs = hand + (c & 1) * (NKX + NKT) * 64;
    frag sf[NKX], yf[NKT];
#pragma unroll
    for (int kb = 0; kb < NKX; ++kb) sf[kb] = hs[kb * 64 + lane];
#pragma unroll
    for (int b = 0; b < NKT; ++b) yf[b] = hs[(NKX + b) * 64 + lane];
    int t0, n;
    chunk_of(x, c, t0, n);
    // rows past the end of the sequence fall outside the buffer range: dropped
    const __amdgpu_buffer_rsrc_t r = make_rsrc(out + (int64_t)t0 * p.so, n * (int)p.so * (int)sizeof(OT));
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      const int t = TPW * ow + tt;
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < NKX; ++kb) Mma<CT>::mma(acc, o.q[tt][kb], sf[kb]);
      acc = acc * o.yo[tt];
#pragma unroll
      for (int b = 0; b < NKT; ++b) Mma<CT>::mma(acc, o.nn[tt][b], yf[b]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        buffer_store(r, (int)((uint32_t)(16 * t + 4 * grp + j) * orow + olane), acc[j], OT(0));
    }
    load_o(o, c + OD);
    lds_barrier();  // end of chunk c+1
  };
  int c = 0;
  for (; c + OD <= x.nchunks; c += OD)
#pragma unroll
    for (int d = 0; d < OD; ++d) ostep(c + d, ops[d]);
  // the last chunks; compile-time indices keep ops in registers
#pragma unroll
  for (int d = 0; d + 1 < OD; ++d)
    if (c + d < x.nchunks) ostep(c + d, ops[d]);
}

// MODE 0: one sequence; 1: one sequence with a captured state; 2: a ragged batch.
template <class CT, class IT, int DK, int MODE>
__global__ __launch_bounds__((Carry<CT, IT, DK>::THREADS)) void scan_carry(ScanParams p) {
  typedef Carry<CT, IT, DK> K;
  constexpr bool VL = MODE == 2, CAP = MODE == 1;
  __shared__ __attribute__((aligned(1024))) char ring[K::D0 * K::SLOT];
  __shared__ __attribute__((aligned(16))) typename K::frag hand[2 * (K::G::NKX + K::G::NKT) * 64];
  __shared__ __attribute__((aligned(16))) float4_t xch[K::NREC > 1 ? K::NREC * 4 * 64 : 1];
  __shared__ unsigned xflag[1];
  if (threadIdx.x == 0) xflag[0] = 0;  // before the prologue barrier

  CarryCtx x;
  x.lane = threadIdx.x & 63;
  x.col = x.lane & 15;
  x.grp = x.lane >> 4;
  const int wave = wave_id();
  // XCD-aware placement: logical work-group L, consecutive L share a k-head,
  // and work-group b runs on XCD b % 8, so a contiguous eighth of the L of a
  // sequence goes to each XCD (its k-heads' keys and queries stay in that
  // XCD's L2).  A ragged batch keeps its launch order (sequences with the most
  // chunks first) and applies the map within each sequence's block.
  const int nwg = gridDim.x;
  const int ntiles = (p.dv + kVT - 1) / kVT;
  const int per_seq = p.Hv * ntiles;
  int L = blockIdx.x;
  if (!VL && (nwg & 7) == 0) {
    L = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  } else if (VL && (per_seq & 7) == 0) {
    const int b = L % per_seq;
    L += (b & 7) * (per_seq >> 3) + (b >> 3) - b;
  }
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
  x.t0s = 0;
  x.lens = p.T;
  if (VL) {  // the first and last chunk of the sequence
    const int2 a = p.chunk_tab[x.c0], z = p.chunk_tab[x.c0 + x.nchunks - 1];
    x.t0s = a.x;
    x.lens = z.x + z.y - a.x;
  }
  if (wave < K::NREC) {
    if (wave == 0) carry_recurrence<CT, IT, DK, VL, CAP, 0>(p, x, ring, hand, xch, xflag);
    if constexpr (K::NREC > 1) {
      if (wave == 1) carry_recurrence<CT, IT, DK, VL, CAP, 1>(p, x, ring, hand, xch, xflag);
    }
    if constexpr (K::NREC > 2) {
      if (wave == 2) carry_recurrence<CT, IT, DK, VL, CAP, 2>(p, x, ring, hand, xch, xflag);
      if (wave == 3) carry_recurrence<CT, IT, DK, VL, CAP, 3>(p, x, ring, hand, xch, xflag);
    }
  } else if (wave < K::NREC + K::NLOAD) {
    carry_loader<CT, IT, DK, VL>(p, x, wave - K::NREC, ring);
  } else {
    const int ow = wave - K::NREC - K::NLOAD;
    const bool vec = p.vec_qk && p.dk == DK;
    if (p.dtype_out == 0) {
      if (vec)
        carry_outputs<CT, IT, DK, float, VL, true>(p, x, ow, hand);
      else
        carry_outputs<CT, IT, DK, float, VL, false>(p, x, ow, hand);
    } else {
      if (vec)
        carry_outputs<CT, IT, DK, half_t, VL, true>(p, x, ow, hand);
      else
        carry_outputs<CT, IT, DK, half_t, VL, false>(p, x, ow, hand);
    }
  }
}

template <class CT, class IT, int DK>
int launch_dk(const ScanParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((scan_prepare<CT, IT, DK>), dim3(p.nchunks, p.Hk), dim3(64 * kPW), 0, stream, p);
  int rc = check_launch("scan_prepare");
  if (rc) return rc;
  const int ntiles = (p.dv + kVT - 1) / kVT;
  const int nseq = p.seq_tab ? p.nseq : 1;
  const dim3 block(Carry<CT, IT, DK>::THREADS);
  if (p.seq_tab)
    hipLaunchKernelGGL((scan_carry<CT, IT, DK, 2>), dim3(nseq * p.Hv * ntiles), block, 0, stream, p);
  else if (p.capture > 0)
    hipLaunchKernelGGL((scan_carry<CT, IT, DK, 1>), dim3(p.Hv * ntiles), block, 0, stream, p);
  else
    hipLaunchKernelGGL((scan_carry<CT, IT, DK, 0>), dim3(p.Hv * ntiles), block, 0, stream, p);
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
