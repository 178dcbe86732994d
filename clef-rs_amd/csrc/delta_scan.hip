// Chunked gated-DeltaNet scan for gfx950.
//
// Semantics: delta_recurrence_prefill (crates/core/src/models/qwen.rs:826-882)
// with repeat-interleave GQA (qwen.rs:727-738); chunkwise algebra as in
// crates/core/src/models/chunk.metal:10-164, restated for C = 64.
//
// For one v-head and a chunk of C tokens with in-chunk cumulative log-decay
// gam_r = sum_{j<=r} g_j (padding rows have g = 0, beta = 0, k = q = v = 0),
// with k^, q^ the normalised keys and scaled queries:
//   A[r][c] = beta_r (k^_r.k^_c) exp(gam_r - gam_c)  (c < r);  Tm = (I + A)^-1
//   M[r][c] = (q^_r.k^_c) exp(gam_r - gam_c)          (c <= r)
//   Y       = diag(beta) (V - diag(exp gam) K^ S)
//   Delta   = Tm Y
//   O       = diag(exp gam) Q^ S + M Delta
//   S'      = exp(gam_last) S + K^^T diag(exp(gam_last - gam)) Delta
// Decay ratios are only formed for c <= r, so g = -1000 underflows to exact
// zeros instead of dividing by an underflowed prefix product.
//
// scan_prepare (grid chunks x Hv, fully parallel) does everything that does
// not depend on the state: it normalises the chunk's q and k rows, forms
// K K^T and Q K^T on MFMA, turns the accumulators directly into A (LDS) and
// M (workspace), inverts I + A by forward substitution, and writes the
// per-row factors exp(gam), exp(gam_last - gam), beta, the row scales of the
// raw q/k rows and the normalised K^T of the chunk.
//
// scan_carry (grid Hv x ceil(dv/16)) runs the chunks in order for one v-head
// and 16 value columns (the columns of S evolve independently).  The f32
// state lives in MFMA accumulators over 4 waves.  Every operand is loaded
// straight from global memory into MFMA fragment registers, one chunk ahead
// (each register set is refilled right after its last use), so a chunk is
// [K;Q] S -> Y -> Tm Y -> (M Delta | K^T Delta) with three LDS hand-offs.
// Work-groups sharing a k-head are placed on one XCD so its rows come from
// that XCD's L2.
#include "common.hpp"
#include "scan.hpp"

namespace clef {
namespace {

constexpr int kC = 64;   // chunk length
constexpr int kVT = 16;  // value columns per carry work-group

template <class T> struct Vec16;  // 16-byte vector of T
template <> struct Vec16<float> { typedef float4_t type; static constexpr int n = 4; };
template <> struct Vec16<half_t> { typedef half8 type; static constexpr int n = 8; };

__device__ __forceinline__ void store_scalar(void* p, int64_t i, int dtype, float v) {
  if (dtype == 0)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<half_t*>(p)[i] = static_cast<half_t>(v);
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

// An MFMA fragment (16 bytes of CT) from EPF consecutive elements of a row of
// IT elements, addresses clamped into the row.
template <class CT, class IT>
__device__ __forceinline__ typename Mma<CT>::frag load_frag_row(const IT* row, int e0, int dk, bool vec_ok) {
  constexpr int EPF = 16 / sizeof(CT);
  typename Mma<CT>::frag f;
  if (sizeof(CT) == sizeof(IT) && vec_ok)
    return *reinterpret_cast<const typename Mma<CT>::frag*>(row + min(e0, dk - EPF));
#pragma unroll
  for (int i = 0; i < EPF; ++i) f[i] = static_cast<CT>(row[min(e0 + i, dk - 1)]);
  return f;
}

__device__ __forceinline__ uint32_t load_bits(const void* p, int64_t i, int dtype) {
  return dtype == 0 ? static_cast<const uint32_t*>(p)[i] : static_cast<const uint16_t*>(p)[i];
}

__device__ __forceinline__ float bits_to_f32(uint32_t b, int dtype) {
  if (dtype == 0) return __uint_as_float(b);
  const uint16_t h = static_cast<uint16_t>(b);
  return static_cast<float>(*reinterpret_cast<const half_t*>(&h));
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------------------
// Kernel 1: per (chunk, v-head) preparation.
// ---------------------------------------------------------------------------
template <class CT, class IT, int DK>
__global__ __launch_bounds__(256) void scan_prepare(ScanParams p) {
  constexpr int VI = Vec16<IT>::n;       // input elements per 16-byte vector
  constexpr int TPR = DK / VI;           // threads per row
  constexpr int RPP = 256 / TPR;         // rows per pass
  constexpr int NPASS = (2 * kC) / RPP;
  constexpr int EPF = 16 / sizeof(CT);   // compute elements per fragment lane
  constexpr int KB = Mma<CT>::kBlock;
  constexpr int LDR = DK + EPF;          // padded LDS row (elements)
  static_assert(TPR <= 64 && (TPR & (TPR - 1)) == 0, "row group must fit a wave");

  __shared__ __attribute__((aligned(16))) CT sK[kC * LDR];
  __shared__ __attribute__((aligned(16))) CT sQ[kC * LDR];
  __shared__ __attribute__((aligned(16))) float sAT[kC * kC];  // A^T: [c][r]
  __shared__ float sGam[kC];
  __shared__ float sBeta[kC];

  const int chunk = blockIdx.x, h = blockIdx.y;
  const int rep = p.Hv / p.Hk;
  const int hk = h / rep;
  const bool kv_writer = (h % rep) == 0;  // one writer of the per-k-head outputs
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int t0 = chunk * kC;
  const int n = min(kC, p.T - t0);
  const int dk = p.dk;
  const int64_t cv = (int64_t)chunk * p.Hv + h;   // (chunk, v-head) index
  const int64_t ck = (int64_t)chunk * p.Hk + hk;  // (chunk, k-head) index

  // 1. issue every load first: q/k rows (clamped), then g and beta
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
  uint32_t gbits = 0, bbits = 0;
  if (wave == 0) {
    const int64_t gi = (int64_t)(t0 + min(lane, n - 1)) * p.sgb + h;
    gbits = load_bits(p.g, gi, p.dtype_gb);
    bbits = load_bits(p.beta, gi, p.dtype_gb);
  }
  // 2. normalise rows into LDS (l2 with eps inside the sqrt, qwen.rs:837-840)
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    const int rr = ps * RPP + tid / TPR;
    const bool isq = rr >= kC;
    const int r = isq ? rr - kC : rr;
    const int e0 = (tid % TPR) * VI;
    float x[VI];
#pragma unroll
    for (int i = 0; i < VI; ++i) x[i] = (r < n && e0 + i < dk) ? static_cast<float>(raw[ps][i]) : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VI; ++i) s += x[i] * x[i];
#pragma unroll
    for (int off = 1; off < TPR; off <<= 1) s += __shfl_xor(s, off, 64);
    const float inv = 1.0f / sqrtf(s + 1e-6f);
    const float scale = isq ? inv * p.qscale : inv;
    CT* dst = (isq ? sQ : sK) + r * LDR + e0;
#pragma unroll
    for (int i = 0; i < VI; ++i) dst[i] = static_cast<CT>(x[i] * scale);
    if (kv_writer && tid % TPR == 0) (isq ? p.scq : p.invk)[ck * kC + r] = r < n ? scale : 0.0f;
  }
  // 3. in-chunk cumulative decay and the per-row factors
  if (wave == 0) {
    const float gv = lane < n ? bits_to_f32(gbits, p.dtype_gb) : 0.0f;
    const float bv = lane < n ? bits_to_f32(bbits, p.dtype_gb) : 0.0f;
    float cs = gv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(cs, off, 64);
      if (lane >= off) cs += o;
    }
    const float gl = __shfl(cs, kC - 1, 64);
    sGam[lane] = cs;
    sBeta[lane] = bv;
    p.eg[cv * kC + lane] = expf(cs);
    p.wl[cv * kC + lane] = expf(gl - cs);
    p.bt[cv * kC + lane] = bv;
    p.gam_ws[cv * kC + lane] = cs;
  }
  lds_barrier();

  // 4. Gram tiles on MFMA, turned directly into A (LDS, transposed) and M.
  //    Lower tiles of K K^T and Q K^T; the strictly upper tiles of M are zero.
  {
    const int col = lane & 15, grp = lane >> 4;
    CT* Mout = static_cast<CT*>(p.Mm) + cv * kC * kC;
    for (int ti = wave; ti < 32; ti += 4) {
      const int mat = ti >> 4, tr = (ti >> 2) & 3, tc = ti & 3;
      const int c = tc * 16 + col;
      if (tc > tr) {  // strictly upper tile: M is zero there, A is never read
        if (mat == 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i) Mout[(tr * 16 + grp * 4 + i) * kC + c] = CT(0);
        }
        continue;
      }
      const CT* a_src = (mat ? sQ : sK) + (tr * 16 + col) * LDR + grp * EPF;
      const CT* b_src = sK + (tc * 16 + col) * LDR + grp * EPF;
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < DK / KB; ++kb)
        Mma<CT>::mma(acc, load_frag<CT>(a_src + kb * KB), load_frag<CT>(b_src + kb * KB));
      const float gc = sGam[c];
      float4_t out;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = tr * 16 + grp * 4 + i;
        const float d = (c <= r) ? expf(sGam[r] - gc) : 0.0f;
        if (mat == 0)
          out[i] = (c < r) ? (sBeta[r] * acc[i]) * d : 0.0f;
        else
          Mout[r * kC + c] = static_cast<CT>((c <= r) ? acc[i] * d : 0.0f);
      }
      if (mat == 0) *reinterpret_cast<float4_t*>(&sAT[c * kC + tr * 16 + grp * 4]) = out;
    }
  }
  lds_barrier();

  // 5. wave 0: Tm = (I + A)^-1 by forward substitution, lane j = column j.
  //    waves 1-3: the normalised K^T of the chunk (one writer per k-head).
  if (wave == 0) {
    float t[kC];
#pragma unroll
    for (int r = 0; r < kC; ++r) t[r] = (r == lane) ? 1.0f : 0.0f;
#pragma unroll
    for (int c = 0; c < kC - 1; ++c) {
      const float tc = t[c];
#pragma unroll
      for (int r4 = ((c + 1) / 4) * 4; r4 < kC; r4 += 4) {
        const float4_t a = *reinterpret_cast<const float4_t*>(sAT + c * kC + r4);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (r4 + s > c) t[r4 + s] = fmaf(-a[s], tc, t[r4 + s]);
      }
    }
    CT* Tout = static_cast<CT*>(p.Tm) + cv * kC * kC;
#pragma unroll
    for (int r = 0; r < kC; ++r) Tout[r * kC + lane] = static_cast<CT>(t[r]);
  } else if (kv_writer) {
    // K^T [DK][64]: each item is EPF consecutive tokens of one dk row
    CT* Kt = static_cast<CT*>(p.Kt) + ck * DK * kC;
    for (int it = tid - 64; it < DK * (kC / EPF); it += 192) {
      const int e = it / (kC / EPF), tok0 = (it % (kC / EPF)) * EPF;
      typename Mma<CT>::frag f;
#pragma unroll
      for (int j = 0; j < EPF; ++j) f[j] = sK[(tok0 + j) * LDR + e];
      *reinterpret_cast<typename Mma<CT>::frag*>(Kt + e * kC + tok0) = f;
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential chunk carry for one (v-head, 16 value columns).
// ---------------------------------------------------------------------------
template <class CT, class IT, int DK>
__global__ __launch_bounds__(256) void scan_carry(ScanParams p) {
  constexpr int EPF = 16 / sizeof(CT);
  constexpr int KB = Mma<CT>::kBlock;
  constexpr int LDK = DK + EPF;       // state^T rows [value][dk]
  constexpr int LDT = kC + EPF;       // [value][token] rows
  constexpr int NST = DK / 16;        // state row tiles
  constexpr int SPW = (NST + 3) / 4;  // state tiles per wave
  constexpr int NKB_X = DK / KB;      // k-blocks over dk
  constexpr int NKB_T = kC / KB;      // k-blocks over tokens
  typedef typename Mma<CT>::frag frag;

  __shared__ __attribute__((aligned(16))) CT sSt[kVT * LDK];
  __shared__ __attribute__((aligned(16))) CT sYt[kVT * LDT];
  __shared__ __attribute__((aligned(16))) CT sDt[kVT * LDT];
  __shared__ __attribute__((aligned(16))) CT sDw[kVT * LDT];
  __shared__ __attribute__((aligned(16))) CT sDc[kVT * LDT];
  __shared__ float sGam[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int col = lane & 15, grp = lane >> 4;

  // XCD-aware placement: logical work-group L -> consecutive L share a k-head.
  const int nwg = gridDim.x;
  int L = blockIdx.x;
  if ((nwg & 7) == 0) L = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int ntiles = (p.dv + kVT - 1) / kVT;
  const int rep = p.Hv / p.Hk;
  const int hk = L / (rep * ntiles);
  const int rem = L % (rep * ntiles);
  const int h = hk * rep + rem / ntiles;
  const int j0 = (rem % ntiles) * kVT;
  const int dk = p.dk, dv = p.dv;
  const int jc = j0 + col;  // this lane's value column
  const bool col_ok = jc < dv;
  const int jcc = min(jc, dv - 1);
  const bool kwave = wave < 2;  // waves 0,1 own the K rows of [K;Q], waves 2,3 the Q rows

  // ---- state in accumulators: tile s of this wave covers dk rows 16*(wave+4s)..
  float4_t S[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    const int tile = wave + 4 * s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = tile * 16 + grp * 4 + i;
      float v = 0.0f;
      if (p.initial && tile < NST && row < dk && col_ok) v = p.initial[((int64_t)h * dk + row) * dv + jc];
      S[s][i] = v;
    }
  }
  auto store_state_lds = [&]() {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int tile = wave + 4 * s;
      if (tile < NST) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sSt[col * LDK + tile * 16 + grp * 4 + i] = static_cast<CT>(S[s][i]);
      }
    }
  };

  // ---- operand registers, each refilled right after its last use
  const IT* xbase = static_cast<const IT*>(kwave ? p.k : p.q);
  const IT* vbase = static_cast<const IT*>(p.v);
  frag xf[2][NKB_X];    // [K;Q] rows of this wave's two row tiles (raw input values)
  float xs[2][4];       // row scales 1/|k| or qscale/|q| of those rows
  float egx[2][4];      // exp(gam) of those rows
  float bv[2][4];       // beta (waves 0,1)
  IT vr[2][4];          // V (waves 0,1)
  frag tf[NKB_T];       // Tm rows of tile `wave`
  float wlr[4];         // exp(gam_last - gam) of the Delta rows of tile `wave`
  frag mf[2][NKB_T];    // M rows (waves 2,3)
  frag kf[SPW][NKB_T];  // K^T rows (dk) of this wave's state tiles
  float el = 0.0f;      // exp(gam_last)
  float gam_l = 0.0f;   // gam of token `lane` (capture only)

  auto load_x = [&](int chunk) {
    const int t0 = chunk * kC, n = min(kC, p.T - t0);
    const int64_t cv = (int64_t)chunk * p.Hv + h, ck = (int64_t)chunk * p.Hk + hk;
    const float* scale = kwave ? p.invk : p.scq;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int r = (wave & 1) * 32 + s * 16 + col;  // fragment row
      const IT* row = xbase + (int64_t)(t0 + min(r, n - 1)) * p.sqk + (int64_t)hk * dk;
#pragma unroll
      for (int kb = 0; kb < NKB_X; ++kb) xf[s][kb] = load_frag_row<CT, IT>(row, kb * KB + grp * EPF, dk, p.vec_qk);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ri = (wave & 1) * 32 + s * 16 + grp * 4 + i;  // accumulator row
        xs[s][i] = scale[ck * kC + ri];
        egx[s][i] = p.eg[cv * kC + ri];
      }
    }
  };
  auto load_y = [&](int chunk) {  // waves 0,1
    const int t0 = chunk * kC, n = min(kC, p.T - t0);
    const int64_t cv = (int64_t)chunk * p.Hv + h;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wave * 32 + s * 16 + grp * 4 + i;
        vr[s][i] = vbase[(int64_t)(t0 + min(r, n - 1)) * p.sv + (int64_t)h * dv + jcc];
        bv[s][i] = p.bt[cv * kC + r];
      }
  };
  auto load_t = [&](int chunk) {
    const int64_t cv = (int64_t)chunk * p.Hv + h;
    const CT* Tm = static_cast<const CT*>(p.Tm) + cv * kC * kC;
#pragma unroll
    for (int kb = 0; kb < NKB_T; ++kb) tf[kb] = load_frag<CT>(Tm + (wave * 16 + col) * kC + kb * KB + grp * EPF);
#pragma unroll
    for (int i = 0; i < 4; ++i) wlr[i] = p.wl[cv * kC + wave * 16 + grp * 4 + i];
    el = p.eg[cv * kC + kC - 1];
    gam_l = p.gam_ws[cv * kC + lane];
  };
  auto load_m = [&](int chunk) {  // waves 2,3
    const int64_t cv = (int64_t)chunk * p.Hv + h;
    const CT* Mm = static_cast<const CT*>(p.Mm) + cv * kC * kC;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb)
        mf[s][kb] = load_frag<CT>(Mm + ((wave - 2) * 32 + s * 16 + col) * kC + kb * KB + grp * EPF);
  };
  auto load_k = [&](int chunk) {
    const int64_t ck = (int64_t)chunk * p.Hk + hk;
    const CT* Kt = static_cast<const CT*>(p.Kt) + ck * DK * kC;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int tile = min(wave + 4 * s, NST - 1);
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb) kf[s][kb] = load_frag<CT>(Kt + (tile * 16 + col) * kC + kb * KB + grp * EPF);
    }
  };

  const int nchunks = p.nchunks;
  const int cap_chunk = p.capture > 0 ? (p.capture - 1) / kC : -1;
  const int cap_row = p.capture > 0 ? (p.capture - 1) % kC : -1;
  load_x(0);
  if (kwave) load_y(0);
  load_t(0);
  if (!kwave) load_m(0);
  load_k(0);
  store_state_lds();
  lds_barrier();
  for (int chunk = 0; chunk < nchunks; ++chunk) {
    const int t0 = chunk * kC;
    const int n = min(kC, p.T - t0);
    const bool more = chunk + 1 < nchunks;
    // ---- X = [K;Q] S for this wave's two row tiles, scaled per row
    float4_t X[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) X[s] = float4_t{0.f, 0.f, 0.f, 0.f};
    {
      const CT* bsrc = sSt + col * LDK + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < NKB_X; ++kb) {
        const frag bf = load_frag<CT>(bsrc + kb * KB);
#pragma unroll
        for (int s = 0; s < 2; ++s) Mma<CT>::mma(X[s], xf[s][kb], bf);
      }
    }
    float sx[2][4], ex[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) sx[s][i] = xs[s][i], ex[s][i] = egx[s][i];
    if (more) load_x(chunk + 1);
    // ---- waves 0,1: Y = beta (V - exp(gam) K^ S) -> Y^T in LDS; waves 2,3: O = exp(gam) Q^ S
    float4_t O[2];
    if (kwave) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int rbase = wave * 32 + s * 16 + grp * 4;
        CT y4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = (rbase + i < n && col_ok) ? static_cast<float>(vr[s][i]) : 0.0f;
          y4[i] = static_cast<CT>(bv[s][i] * (v - ex[s][i] * (X[s][i] * sx[s][i])));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sYt[col * LDT + rbase + i] = y4[i];
      }
      if (more) load_y(chunk + 1);
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) O[s][i] = ex[s][i] * (X[s][i] * sx[s][i]);
    }
    lds_barrier();  // (B) Y^T ready

    // ---- Delta = Tm Y : wave w -> row tile w
    const float el_c = el;
    {
      float4_t D = {0.f, 0.f, 0.f, 0.f};
      const CT* bsrc = sYt + col * LDT + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb) Mma<CT>::mma(D, tf[kb], load_frag<CT>(bsrc + kb * KB));
      const int rbase = wave * 16 + grp * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sDt[col * LDT + rbase + i] = static_cast<CT>(D[i]);
        sDw[col * LDT + rbase + i] = static_cast<CT>(D[i] * wlr[i]);
      }
      if (chunk == cap_chunk) {  // Delta weighted for the state after token `capture`
        if (wave == 0) sGam[lane] = gam_l;
        lds_barrier();
        const float gc = sGam[cap_row];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rbase + i;
          sDc[col * LDT + r] = static_cast<CT>(r <= cap_row ? D[i] * expf(gc - sGam[r]) : 0.0f);
        }
      }
    }
    if (more) load_t(chunk + 1);
    lds_barrier();  // (C) Delta^T ready

    // ---- waves 2,3: O += M Delta, store
    if (!kwave) {
      const CT* bsrc = sDt + col * LDT + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb) {
        const frag bf = load_frag<CT>(bsrc + kb * KB);
#pragma unroll
        for (int s = 0; s < 2; ++s) Mma<CT>::mma(O[s], mf[s][kb], bf);
      }
      if (more) load_m(chunk + 1);
      if (col_ok) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = (wave - 2) * 32 + s * 16 + grp * 4 + i;
            if (r < n)
              store_scalar(p.out, (int64_t)(t0 + r) * p.so + (int64_t)h * dv + jc, p.dtype_out, O[s][i]);
          }
      }
    }
    // ---- optional capture of the state after token `capture`
    if (chunk == cap_chunk) {
      const float ec = expf(sGam[cap_row]);
#pragma unroll
      for (int s = 0; s < SPW; ++s) {
        const int tile = wave + 4 * s;
        if (tile < NST) {
          float4_t acc = S[s] * ec;
          const CT* bsrc = sDc + col * LDT + grp * EPF;
#pragma unroll
          for (int kb = 0; kb < NKB_T; ++kb) Mma<CT>::mma(acc, kf[s][kb], load_frag<CT>(bsrc + kb * KB));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = tile * 16 + grp * 4 + i;
            if (row < dk && col_ok) p.captured[((int64_t)h * dk + row) * dv + jc] = acc[i];
          }
        }
      }
    }
    // ---- S <- exp(gam_last) S + K^^T diag(exp(gam_last - gam)) Delta
    {
      const CT* bsrc = sDw + col * LDT + grp * EPF;
#pragma unroll
      for (int s = 0; s < SPW; ++s) {
        const int tile = wave + 4 * s;
        if (tile < NST) {
          S[s] = S[s] * el_c;
#pragma unroll
          for (int kb = 0; kb < NKB_T; ++kb) Mma<CT>::mma(S[s], kf[s][kb], load_frag<CT>(bsrc + kb * KB));
        }
      }
    }
    if (more) load_k(chunk + 1);
    store_state_lds();  // sSt was last read before barrier (B)
    lds_barrier();      // (A) state ready for the next chunk
  }
  if (p.final_state) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int tile = wave + 4 * s;
      if (tile < NST) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = tile * 16 + grp * 4 + i;
          if (row < dk && col_ok) p.final_state[((int64_t)h * dk + row) * dv + jc] = S[s][i];
        }
      }
    }
  }
}

template <class CT, class IT, int DK>
int launch_dk(const ScanParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((scan_prepare<CT, IT, DK>), dim3(p.nchunks, p.Hv), dim3(256), 0, stream, p);
  int rc = check_launch("scan_prepare");
  if (rc) return rc;
  const int ntiles = (p.dv + kVT - 1) / kVT;
  hipLaunchKernelGGL((scan_carry<CT, IT, DK>), dim3(p.Hv * ntiles), dim3(256), 0, stream, p);
  return check_launch("scan_carry");
}

template <class CT, class IT>
int launch_it(const ScanParams& p, hipStream_t stream) {
  if (p.dk <= 32) return launch_dk<CT, IT, 32>(p, stream);
  if (p.dk <= 64) return launch_dk<CT, IT, 64>(p, stream);
  return launch_dk<CT, IT, 128>(p, stream);
}

int dk_pad(int dk) { return dk <= 32 ? 32 : dk <= 64 ? 64 : 128; }

// Workspace: Tm, M [chunks][Hv][64][64] (compute dtype); eg, wl, beta, gam
// [chunks][Hv][64] f32; K^T [chunks][Hk][DK][64] (compute dtype); 1/|k| and
// qscale/|q| [chunks][Hk][64] f32.
size_t carve(ScanParams* p, char* b, int T, int Hk, int Hv, int dk, int precision) {
  const size_t nchunks = (size_t)(T + kC - 1) / kC;
  const size_t ct = precision == 0 ? 4 : 2;
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = b ? b + off : nullptr;
    off += al(bytes);
    return q;
  };
  char* Tm = take(nchunks * Hv * kC * kC * ct);
  char* Mm = take(nchunks * Hv * kC * kC * ct);
  char* eg = take(nchunks * Hv * kC * 4);
  char* wl = take(nchunks * Hv * kC * 4);
  char* bt = take(nchunks * Hv * kC * 4);
  char* gm = take(nchunks * Hv * kC * 4);
  char* Kt = take(nchunks * Hk * dk_pad(dk) * kC * ct);
  char* ik = take(nchunks * Hk * kC * 4);
  char* sq = take(nchunks * Hk * kC * 4);
  if (p) {
    p->Tm = Tm;
    p->Mm = Mm;
    p->Kt = Kt;
    p->eg = reinterpret_cast<float*>(eg);
    p->wl = reinterpret_cast<float*>(wl);
    p->bt = reinterpret_cast<float*>(bt);
    p->gam_ws = reinterpret_cast<float*>(gm);
    p->invk = reinterpret_cast<float*>(ik);
    p->scq = reinterpret_cast<float*>(sq);
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
  return p.dtype_qkv == 0 ? launch_it<half_t, float>(p, stream) : launch_it<half_t, half_t>(p, stream);
}

}  // namespace clef
