// Chunked gated-DeltaNet scan for gfx950.
//
// Semantics: delta_recurrence_prefill (crates/core/src/models/qwen.rs:826-882)
// with repeat-interleave GQA (qwen.rs:727-738); chunkwise algebra as in
// crates/core/src/models/chunk.metal:10-164, restated for C = 64.
//
// For one v-head and a chunk of C tokens with in-chunk cumulative log-decay
// gam_r = sum_{j<=r} g_j (padding rows have g = 0, beta = 0, k = q = v = 0):
//   A[r][c] = beta_r (k_r.k_c) exp(gam_r - gam_c)  (c < r);  Tm = (I + A)^-1
//   M[r][c] = (q_r.k_c) exp(gam_r - gam_c)          (c <= r)
//   Y       = diag(beta) (V - diag(exp gam) K S)
//   Delta   = Tm Y
//   O       = diag(exp gam) Q S + M Delta
//   S'      = exp(gam_last) S + K^T diag(exp(gam_last - gam)) Delta
// Decay ratios are only formed for c <= r, so g = -1000 underflows to exact
// zeros instead of dividing by an underflowed prefix product.
//
// Kernel 1 (scan_prepare, grid chunks x Hk) is fully parallel: it normalises
// q,k, forms K K^T and Q K^T on MFMA once per k-head, then for each of the
// Hv/Hk v-heads sharing it builds A, M and Tm (forward substitution, one wave
// per v-head, lane = column).  It writes Tm, M (compute dtype), gam, and the
// row scales 1/|k| and qscale/|q| to the workspace.
//
// Kernel 2 (scan_carry, grid Hv x ceil(dv/16)) runs the chunks in order for
// one v-head and 16 value columns (the columns of S evolve independently).
// The f32 state (dk x 16) lives in MFMA accumulators spread over 4 waves; each
// chunk does [K;Q] S, Tm Y, M Delta and K^T Delta on MFMA with operands staged
// in LDS, and prefetches the next chunk's operands into registers while the
// current chunk computes.  Work-groups sharing a k-head are placed on one XCD
// so its q/k chunk is read from that XCD's L2.
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

// Branch-free row loader: fetches the VI elements e0..e0+VI-1 of a row
// (clamped into the row so every address is valid) in the input dtype.
// Conversion and masking happen at use, so the loads stay in flight.
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

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------------------
// Kernel 1: per (chunk, k-head) preparation.
// ---------------------------------------------------------------------------
template <class CT, class IT, int DK>
__global__ __launch_bounds__(256) void scan_prepare(ScanParams p) {
  constexpr int VI = Vec16<IT>::n;       // input elements per 16-byte vector
  constexpr int TPR = DK / VI;           // threads per row
  constexpr int RPP = 256 / TPR;         // rows per pass
  constexpr int EPF = 16 / sizeof(CT);   // compute elements per fragment lane
  constexpr int KB = Mma<CT>::kBlock;
  constexpr int LDR = DK + EPF;          // padded LDS row (elements)
  static_assert(TPR <= 64 && (TPR & (TPR - 1)) == 0, "row group must fit a wave");

  __shared__ __attribute__((aligned(16))) CT sK[kC * LDR];
  __shared__ __attribute__((aligned(16))) CT sQ[kC * LDR];
  __shared__ float sG[2][kC * (kC + 1)];
  __shared__ __attribute__((aligned(16))) float sAT[2][kC * kC];
  __shared__ float sGam[2][kC];
  __shared__ float sBeta[2][kC];

  const int chunk = blockIdx.x, hk = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int t0 = chunk * kC;
  const int n = min(kC, p.T - t0);
  const int dk = p.dk;
  const float qscale = p.qscale;

  // 1. normalise q and k rows into LDS; record the row scales.  All loads
  //    are issued first (clamped, unconditional), then consumed.
  constexpr int NPASS = (2 * kC) / RPP;
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
    const float inv = 1.0f / sqrtf(s + 1e-6f);  // l2 with eps inside sqrt, qwen.rs:837-840
    const float scale = isq ? inv * qscale : inv;
    CT* dst = (isq ? sQ : sK) + r * LDR + e0;
#pragma unroll
    for (int i = 0; i < VI; ++i) dst[i] = static_cast<CT>(x[i] * scale);
    if (tid % TPR == 0) (isq ? p.scq : p.invk)[((int64_t)chunk * p.Hk + hk) * kC + r] = scale;
  }
  lds_barrier();

  // 2. Gram matrices on MFMA: G0 = K K^T, G1 = Q K^T (64 x 64 each).
  {
    const int col = lane & 15, grp = lane >> 4;
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const int ti = wave * 8 + tt;
      const int mat = ti >> 4, tr = (ti >> 2) & 3, tc = ti & 3;
      if (mat == 0 && tc > tr) continue;  // K K^T: only the lower triangle is used
      const CT* a_src = (mat ? sQ : sK) + (tr * 16 + col) * LDR + grp * EPF;
      const CT* b_src = sK + (tc * 16 + col) * LDR + grp * EPF;
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < DK / KB; ++kb)
        Mma<CT>::mma(acc, load_frag<CT>(a_src + kb * KB), load_frag<CT>(b_src + kb * KB));
#pragma unroll
      for (int i = 0; i < 4; ++i) sG[mat][(tr * 16 + grp * 4 + i) * (kC + 1) + tc * 16 + col] = acc[i];
    }
  }
  lds_barrier();

  // 3. per v-head: decay, A (transposed, f32), M, Tm.
  const int rep = p.Hv / p.Hk;
  for (int i0 = 0; i0 < rep; i0 += 2) {
    const int nh = min(2, rep - i0);
    if (wave < nh) {
      const int h = hk * rep + i0 + wave;
      const int64_t gi = (int64_t)(t0 + min(lane, n - 1)) * p.sgb + h;
      const uint32_t gb = load_bits(p.g, gi, p.dtype_gb), bb = load_bits(p.beta, gi, p.dtype_gb);
      const float gv = lane < n ? bits_to_f32(gb, p.dtype_gb) : 0.0f;
      const float bv = lane < n ? bits_to_f32(bb, p.dtype_gb) : 0.0f;
      // inclusive prefix sum over the wave (lane = token in chunk)
      float cs = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(cs, off, 64);
        if (lane >= off) cs += o;
      }
      sGam[wave][lane] = cs;
      sBeta[wave][lane] = bv;
      p.gam[((int64_t)chunk * p.Hv + h) * kC + lane] = cs;
    }
    lds_barrier();
    for (int hi = 0; hi < nh; ++hi) {
      const int h = hk * rep + i0 + hi;
      CT* Mout = static_cast<CT*>(p.Mm) + ((int64_t)chunk * p.Hv + h) * kC * kC;
      {  // A^T[c][r], lanes along r (conflict-free LDS writes)
        const int r = lane;
        const float gr = sGam[hi][r], br = sBeta[hi][r];
        for (int c = wave; c < kC; c += 4) {
          const float a = (c < r) ? (br * sG[0][r * (kC + 1) + c]) * expf(gr - sGam[hi][c]) : 0.0f;
          sAT[hi][c * kC + r] = a;
        }
      }
      {  // M[r][c], lanes along c (coalesced global writes)
        const int c = lane;
        const float gc = sGam[hi][c];
        for (int r = wave; r < kC; r += 4) {
          const float m = (c <= r) ? sG[1][r * (kC + 1) + c] * expf(sGam[hi][r] - gc) : 0.0f;
          Mout[r * kC + c] = static_cast<CT>(m);
        }
      }
    }
    lds_barrier();
    if (wave < nh) {
      // Forward substitution for Tm = (I + A)^-1; lane j owns column j.
      const int h = hk * rep + i0 + wave;
      const float* At = sAT[wave];
      float t[kC];
#pragma unroll
      for (int r = 0; r < kC; ++r) t[r] = (r == lane) ? 1.0f : 0.0f;
#pragma unroll
      for (int c = 0; c < kC - 1; ++c) {
        const float tc = t[c];
#pragma unroll
        for (int r4 = ((c + 1) / 4) * 4; r4 < kC; r4 += 4) {
          const float4_t a = *reinterpret_cast<const float4_t*>(At + c * kC + r4);
#pragma unroll
          for (int s = 0; s < 4; ++s)
            if (r4 + s > c) t[r4 + s] = fmaf(-a[s], tc, t[r4 + s]);
        }
      }
      CT* Tout = static_cast<CT*>(p.Tm) + ((int64_t)chunk * p.Hv + h) * kC * kC;
#pragma unroll
      for (int r = 0; r < kC; ++r) Tout[r * kC + lane] = static_cast<CT>(t[r]);
    }
    lds_barrier();
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential chunk carry for one (v-head, 16 value columns).
//
// Per chunk c (LDS buffer b = c & 1 for the normalised K/Q rows):
//   stage(c) -> barrier A -> prefetch(c+1) into registers ->
//   X = [K;Q] S, Y (waves 0,1) | O = exp(gam) Q S (waves 2,3) -> barrier B ->
//   Delta = Tm Y -> barrier C -> O += M Delta, store | S update.
// The K^T operand of the state update is gathered from the row-major K rows
// (strided 2-byte LDS reads) with the per-token decay folded in, so no
// transposed copy is staged.  Double-buffered K/Q rows remove the barrier
// that would otherwise guard the next chunk's staging.
// ---------------------------------------------------------------------------
template <class CT, class IT, int DK>
__global__ __launch_bounds__(256) void scan_carry(ScanParams p) {
  constexpr int VI = Vec16<IT>::n;
  constexpr int TPR = DK / VI;
  constexpr int RPP = 256 / TPR;
  constexpr int NPASS = (2 * kC) / RPP;  // staging passes (K rows then Q rows)
  constexpr int EPF = 16 / sizeof(CT);
  constexpr int KB = Mma<CT>::kBlock;
  constexpr int LDK = DK + EPF;   // [token][dk] rows
  constexpr int LDT = kC + EPF;   // [value][token] rows
  constexpr int NST = DK / 16;    // state row tiles
  constexpr int SPW = (NST + 3) / 4;  // state tiles per wave
  constexpr int NKB_T = kC / KB;  // k-blocks over tokens
  typedef typename Mma<CT>::frag frag;
  typedef typename Vec16<IT>::type vecI;

  __shared__ __attribute__((aligned(16))) CT sKQ[2][2 * kC * LDK];  // rows 0..63 K, 64..127 Q
  __shared__ __attribute__((aligned(16))) CT sSt[kVT * LDK];
  __shared__ __attribute__((aligned(16))) CT sYt[kVT * LDT];
  __shared__ __attribute__((aligned(16))) CT sDt[kVT * LDT];
  __shared__ float sEg[2][kC];    // exp(gam_r)
  __shared__ float sWl[2][kC];    // exp(gam_last - gam_r)
  __shared__ float sGam[2][kC];
  __shared__ float sBeta[2][kC];

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
  store_state_lds();

  // ---- prefetch registers (raw input dtype; converted at use)
  const IT* qbase = static_cast<const IT*>(p.q);
  const IT* kbase = static_cast<const IT*>(p.k);
  const IT* vbase = static_cast<const IT*>(p.v);
  vecI raw[NPASS];
  float rsc[NPASS];
  frag tfr[NKB_T];      // Tm rows of tile `wave`
  frag mfr[2][NKB_T];   // M rows (waves 2,3)
  IT vraw[2][4];        // V values (waves 0,1)
  float pg = 0.0f;      // gam of token `lane` (wave 0)
  uint32_t pb = 0;      // beta bits of token `lane` (wave 1)

  auto prefetch = [&](int chunk) {
    const int t0 = chunk * kC;
    const int n = min(kC, p.T - t0);
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int rr = ps * RPP + tid / TPR;
      const bool isq = rr >= kC;
      const int r = min(isq ? rr - kC : rr, n - 1);
      const IT* row = (isq ? qbase : kbase) + (int64_t)(t0 + r) * p.sqk + (int64_t)hk * dk;
      raw[ps] = load_row_raw<IT>(row, (tid % TPR) * VI, dk, p.vec_qk);
      rsc[ps] = (isq ? p.scq : p.invk)[((int64_t)chunk * p.Hk + hk) * kC + r];
    }
    const CT* Tm = static_cast<const CT*>(p.Tm) + ((int64_t)chunk * p.Hv + h) * kC * kC;
#pragma unroll
    for (int kb = 0; kb < NKB_T; ++kb)
      tfr[kb] = load_frag<CT>(Tm + (wave * 16 + col) * kC + kb * KB + grp * EPF);
    if (wave >= 2) {
      const CT* Mm = static_cast<const CT*>(p.Mm) + ((int64_t)chunk * p.Hv + h) * kC * kC;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int kb = 0; kb < NKB_T; ++kb)
          mfr[s][kb] = load_frag<CT>(Mm + ((wave - 2) * 32 + s * 16 + col) * kC + kb * KB + grp * EPF);
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = min(wave * 32 + s * 16 + grp * 4 + i, n - 1);
          vraw[s][i] = vbase[(int64_t)(t0 + r) * p.sv + (int64_t)h * dv + jcc];
        }
    }
    if (wave == 0) pg = p.gam[((int64_t)chunk * p.Hv + h) * kC + lane];
    if (wave == 1) pb = load_bits(p.beta, (int64_t)(t0 + min(lane, n - 1)) * p.sgb + h, p.dtype_gb);
  };

  const int nchunks = p.nchunks;
  const int cap_chunk = p.capture > 0 ? (p.capture - 1) / kC : -1;
  const int cap_row = p.capture > 0 ? (p.capture - 1) % kC : -1;
  prefetch(0);
  for (int chunk = 0; chunk < nchunks; ++chunk) {
    const int t0 = chunk * kC;
    const int n = min(kC, p.T - t0);
    const int b = chunk & 1;
    CT* sK = sKQ[b];
    // ---- stage: normalised K and Q rows into LDS buffer b
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int rr = ps * RPP + tid / TPR;
      const int r = rr >= kC ? rr - kC : rr;
      const int e0 = (tid % TPR) * VI;
      CT* dst = sKQ[b] + rr * LDK + e0;
#pragma unroll
      for (int i = 0; i < VI; ++i)
        dst[i] = static_cast<CT>((r < n && e0 + i < dk) ? static_cast<float>(raw[ps][i]) * rsc[ps] : 0.0f);
    }
    if (wave == 0) {
      const float gl = __shfl(pg, kC - 1, 64);
      sGam[b][lane] = pg;
      sEg[b][lane] = expf(pg);
      sWl[b][lane] = expf(gl - pg);
    }
    if (wave == 1) sBeta[b][lane] = lane < n ? bits_to_f32(pb, p.dtype_gb) : 0.0f;
    frag tcur[NKB_T];
    frag mcur[2][NKB_T];
    float vcur[2][4];
#pragma unroll
    for (int kb = 0; kb < NKB_T; ++kb) tcur[kb] = tfr[kb];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb) mcur[s][kb] = mfr[s][kb];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wave * 32 + s * 16 + grp * 4 + i;
        vcur[s][i] = (r < n && col_ok) ? static_cast<float>(vraw[s][i]) : 0.0f;
      }
    }
    lds_barrier();  // (A) operands of this chunk are in LDS
    if (chunk + 1 < nchunks) prefetch(chunk + 1);

    // ---- X = [K; Q] S : wave w -> row tiles 2w, 2w+1 of the 128-row product
    float4_t X[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) X[s] = float4_t{0.f, 0.f, 0.f, 0.f};
    {
      const CT* asrc = sKQ[b] + (wave * 32 + col) * LDK + grp * EPF;
      const CT* bsrc = sSt + col * LDK + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < DK / KB; ++kb) {
        const frag bf = load_frag<CT>(bsrc + kb * KB);
#pragma unroll
        for (int s = 0; s < 2; ++s) Mma<CT>::mma(X[s], load_frag<CT>(asrc + s * 16 * LDK + kb * KB), bf);
      }
    }
    // ---- waves 0,1: Y = beta (V - exp(gam) K S) -> Y^T in LDS
    //      waves 2,3: O starts as exp(gam) Q S
    float4_t O[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int rbase = (wave & 1) * 32 + s * 16 + grp * 4;
      if (wave < 2) {
        CT y4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rbase + i;
          y4[i] = static_cast<CT>(sBeta[b][r] * (vcur[s][i] - sEg[b][r] * X[s][i]));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sYt[col * LDT + rbase + i] = y4[i];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) O[s][i] = sEg[b][rbase + i] * X[s][i];
      }
    }
    lds_barrier();  // (B) Y^T ready

    // ---- Delta = Tm Y : wave w -> row tile w
    {
      float4_t D = {0.f, 0.f, 0.f, 0.f};
      const CT* bsrc = sYt + col * LDT + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb) Mma<CT>::mma(D, tcur[kb], load_frag<CT>(bsrc + kb * KB));
#pragma unroll
      for (int i = 0; i < 4; ++i) sDt[col * LDT + wave * 16 + grp * 4 + i] = static_cast<CT>(D[i]);
    }
    lds_barrier();  // (C) Delta^T ready

    // ---- waves 2,3: O += M Delta, store
    if (wave >= 2) {
      const CT* bsrc = sDt + col * LDT + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < NKB_T; ++kb) {
        const frag bf = load_frag<CT>(bsrc + kb * KB);
#pragma unroll
        for (int s = 0; s < 2; ++s) Mma<CT>::mma(O[s], mcur[s][kb], bf);
      }
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
    // K^T fragment (dk rows of `tile`, tokens of k-block kb) scaled per token by w.
    auto kt_frag = [&](int tile, int kb, const float* w) {
      frag f;
      const int e = tile * 16 + col;
#pragma unroll
      for (int j = 0; j < EPF; ++j) {
        const int tok = kb * KB + grp * EPF + j;
        f[j] = static_cast<CT>(static_cast<float>(sK[tok * LDK + e]) * w[tok]);
      }
      return f;
    };
    // ---- optional capture of the state after token `capture`
    if (chunk == cap_chunk) {
      __shared__ float sWc[kC];
      if (wave == 0) sWc[lane] = lane <= cap_row ? expf(sGam[b][cap_row] - sGam[b][lane]) : 0.0f;
      lds_barrier();
      const float ec = sEg[b][cap_row];
#pragma unroll
      for (int s = 0; s < SPW; ++s) {
        const int tile = wave + 4 * s;
        if (tile < NST) {
          float4_t acc = S[s] * ec;
          const CT* bsrc = sDt + col * LDT + grp * EPF;
#pragma unroll
          for (int kb = 0; kb < NKB_T; ++kb) Mma<CT>::mma(acc, kt_frag(tile, kb, sWc), load_frag<CT>(bsrc + kb * KB));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = tile * 16 + grp * 4 + i;
            if (row < dk && col_ok) p.captured[((int64_t)h * dk + row) * dv + jc] = acc[i];
          }
        }
      }
    }
    // ---- S <- exp(gam_last) S + (diag(w) K)^T Delta
    {
      const float el = sEg[b][kC - 1];
      const CT* bsrc = sDt + col * LDT + grp * EPF;
#pragma unroll
      for (int s = 0; s < SPW; ++s) {
        const int tile = wave + 4 * s;
        if (tile < NST) {
          S[s] = S[s] * el;
#pragma unroll
          for (int kb = 0; kb < NKB_T; ++kb)
            Mma<CT>::mma(S[s], kt_frag(tile, kb, sWl[b]), load_frag<CT>(bsrc + kb * KB));
        }
      }
    }
    store_state_lds();  // sSt is only read before barrier (B)
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
  hipLaunchKernelGGL((scan_prepare<CT, IT, DK>), dim3(p.nchunks, p.Hk), dim3(256), 0, stream, p);
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

}  // namespace

size_t scan_workspace_bytes(int T, int Hk, int Hv, int precision) {
  const size_t nchunks = (size_t)(T + kC - 1) / kC;
  const size_t ct = precision == 0 ? 4 : 2;
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  return 2 * al(nchunks * Hv * kC * kC * ct) + al(nchunks * Hv * kC * 4) + 2 * al(nchunks * Hk * kC * 4);
}

void scan_carve_workspace(ScanParams& p, void* ws, int precision) {
  const size_t nchunks = p.nchunks;
  const size_t ct = precision == 0 ? 4 : 2;
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  char* b = static_cast<char*>(ws);
  p.Tm = b; b += al(nchunks * p.Hv * kC * kC * ct);
  p.Mm = b; b += al(nchunks * p.Hv * kC * kC * ct);
  p.gam = reinterpret_cast<float*>(b); b += al(nchunks * p.Hv * kC * 4);
  p.invk = reinterpret_cast<float*>(b); b += al(nchunks * p.Hk * kC * 4);
  p.scq = reinterpret_cast<float*>(b);
}

int scan_launch(const ScanParams& p, int precision, hipStream_t stream) {
  if (precision == 0)
    return p.dtype_qkv == 0 ? launch_it<float, float>(p, stream) : launch_it<float, half_t>(p, stream);
  return p.dtype_qkv == 0 ? launch_it<half_t, float>(p, stream) : launch_it<half_t, half_t>(p, stream);
}

}  // namespace clef
