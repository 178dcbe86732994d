// Gated causal GQA attention for the full-attention layer (qwen.rs:451-525),
// with the online softmax of ops.rs:62-148 and the sigmoid gate of
// qwen.rs:518-524.  Replaces the reference's Metal flash-attention op
// (metal.rs:415-633).  This file holds the entry point and the f32 kernel
// (also used for f16 shapes attention_f16.hip does not take).
//
// One work-group (4 waves) owns 64 query rows of one head; each wave owns 16
// rows.  Key tiles of 64 are staged in LDS as K [key][d] and V^T [d][key]
// (values arrive transposed from clef_values_transposed), so both S = Q K^T
// and O += P V read 16-byte fragments.  Q stays in registers for the whole
// sweep; P goes through a per-wave LDS tile to change from the accumulator
// layout to the operand layout.  Tiles past the causal limit of the group's
// last row are skipped; the groups with the most key tiles are launched first.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../../include/clef_hip.h"
#include "attention.hpp"
#include "common.hpp"

namespace clef {
namespace {

__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

template <class T, int D>
__global__ __launch_bounds__(256) void attn_kernel(AttnParams p) {
  constexpr int BQ = 64, BKEY = 64;
  constexpr int EPF = 16 / sizeof(T);
  constexpr int KB = Mma<T>::kBlock;
  constexpr int LDK = D + EPF;     // K rows [key][d]
  constexpr int LDV = BKEY + EPF;  // V^T rows [d][key]
  constexpr int LDP = BKEY + EPF;  // P rows [query][key]
  constexpr int NDT = D / 16;      // output tiles along d
  typedef typename Mma<T>::frag frag;
  typedef typename Mma<T>::frag vec;  // 16-byte vector of T

  __shared__ __attribute__((aligned(16))) T sK[BKEY * LDK];
  __shared__ __attribute__((aligned(16))) T sV[D * LDV];
  __shared__ __attribute__((aligned(16))) T sP[4][16 * LDP];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int qtiles = (p.qn + BQ - 1) / BQ;
  const int h = blockIdx.x % p.heads;
  const int qt = qtiles - 1 - static_cast<int>(blockIdx.x / p.heads);  // longest first
  const int kvh = h / (p.heads / p.kvh);
  const int q0 = qt * BQ;
  const int offset = p.kn - p.qn;
  const int d = p.d;

  // global rows are d wide (d % EPF == 0, d <= D); features beyond d read as zero
  const T* Q = static_cast<const T*>(p.q) + (int64_t)h * p.ldq * d;
  const T* K = static_cast<const T*>(p.k) + (int64_t)kvh * p.ldk * d;
  const T* V = static_cast<const T*>(p.vt) + (int64_t)kvh * d * p.ldv;

  // Q fragments of this wave's 16 rows (A operand, k = d)
  frag qf[D / KB];
  {
    const int r = min(q0 + wave * 16 + col, p.qn - 1);
#pragma unroll
    for (int kb = 0; kb < D / KB; ++kb) {
      const int c = kb * KB + grp * EPF;
      qf[kb] = c < d ? *reinterpret_cast<const frag*>(Q + (int64_t)r * d + c) : frag{};
    }
  }
  float4_t O[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) O[i] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
  }

  const int key_end = min(p.kn, offset + q0 + BQ);  // exclusive causal limit of this group
  // K [64][D] and V^T [D][64] of a key tile: loaded into registers during the
  // previous tile's products, written to LDS after them
  constexpr int KV_PER_ROW = D / EPF, V_PER_ROW = BKEY / EPF;
  constexpr int NKL = BKEY * KV_PER_ROW / 256, NVL = D * V_PER_ROW / 256;  // vectors per thread
  static_assert(BKEY * KV_PER_ROW % 256 == 0 && D * V_PER_ROW % 256 == 0, "whole passes");
  vec kreg[NKL], vreg[NVL];
  auto load_tile = [&](int j0) {
#pragma unroll
    for (int u = 0; u < NKL; ++u) {
      const int v = tid + 256 * u;
      const int r = v / KV_PER_ROW, c = (v % KV_PER_ROW) * EPF;
      const int key = min(j0 + r, p.kn - 1);
      kreg[u] = c < d ? *reinterpret_cast<const vec*>(K + (int64_t)key * d + c) : vec{};
    }
#pragma unroll
    for (int u = 0; u < NVL; ++u) {
      const int v = tid + 256 * u;
      const int r = v / V_PER_ROW, c = (v % V_PER_ROW) * EPF;
      const int key = min(j0 + c, p.ldv - EPF);
      vreg[u] = r < d ? *reinterpret_cast<const vec*>(V + (int64_t)r * p.ldv + key) : vec{};
    }
  };
  auto store_tile = [&](int j0) {
#pragma unroll
    for (int u = 0; u < NKL; ++u) {
      const int v = tid + 256 * u;
      const int r = v / KV_PER_ROW, c = (v % KV_PER_ROW) * EPF;
      *reinterpret_cast<vec*>(&sK[r * LDK + c]) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < NVL; ++u) {
      const int v = tid + 256 * u;
      const int r = v / V_PER_ROW, c = (v % V_PER_ROW) * EPF;
      const int key = min(j0 + c, p.ldv - EPF);
      vec vv = vreg[u];
#pragma unroll
      for (int e = 0; e < EPF; ++e)
        if (key + e >= p.kn) vv[e] = T(0);  // keys past kn may be uninitialised
      *reinterpret_cast<vec*>(&sV[r * LDV + c]) = vv;
    }
  };
  load_tile(0);
  store_tile(0);
  lds_barrier();
  for (int j0 = 0; j0 < key_end; j0 += BKEY) {
    const bool more = j0 + BKEY < key_end;  // uniform over the work-group
    if (more) load_tile(j0 + BKEY);

    // ---- S = Q K^T for 16 rows x 64 keys
    float4_t S[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      S[nt] = float4_t{0.f, 0.f, 0.f, 0.f};
      const T* bsrc = sK + (nt * 16 + col) * LDK + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < D / KB; ++kb) Mma<T>::mma(S[nt], qf[kb], load_frag<T>(bsrc + kb * KB));
    }
    // ---- scale, mask, online softmax (rows 4*grp + i of this wave)
    float mt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = q0 + wave * 16 + grp * 4 + i;
      float mx = -INFINITY;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int key = j0 + nt * 16 + col;
        float s = S[nt][i] * p.scale;
        if (key >= p.kn || key > offset + row) s = -INFINITY;
        S[nt][i] = s;
        mx = fmaxf(mx, s);
      }
      mt[i] = lane_max<16>(mx);
    }
    float rescale[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mn = fmaxf(m[i], mt[i]);
      rescale[i] = (m[i] == -INFINITY) ? 0.0f : expf(m[i] - mn);
      m[i] = mn;
      float rs = 0.0f;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const float pv = (S[nt][i] == -INFINITY) ? 0.0f : expf(S[nt][i] - mn);
        S[nt][i] = pv;
        rs += pv;
      }
      rs = lane_sum<16>(rs);  // the association of an xor butterfly
      l[i] = l[i] * rescale[i] + rs;
    }
#pragma unroll
    for (int nt = 0; nt < NDT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) O[nt][i] *= rescale[i];
    // ---- P to LDS (accumulator layout -> operand layout)
    T* P = sP[wave];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) P[(grp * 4 + i) * LDP + nt * 16 + col] = static_cast<T>(S[nt][i]);
    wave_lds_sync();
    // ---- O += P V
    frag pf[BKEY / KB];
#pragma unroll
    for (int kb = 0; kb < BKEY / KB; ++kb) pf[kb] = load_frag<T>(P + col * LDP + kb * KB + grp * EPF);
#pragma unroll
    for (int nt = 0; nt < NDT; ++nt) {
      const T* bsrc = sV + (nt * 16 + col) * LDV + grp * EPF;
#pragma unroll
      for (int kb = 0; kb < BKEY / KB; ++kb) Mma<T>::mma(O[nt], pf[kb], load_frag<T>(bsrc + kb * KB));
    }
    lds_barrier();  // every wave is done with this tile's sK / sV
    if (more) {
      store_tile(j0 + BKEY);
      lds_barrier();
    }
  }

  // ---- epilogue: y = round(round(O / l) * round(sigmoid(gate)))
  const bool half_out = sizeof(T) == 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = q0 + wave * 16 + grp * 4 + i;
    if (row >= p.qn) continue;
    const float inv = 1.0f / l[i];
#pragma unroll
    for (int nt = 0; nt < NDT; ++nt) {
      const int e = nt * 16 + col;
      if (e >= d) continue;
      float a = O[nt][i] * inv;
      const T graw = static_cast<const T*>(p.gate)[(int64_t)row * p.ldg + (int64_t)h * p.hsg + e];
      float sg = 1.0f / (1.0f + expf(-static_cast<float>(graw)));
      if (half_out) {
        a = static_cast<float>(static_cast<T>(a));
        sg = static_cast<float>(static_cast<T>(sg));
      }
      static_cast<T*>(p.y)[(int64_t)row * p.ldy + (int64_t)h * d + e] = static_cast<T>(a * sg);
    }
  }
}

template <class T, int D>
int launch(const AttnParams& p, hipStream_t s) {
  const int qtiles = (p.qn + 63) / 64;
  hipLaunchKernelGGL((attn_kernel<T, D>), dim3(qtiles * p.heads), dim3(256), 0, s, p);
  return check_launch("attention");
}

template <class T>
int launch_d(const AttnParams& p, hipStream_t s) {
  if (p.d <= 32) return launch<T, 32>(p, s);
  if (p.d <= 64) return launch<T, 64>(p, s);
  if (p.d <= 128) return launch<T, 128>(p, s);
  return launch<T, 256>(p, s);
}

}  // namespace
}  // namespace clef

extern "C" int clef_attention_gated(const void* q, int64_t ldq_tok, const void* k, int64_t ldk_tok,
                                    const void* vt, int64_t ldv_tok, int dtype, int heads, int kv_heads,
                                    int qn, int kn, int d, const void* gate, int64_t ldg, int64_t hsg,
                                    void* y, int64_t ldy, void* stream) {
  CLEF_REQUIRE(q && k && vt && gate && y, "attention: null pointer");
  CLEF_REQUIRE(dtype == CLEF_F32 || dtype == CLEF_F16, "attention: dtype");
  CLEF_REQUIRE(heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0, "attention: head counts");
  CLEF_REQUIRE(qn >= 1 && kn >= qn, "attention: causal attention needs 1 <= qn <= kn");
  CLEF_REQUIRE(d >= 1 && d <= 256, "attention: head width must be in 1..256");
  const int epf = dtype == CLEF_F16 ? 8 : 4;
  CLEF_REQUIRE(d % epf == 0, "attention: head width must be a multiple of 16 bytes");
  CLEF_REQUIRE(ldq_tok >= qn && ldk_tok >= kn && ldv_tok >= kn && ldv_tok % epf == 0 && ldv_tok >= 64,
               "attention: token strides (ldv_tok must be >= 64 and a multiple of 16 bytes)");
  CLEF_REQUIRE(hsg >= d && ldg >= (int64_t)(heads - 1) * hsg + d && ldy >= (int64_t)heads * d,
               "attention: gate or output strides");
  clef::AttnParams p{q, k, vt, gate, y, ldq_tok, ldk_tok, ldv_tok, ldg, hsg, ldy, heads, kv_heads, qn, kn, d,
                     static_cast<float>(1.0 / std::sqrt(static_cast<double>(d)))};
  if (dtype == CLEF_F16) {
    if (clef::attn_f16_ok(p)) return clef::attn_f16_launch(p, static_cast<hipStream_t>(stream));
    return clef::launch_d<clef::half_t>(p, static_cast<hipStream_t>(stream));
  }
  return clef::launch_d<float>(p, static_cast<hipStream_t>(stream));
}

extern "C" int clef_attention_gated_qnorm(const void* q_raw, int64_t ldq_row, int64_t hsq, const float* q_norm,
                                          float eps, const float* rot_tab, const void* k, int64_t ldk_tok,
                                          const void* vt, int64_t ldv_tok, int heads, int kv_heads, int qn, int kn,
                                          int d, const void* gate, int64_t ldg, int64_t hsg, void* y, int64_t ldy,
                                          void* stream) {
  CLEF_REQUIRE(q_raw && q_norm && rot_tab && k && vt && gate && y, "attention: null pointer");
  CLEF_REQUIRE(heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0, "attention: head counts");
  CLEF_REQUIRE(qn >= 1 && kn >= qn, "attention: causal attention needs 1 <= qn <= kn");
  CLEF_REQUIRE(d == 256, "attention with the query norm: d = 256");
  CLEF_REQUIRE(hsq >= d && ldq_row >= (int64_t)(heads - 1) * hsq + d, "attention: raw query strides");
  CLEF_REQUIRE(ldk_tok >= kn && ldv_tok >= kn && ldv_tok % 8 == 0 && ldv_tok >= 64,
               "attention: token strides (ldv_tok must be >= 64 and a multiple of 16 bytes)");
  CLEF_REQUIRE(hsg >= d && ldg >= (int64_t)(heads - 1) * hsg + d && ldy >= (int64_t)heads * d,
               "attention: gate or output strides");
  clef::AttnParams p{q_raw, k, vt, gate, y, qn, ldk_tok, ldv_tok, ldg, hsg, ldy, heads, kv_heads, qn, kn, d,
                     static_cast<float>(1.0 / std::sqrt(static_cast<double>(d)))};
  p.qraw = q_raw;
  p.ldqr = ldq_row;
  p.hsr = hsq;
  p.qw = q_norm;
  p.qrot = reinterpret_cast<const float2*>(rot_tab);
  p.qeps = eps;
  p.qinv = static_cast<float>(1.0 / static_cast<double>(d));
  CLEF_REQUIRE(clef::attn_qfuse_ok(p), "attention with the query norm: 16-byte aligned rows, weights and table");
  return clef::attn_f16_launch(p, static_cast<hipStream_t>(stream));
}

extern "C" size_t clef_attention_varlen_workspace(int T, int nseq) {
  if (T < 1 || nseq < 1 || nseq > 4096) return 0;
  return clef::attn_tables_bytes(T, nseq);
}

extern "C" int clef_attention_gated_varlen(const void* q, int64_t ldq_tok, const void* k, int64_t ldk_tok,
                                           const void* vt, int64_t ldv_tok, const int32_t* cu_seqlens, int nseq,
                                           int T, const void* prefix_k, int64_t ldpk_tok, const void* prefix_vt,
                                           int64_t ldpv_tok, int np, int dtype, int heads, int kv_heads, int d,
                                           const void* gate, int64_t ldg, int64_t hsg, void* y, int64_t ldy,
                                           void* workspace, size_t workspace_bytes, void* stream) {
  CLEF_REQUIRE(q && k && vt && gate && y && cu_seqlens && workspace, "attention: null pointer");
  CLEF_REQUIRE(dtype == CLEF_F16, "attention: ragged batches run in the mixed profile (f16)");
  CLEF_REQUIRE(heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0, "attention: head counts");
  CLEF_REQUIRE(T >= 1 && nseq >= 1 && nseq <= 4096, "attention: 1 <= T and 1 <= nseq <= 4096");
  CLEF_REQUIRE(d >= 8 && d <= 256 && d % 8 == 0, "attention: head width must be a multiple of 8 in 8..256");
  CLEF_REQUIRE(ldq_tok >= T && ldk_tok >= T && ldv_tok >= T && ldv_tok % 8 == 0 && ldv_tok >= 64,
               "attention: token strides (ldv_tok must be >= 64 and a multiple of 8)");
  CLEF_REQUIRE(np >= 0 && np % 8 == 0 && (np == 0 || (prefix_k && prefix_vt && ldpk_tok >= np && ldpv_tok >= np)),
               "attention: prefix keys (np % 8 == 0, buffers and strides)");
  CLEF_REQUIRE(hsg >= d && ldg >= (int64_t)(heads - 1) * hsg + d && ldy >= (int64_t)heads * d,
               "attention: gate or output strides");
  CLEF_REQUIRE(workspace_bytes >= clef::attn_tables_bytes(T, nseq) &&
                   (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
               "attention: workspace too small or not 256-byte aligned");
  clef::AttnParams p{q, k, vt, gate, y, ldq_tok, ldk_tok, ldv_tok, ldg, hsg, ldy, heads, kv_heads, T, 0, d,
                     static_cast<float>(1.0 / std::sqrt(static_cast<double>(d)))};
  CLEF_REQUIRE(clef::attn_f16_ok(p), "attention: strides beyond the 32-bit offsets of the f16 kernel");
  p.cu_q = cu_seqlens;
  p.nseq = nseq;
  p.pk = prefix_k;
  p.pvt = prefix_vt;
  p.ldpk = ldpk_tok;
  p.ldpv = ldpv_tok;
  p.np = np;
  clef::attn_carve_tables(p, workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (int rc = clef::attn_f16_tables(p, st)) return rc;
  return clef::attn_f16_launch(p, st);
}
