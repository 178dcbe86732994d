// f16 gated causal GQA attention core (qwen.rs:451-525 with the online
// softmax of ops.rs:62-148), the mixed-profile path of clef_attention_gated.
//
// A work-group of 4 waves owns 128 queries of one head; wave w owns queries
// q0 + 32 w + (0..31).  Keys advance in tiles of 64, staged in LDS by
// global->LDS DMA (K as [key][d], V^T as [d][key]) one tile ahead.
//
// The scores are computed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16_f16:
// the accumulator of a 32-key x 32-query tile leaves lane l one query
// (l % 32) and 16 keys, so each lane does its own query's softmax over its
// keys and combines with one partner lane (l ^ 32) for the row maximum and
// sum.  Key rows are stored in LDS in the order pi(r) = r with bits 2 and 3
// swapped; with that order the 16 probabilities a lane holds are exactly its
// B-operand fragments of O^T = V^T P^T for two 16-key blocks in natural key
// order, so P never leaves registers.  The output accumulator O^T likewise
// gives each lane one query, so the softmax rescale is a per-lane factor.
//
// Rescaling is lazy: the running reference maximum only moves (and O and the
// row sum are rescaled) when the new maximum exceeds it by more than 8 in
// log2 units; otherwise the probabilities exp2((s - m_ref) c) stay below
// 2^8.  Both O and the row sum use the same reference, so O / l is the
// softmax average exactly as in the eager formulation.
#include "attention.hpp"
#include "ragged.hpp"
#include "common.hpp"

namespace clef {
namespace {

// global_load_lds_dwordx4 as inline asm (see gemm_f16.hip): lane l writes 16
// bytes at M0 + 16 l; completion is awaited with an explicit vmcnt wait.
// dma16 takes a per-lane address, dma16s a wave-uniform base plus a per-lane
// 32-bit byte offset (no per-lane address arithmetic).
// The compiler does not see the load inside the asm, so the asm carries the
// wait states its operands need: 1 after the SALU write of M0 that precedes
// an LDS DMA, 5 between a VALU write of an SGPR (the readfirstlane of the
// base) and a vector-memory read of it.
__device__ __forceinline__ void dma16(const void* src_lane, void* lds_block) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_block));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src_lane), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, void* lds_block) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_block));
  // the base is wave-uniform; readfirstlane pins it to SGPRs as the encoding requires
  // (readfirstlane returns int: each half is widened as unsigned)
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(sb), "{m0}"(m0) : "memory");
}

__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

// combine lane l with lane l ^ 32
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// key order of the LDS key rows within a 64-key tile (an involution)
__device__ __forceinline__ int key_perm(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// XOR key of the 16-byte slots of key row r: rows of 256 bytes or more use
// 16 keys (one per 16-byte bank group of a 256-byte bank row), 128-byte rows
// pair up in a bank row and use 8 keys per row pair
template <int D>
__device__ __forceinline__ int kswz(int r) { return D >= 128 ? (r & 15) : ((r >> 1) & 7); }

template <int D>
__global__ __launch_bounds__(256) void attn_f16(AttnParams p) {
  constexpr int BQ = 128, BK = 64;
  constexpr int KS = D / 8;       // 16-byte chunks per key row
  constexpr int NKB = D / 16;     // k-blocks of S^T = K Q^T
  constexpr int NDT = D / 32;     // 32-row tiles of O^T
  constexpr int NDMA = D / 32;    // DMA instructions per wave, per operand and tile
  constexpr int KROWS = 512 / D;  // key rows per 1 KiB DMA instruction
  constexpr int PD = 8;           // LDS fragment reads in flight ahead of the MFMAs
  static_assert(D == 64 || D == 128 || D == 256, "head width tile");

  __shared__ __attribute__((aligned(1024))) half_t sK[2][BK * D];
  __shared__ __attribute__((aligned(1024))) half_t sV[2][D * BK];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;

  // Persistent work-groups (as many as fit on the chip): work items (query
  // tile, head) are numbered longest first and dealt to the work-groups in
  // boustrophedon order (b, 2B-1-b, 2B+b, ...), so every work-group gets a
  // near-equal share of key tiles whatever order the hardware places them in
  // (it does not hand a waiting work-group to the first CU that frees up).
  // Within a rank, consecutive items on one XCD get adjacent heads (with
  // heads % 8 == 0), which share key/value heads and so that XCD's L2.
  const int nitems = (p.cu_q ? *p.npairs : (p.qn + BQ - 1) / BQ) * p.heads;
  const int nwg = gridDim.x;
  for (int round = 0;; ++round) {
  const int item = round * nwg + ((round & 1) ? nwg - 1 - (int)blockIdx.x : (int)blockIdx.x);
  if (item >= nitems) break;
  const int rank = item / p.heads, hi = item % p.heads;
  const int h = (p.heads & 7) == 0 ? (hi & 7) * (p.heads >> 3) + (hi >> 3) : hi;
  // this block's sequence: queries qb0 + (0..qn-1); keys 0..na-1 from the
  // prefix buffers, na..kn-1 from rows kb0 + (0..kn-na-1) of k / vt
  int q0, qb0 = 0, qn = p.qn, kn = p.kn, na = 0;
  if (p.cu_q) {
    const int2 e = p.pairs[rank];
    const int a = min(max(p.cu_q[e.x], 0), p.qn), b = min(max(p.cu_q[e.x + 1], a), p.qn);
    qb0 = a;
    qn = b - a;
    na = p.np;
    kn = na + qn;
    q0 = e.y * BQ;
  } else {
    q0 = ((p.qn + BQ - 1) / BQ - 1 - rank) * BQ;
  }
  const int kb0 = qb0;
  const int kvh = h / (p.heads / p.kvh);
  const int offset = kn - qn;
  const int d = p.d;

  const half_t* Q = static_cast<const half_t*>(p.q) + (int64_t)h * p.ldq * d + (int64_t)qb0 * d;
  const half_t* Kb = static_cast<const half_t*>(p.k) + (int64_t)kvh * p.ldk * d + (int64_t)kb0 * d;
  const half_t* Vb = static_cast<const half_t*>(p.vt) + (int64_t)kvh * d * p.ldv + kb0;
  const half_t* Kp = p.pk ? static_cast<const half_t*>(p.pk) + (int64_t)kvh * p.ldpk * d : nullptr;
  const half_t* Vp = p.pvt ? static_cast<const half_t*>(p.pvt) + (int64_t)kvh * d * p.ldpv : nullptr;

  // Q^T fragments (B operand): lane (n, g) holds d = 16 kb + 8 g .. + 7 of its query
  half8 qf[NKB];
  {
    const int r = min(q0 + 32 * wave + n, qn - 1);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int c = 16 * kb + 8 * g;
      qf[kb] = c < d ? *reinterpret_cast<const half8*>(Q + (int64_t)r * d + c) : half8{};
    }
  }

  // ---- DMA sources.  Instruction t = wave * NDMA + q writes 1 KiB: for K,
  // rows t * KROWS + lane / KS, slot lane % KS holding chunk slot ^ kswz(row)
  // of key pi(row); for V^T, d-row 8 t + lane / 8, slot lane % 8 holding
  // keys 8 c .. 8 c + 7 with c = slot ^ ((row >> 1) & 7).  d past the head
  // width reads in-bounds data that multiplies zero queries (K) or lands in
  // unstored outputs (V).  Tiles inside [0, kn) use a uniform base and the
  // per-lane byte offsets ko / vo; the last tile clamps keys to kn - 1 (K,
  // masked) and ldv - 8 (V, zeroed below).  Ragged batches: tiles inside the
  // prefix or inside the sequence's own keys take the same fast path from
  // their segment's base (V prefix tiles excepted: another row stride); the
  // rest pick each row's segment (na % 8 == 0 keeps 8-key chunks whole).
  uint32_t ko[NDMA], vo[NDMA];
  int kr[NDMA];
#pragma unroll
  for (int q = 0; q < NDMA; ++q) {
    const int row = (wave * NDMA + q) * KROWS + lane / KS;
    kr[q] = key_perm(row);
    const int kc = 8 * min((lane % KS) ^ kswz<D>(row), d / 8 - 1);
    ko[q] = 2u * (uint32_t)(kr[q] * d + kc);
    const int vrow = (wave * NDMA + q) * 8 + (lane >> 3);
    const int vc = 8 * ((lane & 7) ^ ((vrow >> 1) & 7));
    vo[q] = 2u * (uint32_t)(min(vrow, d - 1) * (int)p.ldv + vc);
  }
  const int kn1 = kn - 1, ldv8 = (int)p.ldv - 8 - kb0;
  auto issue_k = [&](int buf, int j0) {
    if (j0 >= na && j0 + BK <= kn) {
      const half_t* kb = Kb + (int64_t)(j0 - na) * d;
#pragma unroll
      for (int q = 0; q < NDMA; ++q) dma16s(kb, ko[q], &sK[buf][(wave * NDMA + q) * 512]);
    } else if (j0 + BK <= na) {
      const half_t* kb = Kp + (int64_t)j0 * d;
#pragma unroll
      for (int q = 0; q < NDMA; ++q) dma16s(kb, ko[q], &sK[buf][(wave * NDMA + q) * 512]);
    } else {
#pragma unroll
      for (int q = 0; q < NDMA; ++q) {
        const int key = min(j0 + kr[q], kn1);
        const half_t* row = key < na ? Kp + (int64_t)key * d : Kb + (int64_t)(key - na) * d;
        const char* src = reinterpret_cast<const char*>(row) + (ko[q] - 2u * (uint32_t)(kr[q] * d));
        dma16(src, &sK[buf][(wave * NDMA + q) * 512]);
      }
    }
  };
  auto issue_v = [&](int buf, int j0) {
    if (j0 >= na && j0 + BK <= kn) {
      const half_t* vb = Vb + (j0 - na);
#pragma unroll
      for (int q = 0; q < NDMA; ++q) dma16s(vb, vo[q], &sV[buf][(wave * NDMA + q) * 512]);
    } else {
#pragma unroll
      for (int q = 0; q < NDMA; ++q) {
        const int vrow = min((wave * NDMA + q) * 8 + (lane >> 3), d - 1);
        const int c0 = j0 + 8 * ((lane & 7) ^ ((((wave * NDMA + q) * 8 + (lane >> 3)) >> 1) & 7));
        const half_t* src = c0 < na ? Vp + (int64_t)vrow * p.ldpv + c0
                                    : Vb + ((int64_t)vrow * p.ldv + min(c0 - na, ldv8));
        dma16(src, &sV[buf][(wave * NDMA + q) * 512]);
      }
    }
  };

  // ---- fragment read offsets (bytes).  K: row 32 kh + n, chunk 2 kb + g at
  // slot chunk ^ kswz(n) (kswz(32 kh + n) = kswz(n)); V^T: row 32 dt + n,
  // chunk 2 kb2 + g at slot chunk ^ ((n >> 1) & 7).  The rest of each address
  // is an immediate.
  constexpr int KPER = D >= 128 ? 8 : 4;  // k-blocks per swizzle period
  int koff[KPER], voff[4];
#pragma unroll
  for (int x = 0; x < KPER; ++x) koff[x] = n * 2 * D + 16 * ((2 * x + g) ^ kswz<D>(n));
#pragma unroll
  for (int x = 0; x < 4; ++x) voff[x] = n * 128 + 16 * ((2 * x + g) ^ ((n >> 1) & 7));
  auto kread = [&](const char* base, int i) {  // S step i: k-block i / 2, key half i % 2
    const int kb = i >> 1, kh = i & 1;
    return *reinterpret_cast<const half8*>(base + koff[kb % KPER] + kh * 64 * D + (kb / KPER) * 32 * KPER);
  };
  auto vread = [&](const char* base, int i) {  // PV step i: key block i / NDT, d tile i % NDT
    return *reinterpret_cast<const half8*>(base + voff[i / NDT] + (i % NDT) * 32 * 128);
  };

  // one pipeline step: MFMA step s of the tile (s < NS1: scores, else PV)
  constexpr int NS1 = 2 * NKB, NS2 = 4 * NDT;
  auto frag = [&](const char* kbase, const char* vbase, int st) {
    return st < NS1 ? kread(kbase, st) : vread(vbase, st - NS1);
  };

  float16_t O[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) O[t][e] = 0.0f;
  float l_run = 0.0f;

  const float c2 = p.scale * 1.4426950408889634f;  // scores to log2 units
  const int key_end = min(kn, offset + q0 + BQ);
  const int ntiles = (key_end + BK - 1) / BK;
  // this lane's query sees keys <= lim; accumulator (kh, e) of lane group g
  // is key j0 + 32 kh + 16 (e / 8) + 8 g + e % 8 of the tile at j0
  const int lim = min(offset + q0 + 32 * wave + n, kn1);
  auto key_in_tile = [](int x) { return 32 * (x >> 4) + 16 * ((x >> 3) & 1) + (x & 7); };  // x = 16 kh + e

  // ---- prologue: K(0), K(1), V(0) resident; scores of tile 0
  issue_k(0, 0);
  if (ntiles > 1) issue_k(1, BK);
  issue_v(0, 0);
  vm_wait_all();
  lds_barrier();
  float16_t Sc[2], Sn[2];
  half8 fb[PD];
  {
    const char* kbase = reinterpret_cast<const char*>(sK[0]);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 16; ++e) Sc[kh][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < PD; ++i) fb[i] = kread(kbase, i);
#pragma unroll
    for (int i = 0; i < NS1; ++i) {
      Sc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[i % PD], qf[i >> 1], Sc[i & 1], 0, 0, 0);
      if (i + PD < NS1) fb[i % PD] = kread(kbase, i + PD);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float m_ref;
  {
    const int thr = lim - 8 * g;
    float mx = -INFINITY;
#pragma unroll
    for (int x = 0; x < 32; ++x) {
      const float sv = key_in_tile(x) > thr ? -INFINITY : Sc[x >> 4][x & 15];
      Sc[x >> 4][x & 15] = sv;
      mx = fmaxf(mx, sv);
    }
    m_ref = halves_max(mx);  // finite: every query sees key 0
  }
  lds_barrier();  // all waves are done with K(0) before K(2) replaces it

  // ---- software pipeline over key tiles.  Iteration j, with K(j+1) and V(j)
  // resident and the masked scores of tile j in Sc:
  //   phase 1: MFMA  Sn = K(j+1) Q^T            VALU  P = exp2(Sc c - m c), row sum
  //   phase 2: MFMA  O^T += V(j)^T P^T          VALU  mask Sn, row max of tile j+1
  // then the reference maximum moves (rare) before tile j+1's exponentials.
  // The DMA of K(j+2) and V(j+1) runs under both phases.  In the last
  // iteration Sn is computed from a stale buffer and discarded.
  for (int j = 0; j < ntiles; ++j) {
    const int j0 = j * BK;
    if (j + 2 < ntiles) issue_k(j & 1, j0 + 2 * BK);
    if (j + 1 < ntiles) issue_v((j + 1) & 1, j0 + BK);
    if (j0 + BK > kn) {  // last tile runs past the keys: zero those value columns
      half_t* v = sV[j & 1];
      for (int x = tid; x < D * 8; x += 256) {
        const int r = x >> 3, slot = x & 7;
        const int k0 = j0 + 8 * (slot ^ ((r >> 1) & 7));
        if (k0 + 8 > kn) {
          half8 val = *reinterpret_cast<half8*>(v + r * 64 + slot * 8);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k0 + e >= kn) val[e] = half_t(0);
          *reinterpret_cast<half8*>(v + r * 64 + slot * 8) = val;
        }
      }
      lds_barrier();
    }
    const char* kbase = reinterpret_cast<const char*>(sK[(j + 1) & 1]);
    const char* vbase = reinterpret_cast<const char*>(sV[j & 1]);
    const float mc = m_ref * c2;
    const int thr = lim - (j0 + BK) - 8 * g;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 16; ++e) Sn[kh][e] = 0.0f;
    half8 pf[4];
    float ps = 0.0f, mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PD; ++i) fb[i] = frag(kbase, vbase, i);
    // phase 1: EPS1 probabilities per score MFMA
    constexpr int EPS1 = 32 / NS1, EPS2 = 32 / NS2;
#pragma unroll
    for (int st = 0; st < NS1; ++st) {
      Sn[st & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[st % PD], qf[st >> 1], Sn[st & 1], 0, 0, 0);
      fb[st % PD] = frag(kbase, vbase, st + PD);
#pragma unroll
      for (int u = 0; u < EPS1; ++u) {
        const int x = st * EPS1 + u;
        const float pv = __builtin_amdgcn_exp2f(fmaf(Sc[x >> 4][x & 15], c2, -mc));
        ps += pv;
        pf[x >> 3][x & 7] = static_cast<half_t>(pv);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // phase 2: EPS2 masked scores of tile j+1 per PV MFMA, two MFMAs behind
    // the end of the score chain (the last 2 EPS2 follow the loop)
    auto mask_max = [&](int x) {
      const float sv = key_in_tile(x) > thr ? -INFINITY : Sn[x >> 4][x & 15];
      Sc[x >> 4][x & 15] = sv;  // phase 1 is done with tile j's scores
      mx = fmaxf(mx, sv);
    };
#pragma unroll
    for (int i = 0; i < NS2; ++i) {
      O[i % NDT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[(NS1 + i) % PD], pf[i / NDT], O[i % NDT], 0, 0, 0);
      if (NS1 + i + PD < NS1 + NS2) fb[(NS1 + i) % PD] = frag(kbase, vbase, NS1 + i + PD);
      if (i >= 2) {
#pragma unroll
        for (int u = 0; u < EPS2; ++u) mask_max((i - 2) * EPS2 + u);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int x = 32 - 2 * EPS2; x < 32; ++x) mask_max(x);
    l_run += ps;
    if (j + 1 < ntiles) {
      // lazy rescale: move the reference only when exp2 would exceed 2^8
      const float m_new = fmaxf(m_ref, halves_max(mx));
      if (__builtin_amdgcn_ballot_w64((m_new - m_ref) * c2 > 8.0f)) {
        const float alpha = __builtin_amdgcn_exp2f((m_ref - m_new) * c2);
#pragma unroll
        for (int t = 0; t < NDT; ++t)
#pragma unroll
          for (int e = 0; e < 16; ++e) O[t][e] *= alpha;
        l_run *= alpha;
        m_ref = m_new;
      }
    }
    vm_wait_all();
    lds_barrier();
  }

  // ---- epilogue: y = round(round(O / l) * round(sigmoid(gate))), the
  // sigmoid on the hardware exp2 and reciprocal (the epilogue's vector ALU
  // work is not hidden: one wave per SIMD).  O^T
  // accumulator e of tile t holds d = 32 t + 8 (e / 4) + 4 g + e % 4: four
  // consecutive features per (t, e / 4).  With 8-byte aligned gate and y
  // rows every gate read is issued before the first store (the loads would
  // otherwise wait one memory latency each).
  const float inv = 1.0f / halves_sum(l_run);
  const int row = q0 + 32 * wave + n;
  const int64_t prow = qb0 + min(row, qn - 1);  // packed row (clamped for the loads)
  const half_t* gate = static_cast<const half_t*>(p.gate) + prow * p.ldg + (int64_t)h * p.hsg;
  half_t* y = static_cast<half_t*>(p.y) + prow * p.ldy + (int64_t)h * d;
  auto out4 = [&](int t, int blk, half4 gv) {
    half4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = static_cast<float>(to_f16(O[t][4 * blk + e] * inv));
      const float sg = static_cast<float>(to_f16(sigmoid_hw(static_cast<float>(gv[e]))));
      r[e] = static_cast<half_t>(a * sg);
    }
    return r;
  };
  if (p.vec_io) {
    half4 gv[NDT][4];
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int d0 = 32 * t + 8 * blk + 4 * g;
        gv[t][blk] = d0 < d ? *reinterpret_cast<const half4*>(gate + d0) : half4{};
      }
    if (row < qn) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
          const int d0 = 32 * t + 8 * blk + 4 * g;
          if (d0 < d) *reinterpret_cast<half4*>(y + d0) = out4(t, blk, gv[t][blk]);
        }
    }
  } else if (row < qn) {
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int d0 = 32 * t + 8 * blk + 4 * g;
        if (d0 < d) {
          half4 gv;
#pragma unroll
          for (int e = 0; e < 4; ++e) gv[e] = gate[d0 + e];
          const half4 r = out4(t, blk, gv);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[d0 + e] = r[e];
        }
      }
  }
  }  // work items (the last key tile ended with a barrier: LDS is free)
}

// ---------------------------------------------------------------------------
// Single-sequence core at two waves per SIMD: a work-group of 8 waves owns
// 128 queries of one head, wave w queries q0 + 16 w + (0..15), on
// v_mfma_f32_16x16x32_f16 (A and B fragments: 8 consecutive k of row or
// column lane % 16; accumulators: rows 4 (lane / 16) + i of column lane % 16).
// S^T = K Q^T gives lane l its query l % 16 and, per 16-key tile t, 4 keys;
// the query's 64 keys of a tile sit in the four lane groups l / 16, which
// combine for the row maximum (the row sum is combined once, at the end).
// Within each 32-key block the LDS key row [u g j] (u: bit 4, g: bits 2-3,
// j: bits 0-1) holds key [g u j], so that the accumulators a lane holds of
// tiles 2b, 2b+1 are its B-operand fragment (8 consecutive keys) of
// O^T = V^T P^T for key block b.  About 200 registers: two waves per SIMD.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int key_perm16(int r) {
  return (r & ~31) | (((r >> 2) & 3) << 3) | (((r >> 4) & 1) << 2) | (r & 3);
}

// Fused query preparation for one query row t of head h, lane group g
// holding features 32 s + 8 g .. + 7 (the Qᵀ fragments): the RMS norm and
// rotary of the per-token q/k kernel (qwen.rs:451-470; pointwise.hip) with
// its roundings and its association of the squares.  That kernel sums runs
// of four consecutive features per lane, then an xor butterfly over the 64
// runs with offsets 32, 16, 8, 4, 2, 1; here run L = 8 s + 2 g + u (u: the
// fragment half), so offsets 32, 16, 8 pair runs inside a lane, 4 and 2 the
// lane groups g ^ 2 and g ^ 1 (lanes 32 and 16 apart), and 1 the halves.
// Rotary on features 0..63: feature i < 32 of fragment 0 pairs with i + 32
// of fragment 1 in the same lane, by the (cos, sin) row of position t.
__device__ __forceinline__ void q_prepare(const AttnParams& p, int t, int h, int g, half8* qf) {
  constexpr int NKS = 8;
  const half_t* src = static_cast<const half_t*>(p.qraw) + (int64_t)t * p.ldqr + (int64_t)h * p.hsr;
  const float4_t* wp = reinterpret_cast<const float4_t*>(p.qw + 8 * g);
  const float4_t* rt = reinterpret_cast<const float4_t*>(p.qrot + (int64_t)t * 32 + 8 * g);
  // every load first (one memory latency): the row, its 64 weights, its 8 (cos, sin) pairs
  float4_t wv[2 * NKS], cs[4];
#pragma unroll
  for (int s = 0; s < NKS; ++s) qf[s] = *reinterpret_cast<const half8*>(src + 32 * s + 8 * g);
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    wv[2 * s] = wp[8 * s];
    wv[2 * s + 1] = wp[8 * s + 1];
  }
#pragma unroll
  for (int e2 = 0; e2 < 4; ++e2) cs[e2] = rt[e2];  // features 8 g + 2 e2 and + 1
  float tot[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float run[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = static_cast<float>(qf[s][4 * u + e]);
        ss += v * v;
      }
      run[s] = ss;
    }
    const float b0 = run[0] + run[4], b1 = run[1] + run[5], b2 = run[2] + run[6], b3 = run[3] + run[7];
    float x = (b0 + b2) + (b1 + b3);
    x += __shfl_xor(x, 32, 64);
    x += __shfl_xor(x, 16, 64);
    tot[u] = x;
  }
  const float inverse = 1.0f / sqrtf(add_rn(mul_rn(tot[0] + tot[1], p.qinv), p.qeps));
#pragma unroll
  for (int s = 0; s < NKS; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      qf[s][e] = to_f16(mul_rn(mul_rn(static_cast<float>(qf[s][e]), inverse), wv[2 * s + e / 4][e % 4]));
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = cs[e / 2][2 * (e % 2)], sn = cs[e / 2][2 * (e % 2) + 1];
    const float a = static_cast<float>(qf[0][e]), b = static_cast<float>(qf[1][e]);
    qf[0][e] = to_f16(add_rn(mul_rn(a, c), mul_rn(b, -sn)));
    qf[1][e] = to_f16(add_rn(mul_rn(b, c), mul_rn(a, sn)));
  }
}

template <int D, bool VL>
__global__ __launch_bounds__(512) void attn_f16_w8(AttnParams p) {
  constexpr int BQ = 128, BK = 64, NW = 8;
  constexpr int KS = D / 8;           // 16-byte chunks per key row
  constexpr int NKS = D / 32;         // 32-deep k-steps of S^T = K Q^T
  constexpr int NDT = D / 16;         // 16-row tiles of O^T
  constexpr int KROWS = 512 / D;      // key rows per 1 KiB DMA instruction
  constexpr int NDK = BK / KROWS / NW;  // K DMA instructions per wave and tile
  constexpr int NDV = D / 8 / NW;       // V^T DMA instructions (8 rows of 64 keys each)
  constexpr int PD = 4;               // LDS fragment reads in flight ahead of the MFMAs
  static_assert(D == 256 || D == 128, "head width");
  static_assert(NDK >= 1 && NDV >= 1, "whole DMA instructions per wave");

  __shared__ __attribute__((aligned(1024))) half_t sK[2][BK * D];
  __shared__ __attribute__((aligned(1024))) half_t sV[2][D * BK];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;

  // work items dealt as in attn_f16 (longest first, boustrophedon); a ragged
  // batch's items are its (sequence, query tile) pairs, ranked by key count
  const int nitems = (VL ? *p.npairs : (p.qn + BQ - 1) / BQ) * p.heads;
  const int nwg = gridDim.x;
  for (int round = 0;; ++round) {
  const int item = round * nwg + ((round & 1) ? nwg - 1 - (int)blockIdx.x : (int)blockIdx.x);
  if (item >= nitems) break;
  const int rank = item / p.heads, hi = item % p.heads;
  const int h = (p.heads & 7) == 0 ? (hi & 7) * (p.heads >> 3) + (hi >> 3) : hi;
  // this item's sequence: queries qb0 + (0..qn-1); keys 0..na-1 from the
  // prefix buffers, na..kn-1 from rows qb0 + (0..kn-na-1) of k / vt
  int q0, qb0 = 0, qn = p.qn, kn = p.kn, na = 0;
  if constexpr (VL) {
    const int2 e = p.pairs[rank];
    const int a = min(max(p.cu_q[e.x], 0), p.qn), b = min(max(p.cu_q[e.x + 1], a), p.qn);
    qb0 = a;
    qn = b - a;
    na = p.np;
    kn = na + qn;
    q0 = e.y * BQ;
  } else {
    q0 = ((qn + BQ - 1) / BQ - 1 - rank) * BQ;
  }
  const int kvh = h / (p.heads / p.kvh);
  const int offset = kn - qn;
  const int d = p.d;

  const half_t* Q = static_cast<const half_t*>(p.q) + (int64_t)h * p.ldq * d + (int64_t)qb0 * d;
  const half_t* Kb = static_cast<const half_t*>(p.k) + (int64_t)kvh * p.ldk * d + (int64_t)qb0 * d;
  const half_t* Vb = static_cast<const half_t*>(p.vt) + (int64_t)kvh * d * p.ldv + qb0;
  const half_t* Kp = VL && p.pk ? static_cast<const half_t*>(p.pk) + (int64_t)kvh * p.ldpk * d : nullptr;
  const half_t* Vp = VL && p.pvt ? static_cast<const half_t*>(p.pvt) + (int64_t)kvh * d * p.ldpv : nullptr;

  // Q^T fragments (B operand): lane (n, g) holds d = 32 s + 8 g .. + 7 of its query
  half8 qf[NKS];
  {
    const int r = min(q0 + 16 * wave + n, qn - 1);
    bool prepared = false;
    if constexpr (!VL) {
      if (p.qraw) {  // raw projection rows: norm and rotary here (attn_qfuse_ok: d = 256)
        q_prepare(p, r, h, g, qf);
        prepared = true;
      }
    }
    if (!prepared) {
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        const int c = 32 * s + 8 * g;
        qf[s] = c < d ? *reinterpret_cast<const half8*>(Q + (int64_t)r * d + c) : half8{};
      }
    }
  }

  // ---- DMA sources.  K instruction t = wave * NDK + q writes 1 KiB: rows
  // t * KROWS + lane / KS, slot lane % KS holding chunk slot ^ (row & 15) of
  // key key_perm16(row).  V^T instruction t: d-row 8 t + lane / 8, slot
  // lane % 8 holding keys 8 c .. 8 c + 7 with c = slot ^ ((row >> 1) & 7).
  // d past the head width reads in-bounds data that multiplies zero queries
  // (K) or lands in unstored outputs (V); the last tile clamps keys to kn - 1
  // (K, masked) and the row end (V, zeroed below).  Ragged batches: tiles
  // inside the prefix (K) or inside the sequence's own keys take the fast
  // path from their segment's base; the rest pick each row's segment
  // (na % 8 == 0 keeps 8-key chunks whole).
  uint32_t ko[NDK], vo[NDV];
  int kr[NDK];
#pragma unroll
  for (int q = 0; q < NDK; ++q) {
    const int row = (wave * NDK + q) * KROWS + lane / KS;
    kr[q] = key_perm16(row);
    const int kc = 8 * min((lane % KS) ^ (row & 15), d / 8 - 1);
    ko[q] = 2u * (uint32_t)(kr[q] * d + kc);
  }
#pragma unroll
  for (int q = 0; q < NDV; ++q) {
    const int vrow = (wave * NDV + q) * 8 + (lane >> 3);
    const int vc = 8 * ((lane & 7) ^ ((vrow >> 1) & 7));
    vo[q] = 2u * (uint32_t)(min(vrow, d - 1) * (int)p.ldv + vc);
  }
  const int kn1 = kn - 1, ldv8 = (int)p.ldv - 8 - qb0;
  auto issue_k = [&](int buf, int j0) {
    if (j0 >= na && j0 + BK <= kn) {
      const half_t* kb = Kb + (int64_t)(j0 - na) * d;
#pragma unroll
      for (int q = 0; q < NDK; ++q) dma16s(kb, ko[q], &sK[buf][(wave * NDK + q) * 512]);
    } else if (j0 + BK <= na) {
      const half_t* kb = Kp + (int64_t)j0 * d;
#pragma unroll
      for (int q = 0; q < NDK; ++q) dma16s(kb, ko[q], &sK[buf][(wave * NDK + q) * 512]);
    } else {
#pragma unroll
      for (int q = 0; q < NDK; ++q) {
        const int key = min(j0 + kr[q], kn1);
        const half_t* row = key < na ? Kp + (int64_t)key * d : Kb + (int64_t)(key - na) * d;
        const char* src = reinterpret_cast<const char*>(row) + (ko[q] - 2u * (uint32_t)(kr[q] * d));
        dma16(src, &sK[buf][(wave * NDK + q) * 512]);
      }
    }
  };
  auto issue_v = [&](int buf, int j0) {
    if (j0 >= na && j0 + BK <= kn) {
#pragma unroll
      for (int q = 0; q < NDV; ++q) dma16s(Vb + (j0 - na), vo[q], &sV[buf][(wave * NDV + q) * 512]);
    } else {
#pragma unroll
      for (int q = 0; q < NDV; ++q) {
        const int vrow = min((wave * NDV + q) * 8 + (lane >> 3), d - 1);
        const int c0 = j0 + 8 * ((lane & 7) ^ ((((wave * NDV + q) * 8 + (lane >> 3)) >> 1) & 7));
        const half_t* src = c0 < na ? Vp + (int64_t)vrow * p.ldpv + c0
                                    : Vb + ((int64_t)vrow * p.ldv + min(c0 - na, ldv8));
        dma16(src, &sV[buf][(wave * NDV + q) * 512]);
      }
    }
  };

  // ---- fragment read offsets (bytes).  K: row 16 t + n, chunk 4 s + g at
  // slot chunk ^ n (row & 15 = n); V^T: row 16 u + n, chunk 4 kb + g at slot
  // chunk ^ ((n >> 1) & 7).  The rest of each address is an immediate.
  constexpr int KPER = 4;  // k-steps per 16-chunk swizzle period (the XOR keeps chunk bit 4)
  int koff[KPER], voff[2];
#pragma unroll
  for (int x = 0; x < KPER; ++x) koff[x] = n * 2 * D + 16 * ((4 * x + g) ^ n);
#pragma unroll
  for (int x = 0; x < 2; ++x) voff[x] = n * 128 + 16 * ((4 * x + g) ^ ((n >> 1) & 7));
  // S step i: key tile i % 4, k-step i / 4; PV step i: d tile i % NDT, key block i / NDT
  auto kread = [&](const char* base, int i) {
    const int t = i & 3, s = i >> 2;
    return *reinterpret_cast<const half8*>(base + koff[s % KPER] + (s / KPER) * 16 * 16 + t * 16 * 2 * D);
  };
  auto vread = [&](const char* base, int i) {
    return *reinterpret_cast<const half8*>(base + voff[i / NDT] + (i % NDT) * 16 * 128);
  };
  constexpr int NS1 = 4 * NKS, NS2 = 2 * NDT;
  auto frag = [&](const char* kbase, const char* vbase, int st) {
    return st < NS1 ? kread(kbase, st) : vread(vbase, st - NS1);
  };

  float4_t O[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) O[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float l_run = 0.0f;

  const float c2 = p.scale * 1.4426950408889634f;  // scores to log2 units
  const int key_end = min(kn, offset + q0 + BQ);
  const int ntiles = (key_end + BK - 1) / BK;
  const int lim = min(offset + q0 + 16 * wave + n, kn1);
  const int lim0 = min(offset + q0 + 16 * wave, kn1);  // the wave's smallest lim
  // key offset within a tile of accumulator element (t, i): LDS row
  // 16 t + 4 g + i holds key 32 (t / 2) + 8 g + 4 (t % 2) + i
  auto kof = [&](int t, int i) { return 32 * (t >> 1) + 4 * (t & 1) + i + 8 * g; };
  auto row_max = [](float x) {
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    return fmaxf(x, __shfl_xor(x, 32, 64));
  };

  // ---- prologue: K(0), K(1), V(0) resident; scores of tile 0
  issue_k(0, 0);
  if (ntiles > 1) issue_k(1, BK);
  issue_v(0, 0);
  vm_wait_all();
  lds_barrier();
  float4_t Sc[4], Sn[4];
  half8 fb[PD];
  {
    const char* kbase = reinterpret_cast<const char*>(sK[0]);
#pragma unroll
    for (int t = 0; t < 4; ++t) Sc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < PD; ++i) fb[i] = kread(kbase, i);
#pragma unroll
    for (int i = 0; i < NS1; ++i) {
      Sc[i & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[i % PD], qf[i >> 2], Sc[i & 3], 0, 0, 0);
      if (i + PD < NS1) fb[i % PD] = kread(kbase, i + PD);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float m_ref;
  {
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sv = kof(t, i) > lim ? -INFINITY : Sc[t][i];
        Sc[t][i] = sv;
        mx = fmaxf(mx, sv);
      }
    m_ref = row_max(mx);  // finite: every query sees key 0
  }
  lds_barrier();  // all waves are done with K(0) before K(2) replaces it

  // ---- software pipeline over key tiles (as attn_f16): iteration j, with
  // K(j+1) and V(j) resident and the masked scores of tile j in Sc:
  //   phase 1: MFMA  Sn = K(j+1) Q^T        VALU  P = exp2(Sc c - m c), row sum
  //   phase 2: MFMA  O^T += V(j)^T P^T      VALU  mask Sn, row max of tile j+1
  auto tile_step = [&](int j, auto masked_t) {
    constexpr bool masked = decltype(masked_t)::value;
    const int j0 = j * BK;
    if (j + 2 < ntiles) issue_k(j & 1, j0 + 2 * BK);
    if (j + 1 < ntiles) issue_v((j + 1) & 1, j0 + BK);
    if (j0 + BK > kn) {  // last tile runs past the keys: zero those value columns
      half_t* v = sV[j & 1];
      for (int x = tid; x < D * 8; x += 512) {
        const int r = x >> 3, slot = x & 7;
        const int k0 = j0 + 8 * (slot ^ ((r >> 1) & 7));
        if (k0 + 8 > kn) {
          half8 val = *reinterpret_cast<half8*>(v + r * 64 + slot * 8);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k0 + e >= kn) val[e] = half_t(0);
          *reinterpret_cast<half8*>(v + r * 64 + slot * 8) = val;
        }
      }
      lds_barrier();
    }
    const char* kbase = reinterpret_cast<const char*>(sK[(j + 1) & 1]);
    const char* vbase = reinterpret_cast<const char*>(sV[j & 1]);
    const float mc = m_ref * c2;
    const int thr = lim - (j0 + BK);
#pragma unroll
    for (int t = 0; t < 4; ++t) Sn[t] = float4_t{0.f, 0.f, 0.f, 0.f};
    half8 pf[2];
    float ps = 0.0f, mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PD; ++i) fb[i] = frag(kbase, vbase, i);
    // phase 1: one probability every second score MFMA (16 per lane and tile)
#pragma unroll
    for (int st = 0; st < NS1; ++st) {
      Sn[st & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[st % PD], qf[st >> 2], Sn[st & 3], 0, 0, 0);
      fb[st % PD] = frag(kbase, vbase, st + PD);
      if ((st & 1) == 0) {
        const int x = st >> 1, t = x >> 2, i = x & 3;  // element (t, i): key block t / 2, slot 4 (t % 2) + i
        const float pv = __builtin_amdgcn_exp2f(fmaf(Sc[t][i], c2, -mc));
        ps += pv;
        pf[t >> 1][4 * (t & 1) + i] = static_cast<half_t>(pv);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // phase 2: one masked score of tile j+1 every second PV MFMA, two MFMAs
    // behind the end of the score chain (unmasked below the diagonal)
    auto mask_max = [&](int x) {
      const int t = x >> 2, i = x & 3;
      const float sv = kof(t, i) > thr ? -INFINITY : Sn[t][i];
      Sc[t][i] = sv;  // phase 1 is done with tile j's scores
      mx = fmaxf(mx, sv);
    };
    auto max_only = [&](int x) {
      const int t = x >> 2, i = x & 3;
      Sc[t][i] = Sn[t][i];
      mx = fmaxf(mx, Sn[t][i]);
    };
    auto phase2 = [&](auto&& scores) {
#pragma unroll
      for (int i = 0; i < NS2; ++i) {
        O[i % NDT] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[(NS1 + i) % PD], pf[i / NDT], O[i % NDT], 0, 0, 0);
        if (NS1 + i + PD < NS1 + NS2) fb[(NS1 + i) % PD] = frag(kbase, vbase, NS1 + i + PD);
        if (i >= 2 && ((i - 2) & 1) == 0 && (i - 2) / 2 < 16) scores((i - 2) / 2);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int x = (NS2 - 2) / 2; x < 16; ++x) scores(x);
    };
    if constexpr (masked)
      phase2(mask_max);
    else
      phase2(max_only);
    l_run += ps;
    if (j + 1 < ntiles) {
      // lazy rescale: move the reference only when exp2 would exceed 2^8
      const float m_new = fmaxf(m_ref, row_max(mx));
      if (__builtin_amdgcn_ballot_w64((m_new - m_ref) * c2 > 8.0f)) {
        const float alpha = __builtin_amdgcn_exp2f((m_ref - m_new) * c2);
#pragma unroll
        for (int t = 0; t < NDT; ++t) O[t] = O[t] * alpha;
        l_run *= alpha;
        m_ref = m_new;
      }
    }
    vm_wait_all();
    lds_barrier();
  };
  // single sequences: first the tiles whose successor lies wholly at or
  // before the wave's first query (no mask), then the rest (a ragged batch's
  // instance keeps one masked body: a second one costs it registers)
  int j = 0;
  if constexpr (!VL)
    for (; j + 1 < ntiles && lim0 - (j + 1) * BK >= BK - 1; ++j) tile_step(j, std::false_type{});
  for (; j < ntiles; ++j) tile_step(j, std::true_type{});

  // ---- epilogue: y = round(round(O / l) * round(sigmoid(gate))); O^T
  // accumulator t holds d = 16 t + 4 g + i of the lane's query
  float lt = l_run + __shfl_xor(l_run, 16, 64);
  lt += __shfl_xor(lt, 32, 64);
  const float inv = 1.0f / lt;
  const int row = q0 + 16 * wave + n;
  const int64_t prow = qb0 + min(row, qn - 1);  // packed row (clamped for the loads)
  const half_t* gate = static_cast<const half_t*>(p.gate) + prow * p.ldg + (int64_t)h * p.hsg;
  half_t* y = static_cast<half_t*>(p.y) + prow * p.ldy + (int64_t)h * d;
  auto out4 = [&](int t, half4 gv) {
    half4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = static_cast<float>(to_f16(O[t][e] * inv));
      const float sg = static_cast<float>(to_f16(sigmoid_hw(static_cast<float>(gv[e]))));
      r[e] = static_cast<half_t>(a * sg);
    }
    return r;
  };
  if (p.vec_io == 2) {
    // 16-byte gate and output rows: round(O / l) of the wave's 16 queries is
    // staged in LDS (free after the last key tile; waves 0-3 in sK, 4-7 in
    // sV; rows PWS halves apart, so the 8-byte writes of a lane half cover
    // the 64 banks once), then each lane takes 8 consecutive d of one query:
    // 16-byte gate loads (issued once O is staged) and stores of whole row
    // pieces
    constexpr int PWS = D + 8, CH = D / 8, RPI = 64 / CH, NR = 16 / RPI;
    static_assert(4 * 16 * PWS <= 2 * BK * D, "four waves' staging fits sK or sV");
    half_t* const stg = (wave < 4 ? &sK[0][0] : &sV[0][0]) + (wave & 3) * (16 * PWS);
    const int c8 = 8 * (lane % CH), rl = lane / CH;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      half4 a4;
#pragma unroll
      for (int e = 0; e < 4; ++e) a4[e] = to_f16(O[t][e] * inv);
      *reinterpret_cast<half4*>(stg + n * PWS + 16 * t + 4 * g) = a4;
    }
    half8 gv[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const int rq = q0 + 16 * wave + RPI * q + rl;
      const int64_t pr = qb0 + min(rq, qn - 1);
      gv[q] = *reinterpret_cast<const half8*>(static_cast<const half_t*>(p.gate) + pr * p.ldg + (int64_t)h * p.hsg + c8);
    }
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const int rr = RPI * q + rl, rq = q0 + 16 * wave + rr;
      const half8 av = *reinterpret_cast<const half8*>(stg + rr * PWS + c8);
      half8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sg = static_cast<float>(to_f16(sigmoid_hw(static_cast<float>(gv[q][e]))));
        r[e] = static_cast<half_t>(static_cast<float>(av[e]) * sg);
      }
      if (rq < qn)
        *reinterpret_cast<half8*>(static_cast<half_t*>(p.y) + (int64_t)(qb0 + rq) * p.ldy + (int64_t)h * d + c8) = r;
    }
    lds_barrier();  // staging reads done before the next item's DMA refills sK / sV
  } else if (p.vec_io) {
    half4 gv[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const int d0 = 16 * t + 4 * g;
      gv[t] = d0 < d ? *reinterpret_cast<const half4*>(gate + d0) : half4{};
    }
    if (row < qn) {
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const int d0 = 16 * t + 4 * g;
        if (d0 < d) *reinterpret_cast<half4*>(y + d0) = out4(t, gv[t]);
      }
    }
  } else if (row < qn) {
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const int d0 = 16 * t + 4 * g;
      if (d0 < d) {
        half4 gv;
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = gate[d0 + e];
        const half4 r = out4(t, gv);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[d0 + e] = r[e];
      }
    }
  }
  }  // work items (the last key tile ended with a barrier: LDS is free)
}

// Query tiles of a ragged batch (one work-group, ragged.hpp): the monotone
// spans (written to `spans`, which the attention kernel then reads as its
// sequence offsets), and per sequence its tiles of 128 queries ranked by key
// count (most first, ties in sequence order) for a longest-first launch;
// beyond 8192 tiles in sequence order.  Any offset table keeps the pair
// table inside its T/128 + nseq entries.
__global__ __launch_bounds__(kTabThreads) void attn_tables(const int* __restrict__ cu, int nseq, int T,
                                                           int* __restrict__ spans, int2* __restrict__ pairs,
                                                           int* __restrict__ npairs) {
  __shared__ int s_part[kTabThreads];
  __shared__ int s_R[kMaxRaggedSeq + 1];
  __shared__ int s_total;
  const int tid = threadIdx.x;
  const Ragged g{cu, nseq, T, s_part, s_R};
  rg_spans_1(g, tid);
  __syncthreads();
  rg_spans_2(g, tid);
  __syncthreads();
  rg_spans_3(g, tid);
  __syncthreads();
  for (int j = tid; j <= nseq; j += kTabThreads) spans[j] = s_R[j];
  rg_count_4(g, tid, 128);
  __syncthreads();
  rg_count_5(g, tid, &s_total);
  __syncthreads();
  if (tid == 0) *npairs = s_total;
  rg_attn_6(g, tid, 128, s_total, reinterpret_cast<int*>(pairs));
}

// work-groups resident at once (CUs x occupancy of the instance), per device
template <int D>
int resident_groups() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, attn_f16<D>, 256, 0) != hipSuccess || per <= 0) per = 1;
    cached[dev] = cus * per;
  }
  return cached[dev];
}

template <int D>
int launch(const AttnParams& p0, hipStream_t s) {
  AttnParams p = p0;
  // 8-byte gate and output accesses: every row and head offset a multiple of 4 halves
  p.vec_io = ((reinterpret_cast<uintptr_t>(p.gate) | reinterpret_cast<uintptr_t>(p.y)) & 7) == 0 &&
             p.ldg % 4 == 0 && p.hsg % 4 == 0 && p.ldy % 4 == 0 && p.d % 4 == 0;
  const int qtiles = p.cu_q ? (p.qn + 127) / 128 + p.nseq : (p.qn + 127) / 128;
  const int items = qtiles * p.heads;
  const int groups = items < resident_groups<D>() ? items : resident_groups<D>();
  hipLaunchKernelGGL((attn_f16<D>), dim3(groups), dim3(256), 0, s, p);
  return check_launch("attention");
}

// the single-sequence core at two waves per SIMD
constexpr bool kW8 = true;
template <int D>
int launch_w8(const AttnParams& p0, hipStream_t s) {
  AttnParams p = p0;
  p.vec_io = ((reinterpret_cast<uintptr_t>(p.gate) | reinterpret_cast<uintptr_t>(p.y)) & 7) == 0 &&
             p.ldg % 4 == 0 && p.hsg % 4 == 0 && p.ldy % 4 == 0 && p.d % 4 == 0;
  // 16-byte gate and output rows (the staged epilogue): a full head width
  if (p.vec_io && ((reinterpret_cast<uintptr_t>(p.gate) | reinterpret_cast<uintptr_t>(p.y)) & 15) == 0 &&
      p.ldg % 8 == 0 && p.hsg % 8 == 0 && p.ldy % 8 == 0 && p.d == D)
    p.vec_io = 2;
  // resident work-groups (CUs x occupancy) of the instance launched, per
  // device: the ragged instance carries the prefix-segment logic and may fit
  // fewer per CU, and a grid above the resident count would lose the
  // longest-first item order
  static int cached[64][2] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  const int vl = p.cu_q ? 1 : 0;
  if (cached[dev][vl] == 0) {
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    const hipError_t e = vl ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, attn_f16_w8<D, true>, 512, 0)
                            : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, attn_f16_w8<D, false>, 512, 0);
    if (e != hipSuccess || per <= 0) per = 1;
    cached[dev][vl] = cus * per;
  }
  const int qtiles = p.cu_q ? (p.qn + 127) / 128 + p.nseq : (p.qn + 127) / 128;
  const int items = qtiles * p.heads;
  const int groups = items < cached[dev][vl] ? items : cached[dev][vl];
  if (p.cu_q)
    hipLaunchKernelGGL((attn_f16_w8<D, true>), dim3(groups), dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((attn_f16_w8<D, false>), dim3(groups), dim3(512), 0, s, p);
  return check_launch("attention");
}

}  // namespace

// Workspace: pairs [tiles] int2, the pair count, spans [nseq + 1] int, each
// region 256-byte aligned.
namespace {
size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }
}  // namespace

size_t attn_tables_bytes(int T, int nseq) {
  const size_t tiles = (size_t)(T + 127) / 128 + nseq;
  return al256(tiles * sizeof(int2)) + 256 + al256(((size_t)nseq + 1) * sizeof(int));
}

void attn_carve_tables(AttnParams& p, void* ws) {
  const size_t tiles = (size_t)(p.qn + 127) / 128 + p.nseq;
  char* b = static_cast<char*>(ws);
  p.pairs = reinterpret_cast<int2*>(b);
  b += al256(tiles * sizeof(int2));
  p.npairs = reinterpret_cast<int*>(b);
  p.spans = reinterpret_cast<int*>(b + 256);
}

int attn_f16_tables(AttnParams& p, hipStream_t s) {
  if (p.nseq < 1 || p.nseq > kMaxRaggedSeq) return fail(-1, "attention: 1..4096 sequences");
  hipLaunchKernelGGL(attn_tables, dim3(1), dim3(kTabThreads), 0, s, p.cu_q, p.nseq, p.qn, p.spans, p.pairs,
                     p.npairs);
  if (int rc = check_launch("attention tables")) return rc;
  p.cu_q = p.spans;  // the attention kernel reads the monotone spans
  return 0;
}

bool attn_f16_ok(const AttnParams& p) {
  // per-head byte offsets are 32-bit
  return p.d % 8 == 0 && p.d <= 256 && p.ldv % 8 == 0 && p.ldv >= 64 &&
         (int64_t)p.ldk * p.d < (int64_t(1) << 30) && (int64_t)p.d * p.ldv < (int64_t(1) << 30);
}

bool attn_qfuse_ok(const AttnParams& p) {
  const auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  return kW8 && p.qraw && p.qw && p.qrot && !p.cu_q && p.d == 256 && attn_f16_ok(p) && a16(p.qraw) && a16(p.qw) &&
         a16(p.qrot) && p.ldqr % 8 == 0 && p.hsr % 8 == 0 && p.hsr >= p.d &&
         p.ldqr >= (int64_t)(p.heads - 1) * p.hsr + p.d;
}

int attn_f16_launch(const AttnParams& p, hipStream_t s) {
  if (p.qraw) {
    if (!attn_qfuse_ok(p)) return fail(-1, "attention: the fused query path takes one f16 sequence, d = 256 and aligned rows");
    return launch_w8<256>(p, s);
  }
  if (kW8 && p.d > 128) return launch_w8<256>(p, s);
  if (p.d <= 64) return launch<64>(p, s);
  if (p.d <= 128) return launch<128>(p, s);
  return launch<256>(p, s);
}

}  // namespace clef
