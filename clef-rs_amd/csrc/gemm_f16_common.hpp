// Pieces of the packed-weight f16 GEMM (gemm_f16_pk.hip): the LDS DMA and
// vmcnt helpers and the LDS-staged epilogue, in the same forms as the
// row-major kernel's own (gemm_f16.hip).
#pragma once
#include "common.hpp"
#include "gemm.hpp"

namespace clef {
namespace gemmf16 {

constexpr int kBM = 256, kBK = 64;

// global_load_lds_dwordx4 written as inline asm: the compiler does not see an
// LDS write it would have to order before every later LDS read (it would
// wait for all DMAs in flight, i.e. for the next stage, before computing on
// the current one).  Completion is awaited explicitly (vmcnt) before the
// barrier that publishes a stage.  The LDS destination goes in M0 (low 32
// bits of the LDS address); lane l writes 16 bytes at M0 + 16 l.  The asm
// carries the one wait state an LDS DMA needs after the SALU write of M0
// (the compiler does not see the DMA inside the asm).
__device__ __forceinline__ void dma16(const void* src_lane, void* lds_block) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_block));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src_lane), "{m0}"(m0) : "memory");
}

// The same DMA from a wave-uniform base plus a per-lane 32-bit byte offset
// (no per-lane 64-bit address kept live).  The base is pinned to SGPRs with
// readfirstlane (each half widened as unsigned), and the asm carries the 5
// wait states between that VALU write of an SGPR and a vector-memory read of it.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, void* lds_block) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_block));
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(sb), "{m0}"(m0) : "memory");
}

__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }
template <int N>
__device__ __forceinline__ void vm_wait() {  // s_waitcnt vmcnt(N)
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Epilogue of a wave's TM x TN blocks of 32 x 32 accumulators, staged through
// its own 32 x WN f32 LDS block (stg; the caller has passed a barrier after
// every wave's last fragment read).  acc[i][j][e] holds row (e/4)*8 +
// (lane/32)*4 + e%4, column lane%32 of block (i, j); a 32-row slab is written
// to stg and read back as 4-column chunks, so the global accesses are 8- or
// 16-byte vectors along the rows.  (LDS operations of one wave complete in
// order, so the write -> read -> next write sequence needs no barrier.)
// row0: the wave's first output row; cbase: its first output column (for
// SwiGLU, EPI 2, the output column of its first gate block: blocks j < TN/2
// are gate, j >= TN/2 the up blocks of the same outputs).
template <int TM, int TN, int EPI>
__device__ __forceinline__ void gemm_epilogue_staged(const GemmParams& p, float16_t (&acc)[TM][TN], float* stg,
                                                     int lane, int row0, int cbase) {
  constexpr int WN = TN * 32;
  const int ccol = lane & 31, rgrp = (lane >> 5) * 4;
  constexpr int OW = EPI == 2 ? WN / 2 : WN;  // output columns per wave
  constexpr int CPR = OW / 4;                  // 4-column chunks per row
  constexpr int PER = 32 * CPR / 64;           // chunks per lane per slab
  const int esz = (EPI == 1 || p.dtype_out != 1) ? 4 : 2;
  const bool yvec = ((reinterpret_cast<uintptr_t>(p.y) | (uintptr_t)(p.ldy * esz)) & (4 * esz - 1)) == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) stg[((e >> 2) * 8 + rgrp + (e & 3)) * WN + j * 32 + ccol] = acc[i][j][e];
    const int rbase = row0 + i * 32;
    float4 v[PER], res[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = q * 64 + lane, row = idx / CPR, c4 = idx % CPR;
      if (EPI == 2) {
        const float4 g = *reinterpret_cast<const float4*>(stg + row * WN + c4 * 4);
        const float4 u = *reinterpret_cast<const float4*>(stg + row * WN + OW + c4 * 4);
        // half roundings of neural.metal:35-42
        auto sw = [](float gv, float uv) {
          const float gh = static_cast<float>(static_cast<half_t>(gv));
          const float sh = static_cast<float>(static_cast<half_t>(gh / (1.0f + expf(-gh))));
          return sh * static_cast<float>(static_cast<half_t>(uv));
        };
        v[q] = make_float4(sw(g.x, u.x), sw(g.y, u.y), sw(g.z, u.z), sw(g.w, u.w));
      } else {
        v[q] = *reinterpret_cast<const float4*>(stg + row * WN + c4 * 4);
      }
    }
    if (EPI == 1) {
      // residual reads all issued before the first store
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int idx = q * 64 + lane, r = rbase + idx / CPR, c = cbase + (idx % CPR) * 4;
        const float* src = static_cast<const float*>(p.y) + (int64_t)r * p.ldy + c;
        if (yvec && r < p.M && c + 3 < p.N) {
          res[q] = *reinterpret_cast<const float4*>(src);
        } else {
          res[q] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (r < p.M) {
            if (c < p.N) res[q].x = src[0];
            if (c + 1 < p.N) res[q].y = src[1];
            if (c + 2 < p.N) res[q].z = src[2];
            if (c + 3 < p.N) res[q].w = src[3];
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = q * 64 + lane, r = rbase + idx / CPR, c = cbase + (idx % CPR) * 4;
      if (r >= p.M) continue;
      float4 o = v[q];
      if (EPI == 1) {
        auto rd = [&](float x) { return p.dtype_out == 1 ? static_cast<float>(static_cast<half_t>(x)) : x; };
        o = make_float4(res[q].x + rd(o.x), res[q].y + rd(o.y), res[q].z + rd(o.z), res[q].w + rd(o.w));
      }
      const int64_t off = (int64_t)r * p.ldy + c;
      if (esz == 2) {
        half_t* dst = static_cast<half_t*>(p.y) + off;
        const half_t h[4] = {static_cast<half_t>(o.x), static_cast<half_t>(o.y), static_cast<half_t>(o.z),
                             static_cast<half_t>(o.w)};
        if (yvec && c + 3 < p.N) {
          *reinterpret_cast<half4*>(dst) = half4{h[0], h[1], h[2], h[3]};
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (c + t < p.N) dst[t] = h[t];
        }
      } else {
        float* dst = static_cast<float*>(p.y) + off;
        if (yvec && c + 3 < p.N) {
          *reinterpret_cast<float4*>(dst) = o;
        } else {
          const float f[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (c + t < p.N) dst[t] = f[t];
        }
      }
    }
  }
}

}  // namespace gemmf16
}  // namespace clef
