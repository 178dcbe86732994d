// f16 projection GEMM for large row counts: y = x . W^T, x [M,K], W [N,K]
// (both K-contiguous), f32 accumulation.  Same contract and epilogues as
// gemm.hip (neural.metal:7-125 tile GEMM, projection.rs:82-95); selected for
// M >= 256, K % 64 == 0 and 16-byte aligned rows.
//
// A work-group of 8 waves (4 x 2, two per SIMD) computes a 256 x BN tile
// (or 128 x BN when 256-row tiles would leave CUs idle), each wave
// BM/4 x BN/2 as 16 x 16 blocks on v_mfma_f32_16x16x32_f16 (at most 128
// accumulator registers per wave, which the register allocator keeps in
// place).  K advances in 64-element stages (two 32-deep k-steps) through LDS
// rings filled by global->LDS DMA (buffer_load_dwordx4 ... lds, 1 KiB per
// wave instruction): three slots per
// operand for 128-wide tiles, two activation and three weight slots for
// wider ones, so a stage's weights land two stages ahead of their use.
// Rows are 128 bytes; the 16-byte chunk c of row r is stored at slot
// c ^ ((r >> 1) & 7), so the fragment reads of 16 consecutive rows hit 16
// distinct bank groups.  The DMA lanes pick their source chunk so that the
// lane-ordered LDS writes produce that layout.
//
// 256 x 256 tiles run on gemm_f16_w4 instead: four waves (one per SIMD,
// 128 x 128 each, 256 accumulator registers) whose products, fragment reads
// and DMA are interleaved in a fixed order, one MFMA at a time; the same
// rings, layout, products and epilogue arithmetic, so the results are
// bit-identical.  At 4096 x 12288 x 2048 the matrix cores are busy 0.66 of
// the time against 0.54 with eight compiler-scheduled waves.  Both kernels
// multiply on 16 x 16 x 32 products: on the 256 x 256 tiles they took the
// in-projection from 183.7 to 172.5 us against 32 x 32 x 16 ones (same
// fragment bytes per stage: twice the products, each half as long, so a
// fragment read or DMA request sits beside every second product instead of
// most of them).
#include <algorithm>
#include <utility>

#include "common.hpp"
#include "gemm.hpp"

namespace clef {

// CUs of the current device (cached per device)
static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

namespace {

constexpr int kBM = 256, kBK = 64;  // largest row tile, K stage

// buffer_load_dwordx4 ... lds written as inline asm: the compiler does not
// see an LDS write it would have to order before every later LDS read (it
// would wait for all DMAs in flight, i.e. for the next stage, before
// computing on the current one).  Completion is awaited explicitly (vmcnt)
// before the barrier that publishes a stage.  The source is a buffer resource
// (SGPR base and size) plus a 32-bit lane byte offset; the LDS destination
// goes in M0 (low 32 bits of the LDS address), lane l writing 16 bytes at
// M0 + 16 l.  The asm carries the one wait state an LDS DMA needs after the
// SALU write of M0.  (1-6% faster than global_load_lds_dwordx4 with 64-bit
// lane addresses on the projection shapes, bit-identical.)
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t off, void* lds_block) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_block));
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(off), "s"(r), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t operand_rsrc(const half_t* base, int64_t rows, int64_t ld) {
  // rows * ld * 2 < 2^32 (checked by gemm_f16_dma_ok)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(base), 0, static_cast<int>(static_cast<uint32_t>(rows * ld * 2)),
                                           0x00020000);
}

__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }
template <int N>
__device__ __forceinline__ void vm_wait() {  // s_waitcnt vmcnt(N)
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// vmcnt(n) for an n that is a constant once loops are unrolled
template <int... Ns>
__device__ __forceinline__ void vm_wait_n(int n, std::integer_sequence<int, Ns...>) {
  ((n == Ns ? (vm_wait<Ns>(), 0) : 0), ...);
}
__device__ __forceinline__ void vm_wait_n(int n) { vm_wait_n(n, std::make_integer_sequence<int, 40>{}); }


template <int BM, int BN, int VM, int NSA, int NSB, int EPI, bool PERSIST>
__global__ __launch_bounds__(VM * 128) void gemm_f16_dma(GemmParams p) {
  constexpr int kWaves = VM * 2;  // VM wave rows x 2 wave columns
  constexpr int WM = BM / VM, WN = BN / 2;
  constexpr int TM = WM / 32;                    // 32-row slabs of the epilogue per wave
  constexpr int TM16 = WM / 16, TN16 = WN / 16;  // 16 x 16 product blocks per wave
  // epilogue staging pitches (f16 and f32 elements): a row 8 halves or 4
  // floats longer than the wave's columns puts rows 4 apart 16 banks apart,
  // so the four lane groups of a 16 x 16 accumulator (rows 4 apart, 32 or 64
  // bytes each) write to disjoint banks
  constexpr int PWH = WN + 8, PWF = WN + 4;
  constexpr int NA = BM * 8 / 64 / kWaves;  // A DMA instructions per wave per stage
  constexpr int NB = BN * 8 / 64 / kWaves;
  typedef half8 frag;

  // rings of NSA A (BM x 64) and NSB B (BN x 64) stages; after the last
  // stage the same bytes stage the accumulators for the epilogue
  constexpr int kStA = BM * kBK, kStB = BN * kBK;
  __shared__ __attribute__((aligned(1024))) half_t smem[NSA * kStA + NSB * kStB];
  auto sA = [&](int st) { return smem + st * kStA; };
  auto sB = [&](int st) { return smem + NSA * kStA + st * kStB; };
  static_assert((NSA == 2 || NSA == 3) && (NSB == NSA || NSB == NSA + 1), "two or three stages per operand");
  static_assert(kWaves * 32 * PWF * 4 <= (int)sizeof(smem), "epilogue staging fits the tile buffers");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- tile index with XCD-compact placement (as gemm.hip).  A persistent
  // launch (one work-group per CU, gridDim.x a multiple of 8) takes the tiles
  // blockIdx.x, blockIdx.x + gridDim.x, ..., which stay on its XCD.
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (EPI == 2 ? (p.N + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN);
  const int ntiles = tiles_m * tiles_n;
  auto coords = [&](int t, int& tm0, int& tn0) {
    if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    const int group = 4;
    const int gsize = group * tiles_n;
    const int first_m = (t / gsize) * group;
    const int gm = min(group, tiles_m - first_m);
    tm0 = (first_m + (t % gsize) % gm) * BM;
    tn0 = ((t % gsize) / gm) * (EPI == 2 ? BN / 2 : BN);
  };
  int tile = blockIdx.x, m0 = 0, n0 = 0;
  coords(tile, m0, n0);

  const half_t* X = static_cast<const half_t*>(p.x);
  const half_t* W = static_cast<const half_t*>(p.w);
  const half_t* W2 = static_cast<const half_t*>(p.w2);

  // ---- DMA sources.  Instruction q of this wave fills LDS slots
  // [64 j, 64 j + 64) with j = wave * N + q: lane l writes slot 64 j + l, i.e.
  // row 8 j + l / 8 with swizzled chunk l % 8.  The row's swizzle key
  // ((8 j + l / 8) >> 1) & 7 = (4 j + l / 16) & 7 depends on j only through
  // its parity, so a lane needs two column offsets; the row offsets are
  // uniform.  (Byte offsets fit 32 bits: checked by gemm_f16_dma_ok.)
  int lcol[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) lcol[par] = (((lane & 7) ^ ((4 * par + (lane >> 4)) & 7)) << 3);
  const int lrow = lane >> 3;
  // (tile origin tm0, tn0; part / nparts: the instructions q with
  // q % nparts == part, so a stage's DMA can be spread over the k-blocks of
  // the stage before it; a null sa or sb skips that operand)
  static_assert(EPI != 2 || (WN / 2) % (8 * NB) == 0, "a wave's B rows are one half of its wave column");
  const __amdgpu_buffer_rsrc_t rA = operand_rsrc(X, p.M, p.ldx);
  const __amdgpu_buffer_rsrc_t rB = operand_rsrc(EPI == 2 && (8 * NB * wave) % WN >= WN / 2 ? W2 : W, p.N, p.ldw);
  auto issue = [&](half_t* sa, half_t* sb, int k0, int tm0, int tn0, int part = 0, int nparts = 1) {
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      if (q % nparts != part || !sa) continue;
      const int j = wave * NA + q;
      const int row = min(tm0 + 8 * j + lrow, p.M - 1);
      bdma16(rA, (uint32_t)(row * (int)p.ldx + lcol[j & 1] + k0) * 2u, sa + j * 512);
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      if (q % nparts != part || !sb) continue;
      const int j = wave * NB + q;
      const int row = 8 * j + lrow;
      int nr;
      if (EPI == 2) {  // wave column wb holds [gate | up] rows of the same outputs
        const int wb = row / WN, within = row % WN;
        nr = min(tn0 + wb * (WN / 2) + (within % (WN / 2)), p.N - 1);
      } else {
        nr = min(tn0 + row, p.N - 1);
      }
      bdma16(rB, (uint32_t)(nr * (int)p.ldw + lcol[j & 1] + k0) * 2u, sb + j * 512);
    }
  };

  // Products on v_mfma_f32_16x16x32_f16 (the four-wave kernel's, so both
  // kernels sum every output in the same order), weights as the A operand:
  // acc[I][J] holds row 16 I + lane % 16, columns 16 J + 4 (lane / 16) + e of
  // the wave's block, so a lane's four results stage as one LDS write.
  float4_t acc[TM16][TN16];

  // fragment reads: row r = (wave offset) + 16 i + lane % 16, 16-byte chunk
  // 4 ks + lane / 16 of k-step ks, at chunk ^ ((r >> 1) & 7); the row's key
  // is (lane % 16 >> 1) & 7, so a lane's byte offset within any 16-row block
  // is one of two values (k-step ks); the block offsets are immediates
  const int r16 = lane & 15, c16 = lane >> 4;
  int goff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) goff[ks] = 2 * (r16 * kBK + (((4 * ks + c16) ^ ((r16 >> 1) & 7)) << 3));
  // k-step 1's fragments are requested during k-step 0's products; dma(ks)
  // issues part ks of a later stage's DMA before them
  auto compute = [&](const half_t* sa, const half_t* sb, auto&& dma) {
    const char* ab = reinterpret_cast<const char*>(sa) + wm * WM * kBK * 2;
    const char* bb = reinterpret_cast<const char*>(sb) + wn * WN * kBK * 2;
    frag af[2][TM16], bf[2][TN16];
    auto load = [&](int ks) {
#pragma unroll
      for (int i = 0; i < TM16; ++i) af[ks][i] = *reinterpret_cast<const frag*>(ab + goff[ks] + i * 16 * kBK * 2);
#pragma unroll
      for (int j = 0; j < TN16; ++j) bf[ks][j] = *reinterpret_cast<const frag*>(bb + goff[ks] + j * 16 * kBK * 2);
    };
    load(0);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      dma(ks);
      if (ks == 0) load(1);
#pragma unroll
      for (int i = 0; i < TM16; ++i)
#pragma unroll
        for (int j = 0; j < TN16; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[ks][j], af[ks][i], acc[i][j], 0, 0, 0);
      // one fragment read of k-step 1 after each product of k-step 0, so the
      // reads stream under the products and are in long before their use
      if (ks == 0) {
#pragma unroll
        for (int q = 0; q < TM16 + TN16; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Rings: stage kt+NSA-1 of A and kt+NSB-1 of B are requested while stage
  // kt is multiplied; each wave then waits for its own requests of stage
  // kt+1 before the barrier that publishes it.  Requests complete in issue
  // order, so what may stay in flight at that wait is what was issued after
  // stage kt+1's last request: stage kt+2 of each three-slot operand (with
  // NSA = 2, NSB = 3 the A stage kt+1 is issued before the B stage kt+2).
  // A persistent work-group requests the next tile's first stages during
  // the last stages of the current one, so the ring runs on across tiles
  // (`next`: the next tile's stages were requested).
  constexpr int KEEP = (NSA == 3 ? NA : 0) + (NSB == 3 ? NB : 0);
  const int nk = p.K / kBK;
  auto wait_next = [&](int kt, bool next) {  // before the barrier that publishes stage kt+1
    if constexpr (KEEP > 0) {
      if (kt + 2 < nk || next) {
        vm_wait<KEEP>();
        return;
      }
    }
    vm_wait_all();
  };
#pragma unroll
  for (int st = 0; st < NSB - 1; ++st) {
    if (st < NSA - 1 && st < nk) issue(sA(st), nullptr, st * kBK, m0, n0);
    if (st < nk) issue(nullptr, sB(st), st * kBK, m0, n0);
  }
  wait_next(-1, false);
  lds_barrier();

  // Residual tiles (EPI 1, 128-wide) are read into registers over the last
  // kPD stages, NRB float4 per lane per stage, instead of in the epilogue:
  // every tile of a one-round launch ends at about the same time, and their
  // residual reads would otherwise meet in one burst after the products.
  // Row r, column c of slab i, chunk q are the epilogue's (below).
  constexpr int OW = EPI == 2 ? WN / 2 : WN;  // output columns per wave
  constexpr int CPR = OW / 4;                  // 4-column chunks per row
  constexpr int PER = 32 * CPR / 64;           // chunks per lane per slab
  constexpr bool PF = EPI == 1 && BN == 128;
  constexpr int kPD = 8, NR = TM * PER, NRB = NR / kPD;
  static_assert(!PF || NR % kPD == 0, "prefetch batches");
  const int esz = (EPI == 1 || p.dtype_out != 1) ? 4 : 2;
  const bool yvec = ((reinterpret_cast<uintptr_t>(p.y) | (uintptr_t)(p.ldy * esz)) & (4 * esz - 1)) == 0;
  const bool yvec8 = ((reinterpret_cast<uintptr_t>(p.y) | (uintptr_t)(p.ldy * 2)) & 15) == 0;  // f16 rows
  float4 pre[PF ? NR : 1];
  auto prefetch = [&](int b) {
#pragma unroll
    for (int u = 0; u < NRB; ++u) {
      const int e = b * NRB + u, i = e / PER, q = e % PER, idx = q * 64 + lane;
      const int r = m0 + wm * WM + i * 32 + idx / CPR, c = n0 + wn * OW + (idx % CPR) * 4;
      pre[e] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.y) + (int64_t)r * p.ldy + c);
    }
  };

  int ca = 0, cb = 0;
  for (;;) {  // the tiles of this work-group
    const int ntile = tile + gridDim.x;
    const bool next = PERSIST && ntile < ntiles;
    int nm0 = 0, nn0 = 0;
    if (next) coords(ntile, nm0, nn0);
    const bool pf = PF && yvec && nk >= kPD && m0 + BM <= p.M && n0 + BN <= p.N;
#pragma unroll
    for (int i = 0; i < TM16; ++i)
#pragma unroll
      for (int j = 0; j < TN16; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
    // requests stage ks of this tile or, past its end, of the next one
    auto issue_at = [&](half_t* sa, half_t* sb, int ks, int part = 0, int nparts = 1) {
      if (ks < nk)
        issue(sa, sb, ks * kBK, m0, n0, part, nparts);
      else if (next)
        issue(sa, sb, (ks - nk) * kBK, nm0, nn0, part, nparts);
    };
    auto stage = [&](int kt) {
      const int na = ca == 0 ? NSA - 1 : ca - 1;  // (ca + NSA - 1) % NSA
      const int nb = cb == 0 ? NSB - 1 : cb - 1;
      compute(sA(ca), sB(cb), [&](int kb) {
        if constexpr (NSA == NSB) {
          // the next stage's DMA, half before each of the first two k-blocks'
          // products (whole prefill 0.7% faster than all of it at the stage
          // start, by interleaved A/B; spread over all four k-blocks, the last
          // quarter has too little time to land when the weights come from HBM:
          // 2% slower)
          if (kb < 2) issue_at(sA(na), sB(nb), kt + NSA - 1, kb, 2);
        } else {
          // A one stage ahead before k-block 0, B two stages ahead before
          // k-block 1 (in that order: see wait_next)
          if (kb == 0) issue_at(sA(na), nullptr, kt + NSA - 1);
          if (kb == 1) issue_at(nullptr, sB(nb), kt + NSB - 1);
        }
      });
    };
    auto advance = [&]() {
      ca = ca + 1 == NSA ? 0 : ca + 1;
      cb = cb + 1 == NSB ? 0 : cb + 1;
    };
    const int kmain = pf ? nk - kPD : nk;
    for (int kt = 0; kt < kmain; ++kt) {
      stage(kt);
      wait_next(kt, next);
      lds_barrier();
      advance();
    }
    if constexpr (PF) {
      if (pf) {
#pragma unroll
        for (int d = 0; d < kPD; ++d) {
          stage(nk - kPD + d);
          prefetch(d);
          // issued after stage kt+1's last request: batch d-1, stage kt+2's
          // DMA (NSA = NSB = 3 here) and batch d
          vm_wait_n((d >= 1 ? NRB : 0) + (d + 2 < kPD ? NA + NB : 0) + NRB);
          lds_barrier();
          advance();
        }
      }
    }

    if constexpr (PERSIST) {
      // ---- epilogue of a persistent work-group.  The next tile's first
      // stages are in flight into the other slots; the slots of this tile's
      // last stage are free, and each wave stages 16 x WN slabs in f16 there
      // (waves 0-3 in the A slot, 4-7 in the B slot; rows PWH apart).  Values
      // are rounded to f16 once, as the stores would round them (EPI 0), or as
      // SwiGLU rounds gate and up before combining them (neural.metal:35-42).
      static_assert(EPI != 1 && kWaves == 8 && 4 * 16 * PWH <= kStA && 4 * 16 * PWH <= kStB,
                    "f16 staging of four waves fits a stage slot");
      // read back as 8-column chunks (16-byte loads and stores)
      constexpr int CPR8 = OW / 8, PER8 = 16 * CPR8 / 64;  // chunks per row, per lane per slab
      static_assert(16 * CPR8 % 64 == 0, "whole chunks per lane");
      const int pa = ca == 0 ? NSA - 1 : ca - 1, pb = cb == 0 ? NSB - 1 : cb - 1;
      half_t* const stg = (wave < 4 ? sA(pa) : sB(pb)) + (wave & 3) * (16 * PWH);
      const int scol = lane & 15, srow = (lane >> 4) * 4;
#pragma unroll
      for (int i = 0; i < TM16; ++i) {  // slab i: product block row i
#pragma unroll
        for (int j = 0; j < TN16; ++j)
          *reinterpret_cast<half4*>(stg + scol * PWH + j * 16 + srow) =
              half4{to_f16(acc[i][j][0]), to_f16(acc[i][j][1]), to_f16(acc[i][j][2]), to_f16(acc[i][j][3])};
        const int rbase = m0 + wm * WM + i * 16;
        const int cbase = n0 + wn * OW;
#pragma unroll
        for (int q = 0; q < PER8; ++q) {
          const int idx = q * 64 + lane, row = idx / CPR8, c8 = idx % CPR8;
          half8 h = *reinterpret_cast<const half8*>(stg + row * PWH + c8 * 8);
          if constexpr (EPI == 2) {
            const half8 u = *reinterpret_cast<const half8*>(stg + row * PWH + OW + c8 * 8);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              // the same function as clef_silu_mul's (neural.rs:484-492)
              const float sh = static_cast<float>(to_f16(silu_hw(static_cast<float>(h[t]))));
              h[t] = static_cast<half_t>(sh * static_cast<float>(u[t]));
            }
          }
          const int r = rbase + row, c = cbase + c8 * 8;
          if (r >= p.M) continue;
          half_t* dst = static_cast<half_t*>(p.y) + (int64_t)r * p.ldy + c;
          if (yvec8 && c + 7 < p.N) {
            *reinterpret_cast<half8*>(dst) = h;
          } else {
#pragma unroll
            for (int t = 0; t < 8; ++t)
              if (c + t < p.N) dst[t] = h[t];
          }
        }
      }
      if (!next) break;
      // every wave's staging reads are done before the next tile's DMA
      // (stage 0) refills these slots
      lds_barrier();
      tile = ntile;
      m0 = nm0;
      n0 = nn0;
      continue;
    }

    // ---- epilogue.  The loop's last barrier follows every wave's last
    // fragment read, so each wave now owns a 32 x WN f32 staging block.
    // A 32-row slab (product block rows 2 i and 2 i + 1) is written there
    // and read back as 4-column chunks, so the global accesses are 8- or
    // 16-byte vectors along the rows.  (LDS operations of one wave complete
    // in order, so the write -> read -> next write sequence needs no barrier.)
    float* const stg = reinterpret_cast<float*>(smem) + wave * (32 * PWF);
    const int scol = lane & 15, srow = (lane >> 4) * 4;
  #pragma unroll
    for (int i = 0; i < TM; ++i) {
  #pragma unroll
      for (int h = 0; h < 2; ++h)
  #pragma unroll
        for (int j = 0; j < TN16; ++j)
          *reinterpret_cast<float4_t*>(stg + (16 * h + scol) * PWF + j * 16 + srow) = acc[2 * i + h][j];
      const int rbase = m0 + wm * WM + i * 32;
      const int cbase = n0 + wn * OW;
      if constexpr (EPI != 1) {
        if (esz == 2) {  // f16 output: 8-column chunks, 16-byte stores
          constexpr int CPR8 = OW / 8, PER8 = 32 * CPR8 / 64;
          static_assert(32 * CPR8 % 64 == 0, "whole chunks per lane");
  #pragma unroll
          for (int q = 0; q < PER8; ++q) {
            const int idx = q * 64 + lane, row = idx / CPR8, c8 = idx % CPR8;
            const float* src = stg + row * PWF + c8 * 8;
            float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
            if constexpr (EPI == 2) {
              const float4 ulo = *reinterpret_cast<const float4*>(src + OW);
              const float4 uhi = *reinterpret_cast<const float4*>(src + OW + 4);
              auto sw = [](float gv, float uv) {  // as below (neural.metal:35-42)
                const float gh = static_cast<float>(to_f16(gv));
                const float sh = static_cast<float>(to_f16(silu_hw(gh)));
                return sh * static_cast<float>(to_f16(uv));
              };
              lo = make_float4(sw(lo.x, ulo.x), sw(lo.y, ulo.y), sw(lo.z, ulo.z), sw(lo.w, ulo.w));
              hi = make_float4(sw(hi.x, uhi.x), sw(hi.y, uhi.y), sw(hi.z, uhi.z), sw(hi.w, uhi.w));
            }
            const int r = rbase + row, c = cbase + c8 * 8;
            if (r >= p.M) continue;
            const half8 h = {static_cast<half_t>(lo.x), static_cast<half_t>(lo.y), static_cast<half_t>(lo.z),
                             static_cast<half_t>(lo.w), static_cast<half_t>(hi.x), static_cast<half_t>(hi.y),
                             static_cast<half_t>(hi.z), static_cast<half_t>(hi.w)};
            half_t* dst = static_cast<half_t*>(p.y) + (int64_t)r * p.ldy + c;
            if (yvec8 && c + 7 < p.N) {
              *reinterpret_cast<half8*>(dst) = h;
            } else {
  #pragma unroll
              for (int t = 0; t < 8; ++t)
                if (c + t < p.N) dst[t] = h[t];
            }
          }
          continue;
        }
      }
      float4 v[PER], res[PER];
  #pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int idx = q * 64 + lane, row = idx / CPR, c4 = idx % CPR;
        if (EPI == 2) {
          const float4 g = *reinterpret_cast<const float4*>(stg + row * PWF + c4 * 4);
          const float4 u = *reinterpret_cast<const float4*>(stg + row * PWF + OW + c4 * 4);
          // half roundings of neural.metal:35-42; SiLU on the hardware exp2 and
          // reciprocal (expf and an IEEE division cost ~1.8% of a prefill
          // here), the same function as clef_silu_mul's, so fused and unfused
          // agree bit for bit (neural.rs:484-492)
          auto sw = [](float gv, float uv) {
            const float gh = static_cast<float>(to_f16(gv));
            const float sh = static_cast<float>(to_f16(silu_hw(gh)));
            return sh * static_cast<float>(to_f16(uv));
          };
          v[q] = make_float4(sw(g.x, u.x), sw(g.y, u.y), sw(g.z, u.z), sw(g.w, u.w));
        } else {
          v[q] = *reinterpret_cast<const float4*>(stg + row * PWF + c4 * 4);
        }
      }
      if (EPI == 1) {
        // residual reads all issued before the first store (or made during
        // the last stages)
  #pragma unroll
        for (int q = 0; q < PER; ++q) {
          if (PF && pf) {
            res[q] = pre[PF ? i * PER + q : 0];
            continue;
          }
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

    break;
  }
}

// ---- 256 x 256 tiles on four waves (one per SIMD, 128 x 128 each as 8 x 8
// blocks of 16 x 16, 256 accumulator registers), with the stage's products,
// its fragment reads and the DMA of the stage two ahead interleaved by hand:
// the compiler's own schedule of the eight-wave kernel leaves the matrix
// cores idle while both waves of a SIMD wait on LDS.  Same rings (A: 2
// stages, B: 3), swizzle, tile order, products and epilogue arithmetic as
// gemm_f16_dma, so results are bit-identical to it.
template <int EPI, bool PERSIST, int BN>
__global__ __launch_bounds__(256) void gemm_f16_w4(GemmParams p) {
  constexpr int BM = 256, VM = 2;
  constexpr int kWaves = VM * 2;
  constexpr int WM = BM / VM, WN = BN / 2, TM = WM / 32;
  constexpr int TN16 = WN / 16;                                         // 16-column blocks per wave
  constexpr int NA = BM * 8 / 64 / kWaves, NB = BN * 8 / 64 / kWaves;  // DMA instructions per stage
  static_assert(TM == 4 && NA == 8 && ((BN == 256 && NB == 8) || (BN == 192 && NB == 6) || (BN == 128 && NB == 4)),
                "the hand schedules below assume 128 x 128, 128 x 96 or 128 x 64 per wave");
  typedef half8 frag;
  constexpr int kStA = BM * kBK, kStB = BN * kBK;
  __shared__ __attribute__((aligned(1024))) half_t smem[2 * kStA + 3 * kStB];
  auto sA = [&](int st) { return smem + st * kStA; };
  auto sB = [&](int st) { return smem + 2 * kStA + st * kStB; };
  // epilogue staging pitches, as gemm_f16_dma's (rows 4 apart 16 banks apart)
  constexpr int PWH = WN + 8, PWF = WN + 4;
  static_assert(kWaves * 32 * PWF * 4 <= (int)sizeof(smem), "one-tile epilogue staging fits");
  static_assert(kWaves * 16 * PWH <= kStB, "persistent epilogue staging fits one B slot");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // tile index with XCD-compact placement, as gemm_f16_dma's
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = (EPI == 2 ? (p.N + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN);
  const int ntiles = tiles_m * tiles_n;
  auto coords = [&](int t, int& tm0, int& tn0) {
    if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    const int group = 4, gsize = group * tiles_n;
    const int first_m = (t / gsize) * group, gm = min(group, tiles_m - first_m);
    tm0 = (first_m + (t % gsize) % gm) * BM;
    tn0 = ((t % gsize) / gm) * (EPI == 2 ? BN / 2 : BN);
  };
  int tile = blockIdx.x, m0 = 0, n0 = 0;
  coords(tile, m0, n0);

  const half_t* X = static_cast<const half_t*>(p.x);
  const half_t* W = static_cast<const half_t*>(p.w);
  const half_t* W2 = static_cast<const half_t*>(p.w2);
  // DMA instruction q of this wave fills LDS slots [64 j, 64 j + 64), j =
  // wave * 8 + q, as gemm_f16_dma's issue()
  int lcol[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) lcol[par] = (((lane & 7) ^ ((4 * par + (lane >> 4)) & 7)) << 3);
  const int lrow = lane >> 3;
  // buffer resources over x and the weights; a wave's B rows lie in one half
  // of its wave column (gate or up rows for SwiGLU), so it takes one resource
  static_assert(EPI != 2 || WN == 2 * 8 * NB, "a wave's B rows are one half of its wave column");
  const __amdgpu_buffer_rsrc_t rA = operand_rsrc(X, p.M, p.ldx);
  const __amdgpu_buffer_rsrc_t rB = operand_rsrc(EPI == 2 && (wave & 1) ? W2 : W, p.N, p.ldw);
  auto dma_a = [&](int slot, int tm0, int ks, int q) {
    const int j = wave * NA + q;
    const int row = min(tm0 + 8 * j + lrow, p.M - 1);
    bdma16(rA, (uint32_t)(row * (int)p.ldx + lcol[j & 1] + ks * kBK) * 2u, sA(slot) + j * 512);
  };
  auto dma_b = [&](int slot, int tn0, int ks, int q) {
    const int j = wave * NB + q;
    const int row = 8 * j + lrow;
    int nr;
    if (EPI == 2) {  // wave column wb holds [gate | up] rows of the same outputs
      const int wb = row / WN, within = row % WN;
      nr = min(tn0 + wb * (WN / 2) + (within % (WN / 2)), p.N - 1);
    } else {
      nr = min(tn0 + row, p.N - 1);
    }
    bdma16(rB, (uint32_t)(nr * (int)p.ldw + lcol[j & 1] + ks * kBK) * 2u, sB(slot) + j * 512);
  };

  // Products on v_mfma_f32_16x16x32_f16: the wave's 128 x 128 as 8 x 8
  // blocks of 16 x 16, a stage as two 32-deep k-steps.  Fragment of block I
  // at k-step ks: lane l holds row 16 I + l % 16, k 32 ks + 8 (l / 16) .. + 7
  // (16 rows x 4 chunks per read: with the (row >> 1) & 7 swizzle, every 16
  // lanes of a read cover all 64 banks).  A block I is read into FA[I] once
  // its eight products of the current k-step are issued; B blocks into the
  // other half of FB.
  const int r16 = lane & 15, c16 = lane >> 4;
  int goff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) goff[ks] = 2 * (r16 * kBK + (((4 * ks + c16) ^ ((r16 >> 1) & 7)) << 3));
  frag FA[8], FB[2][TN16];
  auto rd = [&](int sa, int sb, int ks, int q, int fb) {  // q < 8: A block q, else B block q - 8 into FB[fb]
    if (q < 8)
      FA[q] = *reinterpret_cast<const frag*>(reinterpret_cast<const char*>(sA(sa)) + wm * WM * kBK * 2 + goff[ks] +
                                             q * 16 * kBK * 2);
    else
      FB[fb][q - 8] = *reinterpret_cast<const frag*>(reinterpret_cast<const char*>(sB(sb)) + wn * WN * kBK * 2 +
                                                     goff[ks] + (q - 8) * 16 * kBK * 2);
  };
  // acc[I][J] holds row 16 I + lane % 16, columns 16 J + 4 (lane / 16) + e
  // (weights as the A operand: the transposed block, so a lane's four
  // results are consecutive columns of one row and stage as one 8- or
  // 16-byte LDS write)
  float4_t acc[8][TN16];

  const int nk = p.K / kBK;
  // prologue: stages 0 and 1 requested, stage 0 published, its first k-block
  // read.  Requests complete in issue order, so waiting until NA + NB remain
  // in flight waits for stage 0.
#pragma unroll
  for (int q = 0; q < NA; ++q) dma_a(0, m0, 0, q);
#pragma unroll
  for (int q = 0; q < NB; ++q) dma_b(0, n0, 0, q);
  if (nk > 1) {
#pragma unroll
    for (int q = 0; q < NA; ++q) dma_a(1, m0, 1, q);
#pragma unroll
    for (int q = 0; q < NB; ++q) dma_b(1, n0, 1, q);
    vm_wait<NA + NB>();
  } else {
    vm_wait_all();
  }
  lds_barrier();
#pragma unroll
  for (int q = 0; q < 8 + TN16; ++q) rd(0, 0, 0, q, 0);

  // One stage: 2 k-steps x P products (P = 8 TN16; block row I outer, column
  // J inner).  In k-step 0 the products carry k-step 1's fragment reads (B
  // one per two products from product 1, A block I after its last product)
  // and, from product P/4 + 1, the DMA of B two stages ahead (into the slot
  // stage s-1 freed), one per four products.  In k-step 1 the wave waits at
  // product P/8 - 2 (6 or 2) for its own requests of stage s+1, the barrier
  // publishes them and frees stage s's A slot, and the products carry stage
  // s+1's first fragment reads and the DMA of A two stages ahead (128 x 128
  // per wave: B reads at the odd products 9 .. 23, A requests one per four
  // from product 9; 128 x 96 and 128 x 64: B reads at the even products
  // from 4, A requests one per three from product 5).
  // has1 / has2: stages s+1 / s+2 exist (compile-time, so the steady state
  // has no branches between its instructions); the stage-(s+2) requests go
  // to tile (tm2, tn2) at k-stage ks2.
  // A persistent tile's epilogue issues its global stores after the requests
  // of the next tile's first two stages and before that tile's B(2): when the
  // tile was whole (epi_pending), exactly SEPI stores per wave, so the first
  // stage's wait can leave them in flight (vmcnt counts in issue order).
  // Store epilogue only: with SwiGLU's the flag made the compiler peel the
  // first stage, which spilled registers.
  constexpr int P = 8 * TN16;
  constexpr int SEPI = 8 * (16 * ((EPI == 2 ? WN / 2 : WN) / 8) / 64);
  static_assert(NB + SEPI < 64, "vmcnt is 6 bits");
  bool epi_pending = false;
  int ca = 0, cb = 0;
  auto stage = [&](int tm2, int tn2, int ks2, auto has1_t, auto has2_t) {
    constexpr bool has1 = decltype(has1_t)::value, has2 = decltype(has2_t)::value;
    const int na2 = ca, nb2 = cb == 0 ? 2 : cb - 1;      // slots of A(s+2) and B(s+2)
    const int ca1 = ca ^ 1, cb1 = cb == 2 ? 0 : cb + 1;  // slots of stage s+1
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int m = 0; m < P; ++m) {
        const int I = m / TN16, J = m % TN16;
        acc[I][J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(FB[ks][J], FA[I], acc[I][J], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (ks == 0) {
          if (J == TN16 - 1) rd(ca, cb, 1, I, 0);
          if (m < 2 * TN16 && (m & 1)) rd(ca, cb, 1, 8 + (m >> 1), 1);
          if (m > P / 4 && m <= P / 4 + 4 * NB && ((m - P / 4 - 1) & 3) == 0 && has2)
            dma_b(nb2, tn2, ks2, (m - P / 4 - 1) >> 2);
        } else {
          if (m == P / 8 - 2 && has1) {
            // in flight after stage s+1's requests: B(s+2) only, and in the
            // first stage after a whole tile's epilogue, its stores
            if (has2) {
              if (EPI == 0 && epi_pending)
                vm_wait<NB + SEPI>();
              else
                vm_wait<NB>();
            } else {
              vm_wait_all();
            }
            lds_barrier();
          }
          if (has1) {
            if (J == TN16 - 1) rd(ca1, cb1, 0, I, 0);
            if constexpr (BN == 256) {
              if (m >= 8 && m < 24 && (m & 1)) rd(ca1, cb1, 0, 8 + ((m - 8) >> 1), 0);
              if (m >= 9 && m < 41 && ((m - 9) & 3) == 0 && has2) dma_a(na2, tm2, ks2, (m - 9) >> 2);
            } else {
              if (m >= 4 && m < 4 + 2 * TN16 && !(m & 1)) rd(ca1, cb1, 0, 8 + ((m - 4) >> 1), 0);
              if (m >= 5 && m < 29 && (m - 5) % 3 == 0 && has2) dma_a(na2, tm2, ks2, (m - 5) / 3);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    ca = ca1;
    cb = cb1;
    epi_pending = false;
  };
  typedef std::true_type Y_;
  typedef std::false_type N_;

  const int esz = (EPI == 1 || p.dtype_out != 1) ? 4 : 2;
  const bool yvec = ((reinterpret_cast<uintptr_t>(p.y) | (uintptr_t)(p.ldy * esz)) & (4 * esz - 1)) == 0;
  const bool yvec8 = ((reinterpret_cast<uintptr_t>(p.y) | (uintptr_t)(p.ldy * 2)) & 15) == 0;  // f16 rows
  constexpr int OW = EPI == 2 ? WN / 2 : WN;  // output columns per wave
  constexpr int CPR = OW / 4, PER = 32 * CPR / 64;
  const int scol = lane & 15, srow = (lane >> 4) * 4;
  auto zero = [&] {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < TN16; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  };

  if constexpr (PERSIST) {
    // f16 output, more tiles than CUs (nk >= 2, checked by the launch): one
    // work-group per CU runs the tiles blockIdx.x, blockIdx.x + gridDim.x,
    // ...; the last two stages of a tile request the next tile's first two,
    // and the last tile re-requests its own (in bounds, never read), which
    // keeps one straight-line stage sequence for every tile
    for (;;) {
      const int ntile = tile + gridDim.x;
      const bool next = ntile < ntiles;
      int nm0 = m0, nn0 = n0;
      if (next) coords(ntile, nm0, nn0);
      zero();
      for (int s = 0; s + 2 < nk; ++s) stage(m0, n0, s + 2, Y_{}, Y_{});
      stage(nm0, nn0, 0, Y_{}, Y_{});
      stage(nm0, nn0, 1, Y_{}, Y_{});

      // epilogue: the B slot of this tile's last stage is free (every wave
      // passed that stage's barrier, and the next request into it is the
      // next tile's B(2)); each wave stages its 16 x WN slabs there in f16
      // (rows PWH apart), rounded once as the stores would be, and as SwiGLU
      // rounds gate and up before combining them (neural.metal:35-42).  Slab
      // i holds the 16-row block i.
      // read back as 8-column chunks (16-byte loads and stores)
      constexpr int CPR8 = OW / 8, PER8 = 16 * CPR8 / 64;  // chunks per row, per lane per slab
      static_assert(16 * CPR8 % 64 == 0, "whole chunks per lane");
      const int lastb = cb == 0 ? 2 : cb - 1;
      half_t* const stg = sB(lastb) + wave * (16 * PWH);
      const bool whole = yvec8 && m0 + BM <= p.M && n0 + (EPI == 2 ? BN / 2 : BN) <= p.N;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < TN16; ++j)
          *reinterpret_cast<half4*>(stg + scol * PWH + j * 16 + srow) =
              half4{to_f16(acc[i][j][0]), to_f16(acc[i][j][1]), to_f16(acc[i][j][2]), to_f16(acc[i][j][3])};
        const int rbase = m0 + wm * WM + i * 16;
        const int cbase = n0 + wn * OW;
#pragma unroll
        for (int q = 0; q < PER8; ++q) {
          const int idx = q * 64 + lane, row = idx / CPR8, c8 = idx % CPR8;
          half8 h = *reinterpret_cast<const half8*>(stg + row * PWH + c8 * 8);
          if constexpr (EPI == 2) {
            const half8 u = *reinterpret_cast<const half8*>(stg + row * PWH + OW + c8 * 8);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              // the same function as clef_silu_mul's (neural.rs:484-492)
              const float sh = static_cast<float>(to_f16(silu_hw(static_cast<float>(h[t]))));
              h[t] = static_cast<half_t>(sh * static_cast<float>(u[t]));
            }
          }
          const int r = rbase + row, c = cbase + c8 * 8;
          half_t* dst = static_cast<half_t*>(p.y) + (int64_t)r * p.ldy + c;
          if (whole) {  // one 16-byte store per chunk: SEPI per wave
            *reinterpret_cast<half8*>(dst) = h;
          } else {
            if (r >= p.M) continue;
            if (yvec8 && c + 7 < p.N) {
              *reinterpret_cast<half8*>(dst) = h;
            } else {
#pragma unroll
              for (int t = 0; t < 8; ++t)
                if (c + t < p.N) dst[t] = h[t];
            }
          }
        }
      }
      epi_pending = EPI == 0 && whole;
      if (!next) break;
      // every wave's staging reads are done before the next tile's first
      // stage requests B(2) into this slot
      lds_barrier();
      tile = ntile;
      m0 = nm0;
      n0 = nn0;
    }
    vm_wait_all();  // the re-requested stages land before the work-group ends
  } else {
    zero();
    if (nk >= 2) {
      // the persistent form's straight-line stage sequence: the last two
      // stages re-request this tile's first two (in bounds, never read), so
      // every stage is the same code (with separate tail stages the register
      // allocator spills inside the K loop); those requests land before the
      // epilogue reuses their slots
      for (int s = 0; s + 2 < nk; ++s) stage(m0, n0, s + 2, Y_{}, Y_{});
      stage(m0, n0, 0, Y_{}, Y_{});
      stage(m0, n0, 1, Y_{}, Y_{});
      vm_wait_all();
    } else {
      stage(0, 0, 0, N_{}, N_{});
    }

    // epilogue of a one-tile work-group: each wave stages 32 x WN f32 slabs
    // (rows PWF apart) in its own 16.5 KiB of the tile buffers, which the
    // last stage may still be reading for a slower wave: the barrier comes
    // first (no request is in flight)
    lds_barrier();
    float* const stg = reinterpret_cast<float*>(smem) + wave * (32 * PWF);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < TN16; ++j)
          *reinterpret_cast<float4_t*>(stg + (16 * h + scol) * PWF + j * 16 + srow) = acc[2 * i + h][j];
      const int rbase = m0 + wm * WM + i * 32;
      const int cbase = n0 + wn * OW;
      float4 v[PER], res[PER];
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int idx = q * 64 + lane, row = idx / CPR, c4 = idx % CPR;
        if (EPI == 2) {
          const float4 g = *reinterpret_cast<const float4*>(stg + row * PWF + c4 * 4);
          const float4 u = *reinterpret_cast<const float4*>(stg + row * PWF + OW + c4 * 4);
          auto sw = [](float gv, float uv) {  // as gemm_f16_dma's (neural.metal:35-42)
            const float gh = static_cast<float>(to_f16(gv));
            const float sh = static_cast<float>(to_f16(silu_hw(gh)));
            return sh * static_cast<float>(to_f16(uv));
          };
          v[q] = make_float4(sw(g.x, u.x), sw(g.y, u.y), sw(g.z, u.z), sw(g.w, u.w));
        } else {
          v[q] = *reinterpret_cast<const float4*>(stg + row * PWF + c4 * 4);
        }
      }
      if (EPI == 1) {  // residual reads all issued before the first store
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
          auto rdd = [&](float x) { return p.dtype_out == 1 ? static_cast<float>(static_cast<half_t>(x)) : x; };
          o = make_float4(res[q].x + rdd(o.x), res[q].y + rdd(o.y), res[q].z + rdd(o.z), res[q].w + rdd(o.w));
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
}

template <int BM, int BN, int EPI>
int launch(const GemmParams& p, hipStream_t s) {
  // three stages where they fit in LDS (128-wide tiles: 3 x 48 KiB, or
  // 3 x 32 KiB for 128 x 128): the DMA then runs two stages ahead (whole
  // prefill 1.4% faster, interleaved A/B, all from the residual GEMMs).
  // Wider tiles keep two A stages and three B (weight) stages: 160 KiB at
  // 256 x 256, 136 KiB at 256 x 192.
  constexpr int NSA = BN == 128 ? 3 : 2, NSB = 3;
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tiles_n = EPI == 2 ? (p.N + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  constexpr int VM = 4;  // 8 waves, two per SIMD (WM = BM / 4 rows each)
  const int ntiles = tiles_m * tiles_n, cus = device_cus();
  // More tiles than CUs: one persistent work-group per CU runs its tiles
  // back to back, requesting the next tile's first stages during the last
  // stages of the current one (no prologue wait, no gap between work-groups).
  // It stages the epilogue in f16 in the slots the last stage frees: f16
  // output, the store and SwiGLU epilogues.
  // (256 x 256 tiles: the four-wave kernel, whose persistent form also
  // serves launches of one round, one tile per work-group, 1% faster there
  // than its one-tile form, which stages the epilogue in f32 and serves f32
  // output and the residual add)
  const bool persistent = EPI != 1 && p.dtype_out == 1 && ntiles > cus && (cus & 7) == 0 && p.K / kBK >= 2;
  if constexpr (BM == 256 && (BN == 256 || (BN != 256 && EPI != 1))) {
    if constexpr (EPI != 1) {
      if (p.dtype_out == 1 && (cus & 7) == 0 && p.K / kBK >= 2) {
        hipLaunchKernelGGL((gemm_f16_w4<EPI, true, BN>), dim3(ntiles < cus ? ntiles : cus), dim3(256), 0, s, p);
        return check_launch("gemm");
      }
    }
    hipLaunchKernelGGL((gemm_f16_w4<EPI, false, BN>), dim3(ntiles), dim3(256), 0, s, p);
  } else {
    if constexpr (EPI != 1) {
      if (persistent) {
        hipLaunchKernelGGL((gemm_f16_dma<BM, BN, VM, NSA, NSB, EPI, true>), dim3(cus), dim3(VM * 128), 0, s, p);
        return check_launch("gemm");
      }
    }
    hipLaunchKernelGGL((gemm_f16_dma<BM, BN, VM, NSA, NSB, EPI, false>), dim3(ntiles), dim3(VM * 128), 0, s, p);
  }
  return check_launch("gemm");
}

// w_ab [2 Hv, K] in MFMA fragment order: k-step s (32 columns), output block
// j (16 rows), lane l, element e hold w_ab[16 j + l % 16][32 s + 8 (l / 16) + e],
// so a wave reads one block's fragment as 1 KiB of consecutive bytes.
__global__ void ab_pack_f16(const half_t* __restrict__ w, int64_t ldw, int K, int no, half8* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (s, j, lane)
  const int nb = no / 16;
  if (idx >= (int64_t)(K / 32) * nb * 64) return;
  const int lane = static_cast<int>(idx % 64), j = static_cast<int>((idx / 64) % nb);
  const int st = static_cast<int>(idx / (64 * nb));
  out[idx] = *reinterpret_cast<const half8*>(w + (int64_t)(16 * j + lane % 16) * ldw + 32 * st + 8 * (lane / 16));
}

// [a | b] = x . w_ab^T and the DeltaNet gates for 16 tokens per work-group of
// 16 waves (v_mfma_f32_16x16x32_f16).  The tokens' x rows go to LDS once, with
// row-contiguous 16-byte loads, the 16-byte column chunk c of row r stored at
// c ^ (r & 7); wave q then takes the k-steps q, q + 16, ..., its x fragments
// from LDS and its w_ab fragments straight from the packed copy (1 KiB per
// load, L2-resident), and the 16 partial sums meet in LDS in a fixed order
// (a token's result does not depend on its position in the batch).  With 16
// waves a group has its whole share of loads in flight at once.
// (Fragments read from row-major global memory would touch 16 rows per
// instruction, which leaves the address unit the bottleneck.)  Each output is
// rounded to f16 as the reference's separate a and b projections store it
// (qwen.rs:612-623), then turned into the decay or the strength.
template <int HV>
__global__ __launch_bounds__(1024) void ab_gates_f16(const half_t* __restrict__ x, int64_t ldx,
                                                    const half8* __restrict__ wpk, int K,
                                                    const float* __restrict__ dt, const float* __restrict__ alog,
                                                    float* __restrict__ g, float* __restrict__ beta, int T) {
  constexpr int NB = 2 * HV / 16;  // 16-output blocks
  constexpr int NW = 16;           // waves
  extern __shared__ __attribute__((aligned(16))) half_t sx[];  // [16][K], then the partial sums
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.x * 16;
  const int nsteps = K / 32;
  constexpr int U = 16 / NB;  // k-steps per batch of w_ab loads (16 loads)
  half8 b[U][NB];
  auto load_b = [&](int s0) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s0 + NW * u < nsteps)
#pragma unroll
        for (int j = 0; j < NB; ++j) b[u][j] = wpk[((int64_t)(s0 + NW * u) * NB + j) * 64 + lane];
  };
  load_b(wave);  // independent of x: in flight while x is staged
  // x: 512-byte row segments, 32 threads each; K / 256 segments per row
  {
    const int spr = K / 256, nseg = 16 * spr, l32 = tid & 31;
    constexpr int XB = 4;  // segments per thread in flight together
    for (int s0 = tid >> 5; s0 < nseg; s0 += 32 * XB) {
      half8 v[XB];
#pragma unroll
      for (int i = 0; i < XB; ++i) {
        const int sg = s0 + 32 * i;
        if (sg < nseg) {
          const int r = sg / spr, c = (sg % spr) * 32 + l32;
          v[i] = *reinterpret_cast<const half8*>(x + (int64_t)min(t0 + r, T - 1) * ldx + c * 8);
        }
      }
#pragma unroll
      for (int i = 0; i < XB; ++i) {
        const int sg = s0 + 32 * i;
        if (sg < nseg) {
          const int r = sg / spr, c = (sg % spr) * 32 + l32;
          *reinterpret_cast<half8*>(sx + r * K + ((c ^ (r & 7)) << 3)) = v[i];
        }
      }
    }
  }
  __syncthreads();
  float4_t acc[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) acc[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // fragment lane layout: row lane % 16, k 8 (lane / 16) .. + 7 of the k-step
  const int fr = lane & 15, fg = lane >> 4;
  for (int s0 = wave; s0 < nsteps; s0 += NW * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = s0 + NW * u;
      if (st < nsteps) {
        const int c = 4 * st + fg;
        const half8 a = *reinterpret_cast<const half8*>(sx + fr * K + ((c ^ (fr & 7)) << 3));
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[u][j], acc[j], 0, 0, 0);
      }
    }
    if (s0 + NW * U < nsteps) load_b(s0 + NW * U);
  }
  __syncthreads();  // x no longer read: its LDS holds the partial sums
  float4_t* part = reinterpret_cast<float4_t*>(sx);  // [NW][NB][64]
#pragma unroll
  for (int j = 0; j < NB; ++j) part[(wave * NB + j) * 64 + lane] = acc[j];
  __syncthreads();
  // block j's sums, row r: token t0 + 4 (lane / 16) + r, output 16 j + lane % 16
  if (wave >= NB) return;
  const int j = wave;
  float4_t v4 = part[j * 64 + lane];
  for (int q = 1; q < NW; ++q) v4 += part[(q * NB + j) * 64 + lane];
  const int n = j * 16 + fr;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * fg + r;
    if (t >= T) continue;
    const float v = static_cast<float>(static_cast<half_t>(v4[r]));
    if (n < HV)
      g[(int64_t)t * HV + n] = delta_decay(v, dt[n], alog[n]);
    else
      beta[(int64_t)t * HV + n - HV] = delta_strength(v);
  }
}

}  // namespace

int ab_pack_f16_launch(const void* w_ab, int64_t ldw, int K, int Hv, void* packed, hipStream_t s) {
  const int64_t n = (int64_t)(K / 32) * (2 * Hv / 16) * 64;
  hipLaunchKernelGGL(ab_pack_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     static_cast<const half_t*>(w_ab), ldw, K, 2 * Hv, static_cast<half8*>(packed));
  return check_launch("delta_gates_pack");
}

int ab_gates_f16_launch(const void* x, int64_t ldx, const void* packed, int K, const float* dt, const float* a_log,
                        float* g, float* beta, int T, int Hv, hipStream_t s) {
  const dim3 grid((T + 15) / 16);
  // 16 rows of x (f16), reused for the 16 x (2 Hv / 16) x 1 KiB partial sums
  const size_t lds = std::max((size_t)32 * K, (size_t)16 * (2 * Hv / 16) * 1024);
  auto X = static_cast<const half_t*>(x);
  auto P = static_cast<const half8*>(packed);
  if (Hv == 16)
    hipLaunchKernelGGL(ab_gates_f16<16>, grid, dim3(1024), lds, s, X, ldx, P, K, dt, a_log, g, beta, T);
  else if (Hv == 32)
    hipLaunchKernelGGL(ab_gates_f16<32>, grid, dim3(1024), lds, s, X, ldx, P, K, dt, a_log, g, beta, T);
  else if (Hv == 64)
    hipLaunchKernelGGL(ab_gates_f16<64>, grid, dim3(1024), lds, s, X, ldx, P, K, dt, a_log, g, beta, T);
  else
    return fail(-1, "gates projection: Hv must be 16, 32 or 64");
  return check_launch("delta_gates_proj");
}

// (the DMA reads x and the weights through buffer resources: byte offsets
// below 2^32)
bool gemm_f16_dma_ok(const GemmParams& p) {
  return p.dtype_in == 1 && p.vec && p.M >= kBM && p.K % kBK == 0 &&
         (int64_t)p.M * p.ldx < (int64_t(1) << 31) && (int64_t)p.N * p.ldw < (int64_t(1) << 31);
}


// Tile shape: one tile per CU at a time (the LDS holds one), so a launch
// takes ceil(tiles / CUs) rounds, each as long as a tile; a smaller tile
// costs a little more per output (fewer products per fragment read and per
// byte moved).  The shape with the least rounds x area x that cost wins,
// e.g. 256 x 256 for N = 12288, 256 x 192 for N = 9216 (768 tiles: 3 full
// rounds instead of 2.25), 256 x 128 for M = 4096, N = 2048 (256 tiles: one
// round), 128 x 128 for M = N = 2048 (256 tiles instead of 128 of 256 x 128,
// which leave half the CUs idle).  SwiGLU keeps widths 256 or 128 (its wave
// columns pair gate and up blocks).  Returns the width; *bm the row tile.
int gemm_f16_tile_shape(const GemmParams& p, int epilogue, int* bm) {
  const int n_eff = epilogue == 2 ? 2 * p.N : p.N;
  const long cus = device_cus();
  auto cost = [&](int rows, int bn, double per_out) {
    const long tiles = (long)((p.M + rows - 1) / rows) * ((n_eff + bn - 1) / bn);
    return (double)((tiles + cus - 1) / cus) * rows * bn * per_out;
  };
  struct Cand { int bm, bn; double c; };
  const Cand cands[] = {{256, 256, cost(256, 256, 1.0)},
                        {256, 192, epilogue == 2 ? 1e300 : cost(256, 192, 1.1)},
                        {256, 128, cost(256, 128, 1.2)},
                        {128, 128, cost(128, 128, 1.5)}};
  Cand best = cands[0];
  for (const Cand& c : cands)
    if (c.c < best.c) best = c;
  *bm = best.bm;
  return best.bn;
}

int gemm_f16_dma_launch(const GemmParams& p, int epilogue, hipStream_t s) {
  int bm = kBM;
  const int bn = gemm_f16_tile_shape(p, epilogue, &bm);
  if (bm == 128) {
    if (epilogue == 0) return launch<128, 128, 0>(p, s);
    if (epilogue == 1) return launch<128, 128, 1>(p, s);
    return launch<128, 128, 2>(p, s);
  }
  if (epilogue == 0)
    return bn == 256 ? launch<256, 256, 0>(p, s) : bn == 192 ? launch<256, 192, 0>(p, s) : launch<256, 128, 0>(p, s);
  if (epilogue == 1)
    return bn == 256 ? launch<256, 256, 1>(p, s) : bn == 192 ? launch<256, 192, 1>(p, s) : launch<256, 128, 1>(p, s);
  return bn == 256 ? launch<256, 256, 2>(p, s) : launch<256, 128, 2>(p, s);
}

}  // namespace clef
