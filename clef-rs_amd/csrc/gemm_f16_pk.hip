// f16 projection GEMM with pre-packed weights: y = x . W^T, x [M,K] row-major
// (activations), W packed once into MFMA fragment order (weights are static).
// Same contract and epilogues as gemm_f16.hip (neural.metal:7-125 tile GEMM,
// projection.rs:82-95).
//
// Why packed: with both operands staged through LDS, a 256 x 256 tile of 8
// waves reads 48 KiB of fragments and writes 16 KiB of DMA per 16-wide k-step
// and CU, about the LDS's whole 128 bytes per clock at full MFMA rate.  Here
// only x goes through LDS; each wave loads its W fragments straight from the
// packed copy (1 KiB of consecutive bytes per wave instruction, L2-resident).
// Waves: 8 (2 x 4, two per SIMD, 128 x BN/4 each) for 256- and 128-wide
// tiles, 4 (2 x 2, 128 x 96) for 192-wide ones.
//
// Pipeline (K in 64-wide stages; four LDS stages for x):
//   - x of stage kt+3 is DMA'd (global_load_lds_dwordx4) while stage kt is
//     multiplied; stage kt+2 is published (vmcnt + barrier) at the end of
//     stage kt, so the first fragments of stage kt+1 are read during the last
//     k-block of stage kt without a barrier in between;
//   - W fragments of stage kt+1 are loaded into registers during stage kt
//     (two register sets, the stage loop unrolled by two).
// Packed layout (gemm_pack_f16): block nb of 32 rows, k16 step s, lane l hold
// W[32 nb + l % 32][16 s + 8 (l / 32) .. + 7] at ((nb * K/16) + s) * 64 + l
// (16 bytes each); rows are zero-padded to cover every tile width.
// Epilogues: store and residual add (SwiGLU stays on the row-major kernel).
#include <algorithm>
#include <type_traits>

#include "gemm_f16_common.hpp"

namespace clef {
namespace {

using namespace gemmf16;
constexpr int kNS = 4;  // x stages in LDS

__global__ void gemm_pack_f16(const half_t* __restrict__ w, int64_t ldw, int N, int K, int rows,
                              half8* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (nb, s, lane)
  const int ks = K / 16;
  if (idx >= (int64_t)rows / 32 * ks * 64) return;
  const int lane = static_cast<int>(idx % 64), st = static_cast<int>((idx / 64) % ks);
  const int nb = static_cast<int>(idx / (64 * ks));
  const int r = 32 * nb + (lane & 31);
  half8 v = {};
  if (r < N) v = *reinterpret_cast<const half8*>(w + (int64_t)r * ldw + 16 * st + 8 * (lane >> 5));
  out[idx] = v;
}

template <int BN, int NW, int EPI>
__global__ __launch_bounds__(NW * 64) void gemm_f16_pk(GemmParams p) {
  static_assert(EPI == 0 || EPI == 1, "store or residual epilogue");
  static_assert(NW == 4 || NW == 8, "2 x 2 or 2 x 4 waves");
  static_assert(BN % (NW / 2 * 32) == 0, "whole 32-column blocks per wave");
  constexpr int WM = 128, WN = BN / (NW / 2);
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int NA = kBM * 8 / 64 / NW;  // x DMA instructions per wave per stage
  constexpr int kSt = kBM * kBK;        // halves per x stage
  typedef half8 frag;
  static_assert(NW * 32 * WN * 4 <= kNS * kSt * 2, "epilogue staging fits the x stages");

  __shared__ __attribute__((aligned(1024))) half_t smem[kNS * kSt];
  auto sA = [&](int st) { return smem + (st & (kNS - 1)) * kSt; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);

  // ---- tile index with XCD-compact placement (as gemm_f16.hip)
  const int tiles_m = (p.M + kBM - 1) / kBM;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int ntiles = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
  const int group = 4;
  const int gsize = group * tiles_n;
  const int gid = t / gsize;
  const int first_m = gid * group;
  const int gm = min(group, tiles_m - first_m);
  const int tm = first_m + (t % gsize) % gm;
  const int tn = (t % gsize) / gm;
  const int m0 = tm * kBM;
  const int pn0 = tn * BN;  // first packed row of the tile

  const half_t* X = static_cast<const half_t*>(p.x);
  const int ks = p.K / 16;
  // this wave's W fragments: block j, k16 step s at wb + (j * ks + s) * 64 +
  // lane (a uniform base, so each load is a scalar address plus the lane's
  // 16-byte offset)
  const frag* wb = static_cast<const frag*>(p.w) + (int64_t)(pn0 / 32 + wn * TN) * ks * 64;

  // ---- x DMA (as gemm_f16.hip): instruction q of this wave fills 64 slots
  // of 16 bytes, rows 8 j .. 8 j + 7 with j = wave * NA + q, chunk c of row r
  // landing at slot c ^ ((r >> 1) & 7)
  // (byte offsets from the stage's column base; M * ldx < 2^31 is checked)
  uint32_t xoff[NA];
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    const int j = wave * NA + q;
    const int row = min(m0 + 8 * j + (lane >> 3), p.M - 1);
    xoff[q] = 2u * (uint32_t)(row * (int)p.ldx + (((lane & 7) ^ ((4 * (j & 1) + (lane >> 4)) & 7)) << 3));
  }
  auto issue = [&](half_t* sa, int k0) {
#pragma unroll
    for (int q = 0; q < NA; ++q) dma16s(X + k0, xoff[q], sa + (wave * NA + q) * 512);
  };

  float16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // x fragment reads (as gemm_f16.hip): k-block kb of a 32-row block at foff[kb]
  const int frow = lane & 31, fkc = lane >> 5;
  int foff[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) foff[kb] = 2 * (frow * kBK + (((2 * kb + fkc) ^ ((frow >> 1) & 7)) << 3));
  frag af[2][TM];
  auto load_a = [&](const half_t* sa, int kb, frag* a) {
    const char* ab = reinterpret_cast<const char*>(sa) + wm * WM * kBK * 2 + foff[kb];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const frag*>(ab + i * 32 * kBK * 2);
  };

  const int nk = p.K / kBK;
  frag b0[4][TN], b1[4][TN];

  // one stage: x of stage kt+3 requested; per k-block the W fragments of
  // stage kt+1 and the next x fragments are read under the products; at the
  // end stage kt+2 is published and buffer kt is released
  // (steady: kt + 3 < nk, so every request below is made and the stage is
  // compiled without branches; the last stages take the checked form)
  auto stage = [&](auto steady, int kt, frag (&bc)[4][TN], frag (&bn)[4][TN]) {
    constexpr bool S = decltype(steady)::value;
    const half_t* cur = sA(kt);
    if (S || kt + 3 < nk) issue(sA(kt + 3), (kt + 3) * kBK);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      // the next x fragments: this stage's k-block kb+1, or stage kt+1's first
      const half_t* na = kb < 3 ? cur : sA(kt + 1);
      const bool more_a = S || kb < 3 || kt + 1 < nk;
      const char* ab = reinterpret_cast<const char*>(na) + wm * WM * kBK * 2 + foff[(kb + 1) & 3];
      // column block j: its TM products, then the W fragment that replaces it
      // (stage kt+1, same k-block; the register is free once the products
      // have read it); the next x fragments are all requested after the
      // first block, so they have the rest of this k-block to arrive
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kb & 1][i], bc[kb][j], acc[i][j], 0, 0, 0);
        if (j == 0 && more_a)
#pragma unroll
          for (int i = 0; i < TM; ++i) af[(kb + 1) & 1][i] = *reinterpret_cast<const frag*>(ab + i * 32 * kBK * 2);
        if (S || kt + 1 < nk) bn[kb][j] = wb[((int64_t)j * ks + 4 * (kt + 1) + kb) * 64 + lane];
        __builtin_amdgcn_sched_group_barrier(0x008, TM, 0);  // MFMA
        if (j == 0) __builtin_amdgcn_sched_group_barrier(0x100, TM, 0);  // LDS reads
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // newer than this wave's DMA of stage kt+2: the W loads of two stages and
    // the DMA of stage kt+3 (in order of issue, so vmcnt counts them)
    if (S || kt + 3 < nk)
      vm_wait<8 * TN + NA>();
    else
      vm_wait_all();
    lds_barrier();
  };

  // ---- prologue: x stages 0..2 requested, W of stage 0 loaded, stages 0
  // and 1 published, first x fragments read
#pragma unroll
  for (int st = 0; st < 3; ++st)
    if (st < nk) issue(sA(st), st * kBK);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int j = 0; j < TN; ++j) b0[kb][j] = wb[((int64_t)j * ks + kb) * 64 + lane];
  if (nk >= 3)
    vm_wait<NA + 4 * TN>();
  else
    vm_wait<4 * TN>();
  lds_barrier();
  load_a(sA(0), 0, af[0]);
  int kt = 0;
  for (; kt + 4 < nk; kt += 2) {
    stage(std::true_type{}, kt, b0, b1);
    stage(std::true_type{}, kt + 1, b1, b0);
  }
  for (; kt < nk; kt += 2) {
    stage(std::false_type{}, kt, b0, b1);
    if (kt + 1 < nk) stage(std::false_type{}, kt + 1, b1, b0);
  }

  // ---- epilogue (the last barrier follows every wave's last fragment read)
  gemm_epilogue_staged<TM, TN, EPI>(p, acc, reinterpret_cast<float*>(smem) + wave * (32 * WN), lane, m0 + wm * WM,
                                    pn0 + wn * WN);
}

// 8 waves (2 x 4, two per SIMD, 128 x BN/4 each) where BN/4 is a whole
// number of 32-column blocks, else 4 (2 x 2, 128 x BN/2 each)
template <int BN, int EPI>
int launch(const GemmParams& p, hipStream_t s) {
  constexpr int NW = BN % 128 == 0 ? 8 : 4;
  const int tiles_m = (p.M + kBM - 1) / kBM;
  const int tiles_n = (p.N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_f16_pk<BN, NW, EPI>), dim3(tiles_m * tiles_n), dim3(NW * 64), 0, s, p);
  return check_launch("gemm (packed)");
}

}  // namespace

// packed rows: zero-padded so that every tile width's last tile is in bounds
size_t gemm_pack_f16_bytes(int N, int K) {
  const int64_t n = N;
  int64_t rows = 0;
  for (int bn : {256, 192, 128}) rows = std::max(rows, (n + bn - 1) / bn * bn);
  return (size_t)rows * K * 2;
}

int gemm_pack_f16_launch(const void* w, int64_t ldw, int N, int K, void* packed, hipStream_t s) {
  const int rows = static_cast<int>(gemm_pack_f16_bytes(N, K) / ((size_t)K * 2));
  const int64_t n = (int64_t)rows / 32 * (K / 16) * 64;
  hipLaunchKernelGGL(gemm_pack_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     static_cast<const half_t*>(w), ldw, N, K, rows, static_cast<half8*>(packed));
  return check_launch("gemm pack");
}

// packed path: any M >= 1 (rows past M are clamped reads, not stored),
// K % 64 == 0; tile width as gemm_f16_dma_launch; epilogues 0 and 1
int gemm_f16_pk_launch(const GemmParams& p, int epilogue, hipStream_t s) {
  const int bn = gemm_f16_tile_width(p, epilogue);
  if (epilogue == 0) return bn == 256 ? launch<256, 0>(p, s) : bn == 192 ? launch<192, 0>(p, s) : launch<128, 0>(p, s);
  return bn == 256 ? launch<256, 1>(p, s) : bn == 192 ? launch<192, 1>(p, s) : launch<128, 1>(p, s);
}

}  // namespace clef
