// Launch tables of a ragged batch (sequences packed along the token axis by
// cu_seqlens), built on the device by one 256-thread work-group and, from
// the same code, on the host (clef_ragged_plan) for inspection and tests.
//
// The offsets are first made monotone: R[j] = max_{i<=j} clamp(cu[i], 0, T)
// for j = 0..nseq, and sequence s spans [R[s], R[s+1]).  For a valid table
// (non-decreasing offsets in [0, T]) R equals cu.  Any other table still
// yields disjoint spans inside [0, T], so the per-sequence unit counts sum
// to at most ceil(T / unit) + nseq, the capacity the workspaces reserve,
// and every kernel that reads the spans stays inside its buffers.
//
// Each step is a function of the thread index over plain arrays; the
// device kernels run the steps with a barrier between them, the host runs
// each step for all 256 thread indices in turn.
#pragma once
#include <hip/hip_runtime.h>

namespace clef {

constexpr int kTabThreads = 256;
constexpr int kMaxRaggedSeq = 4096;

struct Ragged {
  const int* cu;
  int nseq, T;
  int* part;  // [kTabThreads] per-thread partials
  int* R;     // [nseq + 1] monotone offsets
};

__host__ __device__ inline int rg_clamp(int x, int T) { return x < 0 ? 0 : x > T ? T : x; }
__host__ __device__ inline int rg_min(int a, int b) { return a < b ? a : b; }
__host__ __device__ inline int rg_max(int a, int b) { return a > b ? a : b; }

// Entries [j0, j1) of an array of n entries that thread tid owns.
__host__ __device__ inline void rg_range(int tid, int n, int& j0, int& j1) {
  const int per = (n + kTabThreads - 1) / kTabThreads;
  j0 = rg_min(tid * per, n);
  j1 = rg_min(j0 + per, n);
}

// step 1: the largest clamped offset among the thread's entries of cu
__host__ __device__ inline void rg_spans_1(const Ragged& g, int tid) {
  int j0, j1, m = 0;
  rg_range(tid, g.nseq + 1, j0, j1);
  for (int j = j0; j < j1; ++j) m = rg_max(m, rg_clamp(g.cu[j], g.T));
  g.part[tid] = m;
}
// step 2 (thread 0): exclusive running maximum over the threads
__host__ __device__ inline void rg_spans_2(const Ragged& g, int tid) {
  if (tid != 0) return;
  int run = 0;
  for (int i = 0; i < kTabThreads; ++i) {
    const int v = g.part[i];
    g.part[i] = run;
    run = rg_max(run, v);
  }
}
// step 3: R for the thread's entries
__host__ __device__ inline void rg_spans_3(const Ragged& g, int tid) {
  int j0, j1;
  rg_range(tid, g.nseq + 1, j0, j1);
  int run = g.part[tid];
  for (int j = j0; j < j1; ++j) {
    run = rg_max(run, rg_clamp(g.cu[j], g.T));
    g.R[j] = run;
  }
}

__host__ __device__ inline int rg_units(const Ragged& g, int s, int unit) {
  return (g.R[s + 1] - g.R[s] + unit - 1) / unit;
}

// step 4: units (chunks or query tiles) of the thread's sequences
__host__ __device__ inline void rg_count_4(const Ragged& g, int tid, int unit) {
  int s0, s1, sum = 0;
  rg_range(tid, g.nseq, s0, s1);
  for (int s = s0; s < s1; ++s) sum += rg_units(g, s, unit);
  g.part[tid] = sum;
}
// step 5 (thread 0): exclusive prefix sum over the threads; the total
__host__ __device__ inline void rg_count_5(const Ragged& g, int tid, int* total) {
  if (tid != 0) return;
  int acc = 0;
  for (int i = 0; i < kTabThreads; ++i) {
    const int v = g.part[i];
    g.part[i] = acc;
    acc += v;
  }
  *total = acc;
}

// Scan, step 6: per sequence its chunks' token spans (ctab: first token,
// tokens) and its entry in stab ({sequence, first chunk, chunks, 0}) at its
// rank by chunk count (most first, ties in sequence order).
__host__ __device__ inline void rg_scan_6(const Ragged& g, int tid, int chunk, int* ctab, int* stab) {
  int s0, s1;
  rg_range(tid, g.nseq, s0, s1);
  int first = g.part[tid];
  for (int s = s0; s < s1; ++s) {
    const int nc = rg_units(g, s, chunk);
    int rank = 0;
    for (int j = 0; j < g.nseq; ++j) {
      const int nj = rg_units(g, j, chunk);
      rank += (nj > nc) || (nj == nc && j < s);
    }
    int* e = stab + 4 * rank;
    e[0] = s, e[1] = first, e[2] = nc, e[3] = 0;
    const int t0 = g.R[s], len = g.R[s + 1] - t0;
    for (int c = 0; c < nc; ++c) {
      ctab[2 * (first + c)] = t0 + c * chunk;
      ctab[2 * (first + c) + 1] = rg_min(chunk, len - c * chunk);
    }
    first += nc;
  }
}

// Attention, step 6: (sequence, tile) pairs ranked by key count (most
// first, ties in table order); beyond 8192 tiles in table order.  Query tile
// t of sequence s sees np + min(tile (t + 1), len_s) keys; np is common to
// all tiles, so the order is that of m = min(tile (t + 1), len_s).  A
// sequence's m values are tile, 2 tile, ..., tile (n_s - 1), len_s, rising,
// so how many of them exceed m, and whether one equals m, are closed forms:
// a tile's rank costs one pass over the sequences.
__host__ __device__ inline int rg_tiles_above(int len, int nt, int m, int tile) {
  return len > m ? rg_max(0, nt - m / tile) : 0;
}
__host__ __device__ inline bool rg_tile_at(int len, int m, int tile) {
  return len > 0 && (m == len || (m % tile == 0 && m < len));
}
__host__ __device__ inline void rg_attn_6(const Ragged& g, int tid, int tile, int total, int* pairs) {
  int s0, s1;
  rg_range(tid, g.nseq, s0, s1);
  int f = g.part[tid];
  for (int s = s0; s < s1; ++s) {
    const int len = g.R[s + 1] - g.R[s], nt = rg_units(g, s, tile);
    for (int t = 0; t < nt; ++t) {
      int rank = f + t;
      if (total <= 8192) {
        const int m = rg_min(tile * (t + 1), len);
        rank = 0;
        for (int j = 0; j < g.nseq; ++j) {
          const int lj = g.R[j + 1] - g.R[j];
          rank += rg_tiles_above(lj, (lj + tile - 1) / tile, m, tile) + (j < s && rg_tile_at(lj, m, tile));
        }
      }
      pairs[2 * rank] = s;
      pairs[2 * rank + 1] = t;
    }
    f += nt;
  }
}

}  // namespace clef
