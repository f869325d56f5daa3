// schedule.h - tile/phase schedule of the dual-window attention kernels.
//
// Shared verbatim by the gfx950 kernels (attn.hip) and by the host-side
// replay ttcd_attn_schedule_coverage (api.hip), so the CPU test suite proves
// the exact iteration logic the GPU runs: every (query, key) pair inside a
// window is folded into that window's output exactly once.
//
// Geometry. A workgroup owns kBlockM = 128 consecutive query tokens of one
// query head; each of its 4 wavefronts owns 32 of them (rows r0..r0+31).
// Keys are swept in tiles of kBlockN = 64, tile n covering keys
// [64n - kshift, 64n - kshift + 63], from the tile holding the workgroup's
// diagonal downward (the same backward-from-diagonal order as
// profiling/fused_dual_attn.py:91,119,151,176,191).
//
// Phases. A band {lo, hi} selects keys with lo <= i - j < hi. The dual kernel
// runs phase 1 = student band {0, ws} and then phase 2 = far band {ws, wt}
// on ONE online-softmax accumulator: when a wave finishes phase 1 it writes
// the student output from the accumulator and keeps going, so the teacher
// output is the same accumulator after phase 2. This replaces the two
// accumulators of the reference kernel (fused_dual_attn.py:68-73) and its
// five segments A-E (:90-232) with a schedule that never needs a second
// output accumulator in registers.
//
// The single-accumulator order needs every wave's "mixed" keys (keys that
// are student-visible for some of its rows and far for others: the 31 keys
// [r0-ws+1, r0+31-ws]) to sit in one tile, so that all phase-1 tiles of a
// wave precede all of its phase-2-only tiles. With r0 a multiple of 32 this
// holds iff tile starts are congruent to (1 - ws) or (-ws) modulo 32, hence
// kshift = ws mod 32 for the dual kernel (0 for single-band calls).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define TTCD_HD __host__ __device__ __forceinline__
#else
#define TTCD_HD inline
#endif

namespace ttcd {

constexpr int kBlockN = 64;    // keys per K/V tile
constexpr int kWaveRows = 32;  // query rows per wavefront
constexpr int kWaves = 4;      // wavefronts per workgroup
constexpr int kBlockM = kWaveRows * kWaves;  // query tokens per workgroup

struct Band {
  int lo;  // inclusive lower bound of i - j
  int hi;  // exclusive upper bound of i - j
};

// Floor division for b > 0 and any a (C++ '/' truncates toward zero).
TTCD_HD int floordiv(int a, int b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

struct Schedule {
  int T;       // sequence length (queries == keys)
  int dual;    // 1: phase 1 = student, phase 2 = far band; 0: phase 1 only
  Band p1;     // phase-1 band
  Band p2;     // phase-2 band (dual only; empty when lo == hi)
  int kshift;  // tile n starts at key 64n - kshift

  TTCD_HD int tile_of(int j) const { return floordiv(j + kshift, kBlockN); }
  TTCD_HD int tile_start(int n) const { return n * kBlockN - kshift; }

  // Tile range [n_lo, n_hi] swept by the workgroup owning tokens t0..t_last.
  // Returns false when no row of the workgroup has a key in any band.
  TTCD_HD bool wg_range(int t0, int t_last, int* n_hi, int* n_lo) const {
    const int top = t_last - p1.lo;  // phase 1 always has the smallest lo
    const int widest = (dual && p2.lo < p2.hi) ? p2.hi : p1.hi;
    int bottom = t0 - widest + 1;
    if (bottom < 0) bottom = 0;
    if (top < 0 || top < bottom) return false;
    *n_hi = tile_of(top);
    *n_lo = tile_of(bottom);
    return true;
  }
};

// Does tile [j0, j0+63] hold a key of band b for some row of the wave r0..r0+31?
TTCD_HD bool wave_touches(int r0, Band b, int j0) {
  return b.lo < b.hi && j0 + kBlockN - 1 >= r0 - b.hi + 1 &&
         j0 <= r0 + kWaveRows - 1 - b.lo;
}

// Is every (row, key) pair of the tile inside band b (no mask needed)?
TTCD_HD bool wave_full(int r0, Band b, int j0) {
  return j0 >= 0 && r0 - (j0 + kBlockN - 1) >= b.lo &&
         r0 + kWaveRows - 1 - j0 < b.hi;
}

// Is this the wave's last tile of band b in the backward sweep?
TTCD_HD bool wave_last(int r0, Band b, int j0) {
  return j0 <= r0 - b.hi + 1 || j0 <= 0;
}

// Per-element visibility used by masked tiles.
TTCD_HD bool visible(int i, int j, Band b, int T) {
  const int d = i - j;
  return d >= b.lo && d < b.hi && j >= 0 && j < T;
}

// Schedules built by the C ABI entry points (windows already validated).
TTCD_HD Schedule make_dual_schedule(int T, int ws, int wt) {
  if (wt > T) wt = T;
  if (ws > wt) ws = wt;
  Schedule s;
  s.T = T;
  s.dual = 1;
  s.p1.lo = 0;
  s.p1.hi = ws;
  s.p2.lo = ws;
  s.p2.hi = wt;
  s.kshift = ws % kWaveRows;
  return s;
}

TTCD_HD Schedule make_band_schedule(int T, int lo, int hi) {
  if (hi > T) hi = T;
  if (lo > hi) lo = hi;
  Schedule s;
  s.T = T;
  s.dual = 0;
  s.p1.lo = lo;
  s.p1.hi = hi;
  s.p2.lo = hi;
  s.p2.hi = hi;
  s.kshift = 0;
  return s;
}

}  // namespace ttcd
