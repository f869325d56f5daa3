// schedule.h - tile/phase schedule of the dual-window attention kernels.
//
// Shared verbatim by the gfx950 kernels (attn.hip) and by the host-side
// replay ttcd_attn_schedule_coverage (api.hip), so the CPU test suite proves
// the exact iteration logic the GPU runs: every (query, key) pair inside a
// window is folded into that window's output exactly once.
//
// Geometry. A workgroup has 4 wavefronts; each wavefront owns R consecutive
// query rows (r0..r0+R-1), R = Schedule::rows: 32 rows of one query head, or,
// for an even GQA group, 16 rows of each of two query heads of the group (the
// 32 columns of one score MFMA; both heads read the same K/V, so every MFMA
// operand is shared). A workgroup owns 4R tokens. Keys are swept in tiles of
// kBlockN = 64, tile n covering keys [64n - kshift, 64n - kshift + 63], from
// the tile holding the workgroup's last diagonal downward (the same
// backward-from-diagonal order as profiling/fused_dual_attn.py:91,119,151,
// 176,191); every wave of the workgroup steps through the same tiles.
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
// are student-visible for some of its rows and far for others: the R-1 keys
// [r0-ws+1, r0+R-1-ws]) to sit in one tile, so that all phase-1 tiles of a
// wave precede all of its phase-2-only tiles. With r0 a multiple of R this
// holds iff tile starts are congruent to (1 - ws) or (-ws) modulo R, so
// kshift = ws mod 32 serves both geometries (0 for single-band calls). It
// also makes the waves of each aligned 64-row run share their mixed tile:
// one repeated tile per 16-row-wave workgroup (two for 32-row waves) when
// ws mod 64 < 32. The tile boundaries, and with them every row's order of
// accumulation, are the same in both geometries.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define TTCD_HD __host__ __device__ __forceinline__
#else
#define TTCD_HD inline
#endif

namespace ttcd {

constexpr int kBlockN = 64;    // keys per K/V tile
constexpr int kWaveRows = 32;  // query columns per wavefront (score MFMA columns)
constexpr int kWaves = 4;      // wavefronts per workgroup
constexpr int kBlockM = kWaveRows * kWaves;  // query tokens per workgroup, one head per wave

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
  int rows;    // query rows (tokens) per wavefront: 32, or 16 of each of two heads

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

// Does tile [j0, j0+63] hold a key of band b for some row of the wave r0..r0+R-1?
TTCD_HD bool wave_touches(int r0, int R, Band b, int j0) {
  return b.lo < b.hi && j0 + kBlockN - 1 >= r0 - b.hi + 1 && j0 <= r0 + R - 1 - b.lo;
}

// Is every (row, key) pair of the tile inside band b (no mask needed)?
TTCD_HD bool wave_full(int r0, int R, Band b, int j0) {
  return j0 >= 0 && r0 - (j0 + kBlockN - 1) >= b.lo && r0 + R - 1 - j0 < b.hi;
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

// Slots. A workgroup sweeps a sequence of slots, one tile per slot. For the
// dual kernel each distinct "mixed" tile of its waves (a tile holding both
// student and far keys of a wave, at most one per wave) appears twice in a
// row: in the first slot its waves fold the student keys and then write the
// student output; in the repeated slot they fold the far keys. Waves whose
// mixed tile it is not skip the repeated slot. Every wave therefore carries
// one accumulator and one pending P^T between phases, as in the band kernel.
constexpr int kMaxDup = kWaves;
constexpr int kNoTile = -0x7fffffff - 1;

// All loops below have compile-time trip counts and static indices, so on the
// GPU the plan lives in scalar registers (no scratch memory).
struct SlotPlan {
  int n_hi;            // first (highest) tile
  int count;           // tiles n_hi .. n_hi - count + 1
  int ndup;            // repeated (mixed) tiles
  int dup[kMaxDup];    // their tile indices, descending; kNoTile for unused entries

  TTCD_HD int slots() const { return count + ndup; }

  // Tile of slot k and whether it is a repeat.
  TTCD_HD int tile(int k, bool* repeat) const {
    int n = n_hi - k;
    int before = 0;       // repeats already placed
    int rep_tile = kNoTile;
#pragma unroll
    for (int i = 0; i < kMaxDup; ++i) {
      if (dup[i] != kNoTile) {
        const int first = n_hi - dup[i] + before;  // slot of dup[i]'s first pass
        if (k == first + 1) rep_tile = dup[i];
        if (k > first + 1) n += 1;
        before += 1;
      }
    }
    *repeat = rep_tile != kNoTile;
    return *repeat ? rep_tile : n;
  }
};

// The wave's mixed tile, or kNoTile when it has none.
TTCD_HD int wave_mixed_tile(const Schedule& sc, int r0) {
  if (!sc.dual) return kNoTile;
  int lowest = r0 - sc.p1.hi + 1;  // lowest student key of the wave
  if (lowest < 0) lowest = 0;
  const int n = sc.tile_of(lowest);
  const int j0 = sc.tile_start(n);
  return (wave_touches(r0, sc.rows, sc.p1, j0) && wave_touches(r0, sc.rows, sc.p2, j0)) ? n
                                                                                   : kNoTile;
}

// Slot plan of a workgroup whose wave w starts at row r0_of_wave(w) (rows >= T
// are idle waves) and whose tiles are n_hi down to n_lo.
template <typename R0>
TTCD_HD SlotPlan make_slot_plan(const Schedule& sc, R0 r0_of_wave, int n_hi, int n_lo) {
  SlotPlan sp;
  sp.n_hi = n_hi;
  sp.count = n_hi - n_lo + 1;
  int* d = sp.dup;
#pragma unroll
  for (int w = 0; w < kMaxDup; ++w) {
    const int r0 = r0_of_wave(w);
    const int n = r0 < sc.T ? wave_mixed_tile(sc, r0) : kNoTile;
    d[w] = (n >= n_lo && n <= n_hi) ? n : kNoTile;
  }
  // sort descending (kNoTile is the smallest int), blank out repeats, then
  // sort again so the distinct tiles lead the array
  auto sort_desc = [](int* v) {
#pragma unroll
    for (int a = 0; a < kMaxDup; ++a)
#pragma unroll
      for (int b = 0; b + 1 < kMaxDup - a; ++b)
        if (v[b] < v[b + 1]) {
          const int t = v[b];
          v[b] = v[b + 1];
          v[b + 1] = t;
        }
  };
  sort_desc(d);
  sp.ndup = 0;
  int prev = kNoTile;
#pragma unroll
  for (int i = 0; i < kMaxDup; ++i) {
    const int v = d[i];
    d[i] = (v == prev) ? kNoTile : v;
    prev = v;
    sp.ndup += d[i] != kNoTile;
  }
  sort_desc(d);
  return sp;
}

// What a wave folds in a slot: nothing, one band (mask chosen by wave_full),
// the student part of its mixed tile (then writes the student output) or the
// far part (repeat slot).
enum SlotAction { kSkip = 0, kBand1 = 1, kBand2 = 2, kStudentLast = 3, kFar = 4 };

TTCD_HD int slot_action(const Schedule& sc, int r0, int j0, bool repeat) {
  const bool in1 = wave_touches(r0, sc.rows, sc.p1, j0);
  const bool in2 = sc.dual && wave_touches(r0, sc.rows, sc.p2, j0);
  if (repeat) return (in1 && in2) ? kFar : kSkip;
  if (in1 && (in2 || (sc.dual && wave_last(r0, sc.p1, j0)))) return kStudentLast;
  return in1 ? kBand1 : (in2 ? kBand2 : kSkip);
}

// Per-wave slot actions in closed form: the tile-index ranges behind
// slot_action() and wave_full(), computed once per wave so that each slot
// costs a few branch-free scalar compares. Must agree with those functions
// on every tile of the sweep (checked by ttcd_attn_schedule_coverage).
struct WaveSlots {
  int n1a, n1b;  // tiles touched by phase 1 (empty: n1a > n1b)
  int n2a, n2b;  // tiles touched by phase 2 (dual kernel)
  int nl;        // tiles n <= nl end the student phase (wave_last)
  int f1a, f1b;  // tiles fully inside band 1
  int f2a, f2b;  // tiles fully inside band 2
  int dual;

  TTCD_HD WaveSlots(const Schedule& sc, int r0) : dual(sc.dual) {
    const int big = 0x3fffffff;
    auto range = [&](Band b, int* a, int* z) {
      if (b.lo < b.hi) {
        *a = sc.tile_of(r0 - b.hi + 1);
        *z = sc.tile_of(r0 + sc.rows - 1 - b.lo);
      } else {
        *a = big;
        *z = -big;
      }
    };
    range(sc.p1, &n1a, &n1b);
    if (sc.dual) {
      range(sc.p2, &n2a, &n2b);
    } else {
      n2a = big;
      n2b = -big;
    }
    const int lowest = r0 - sc.p1.hi + 1;
    nl = sc.tile_of(lowest > 0 ? lowest : 0);
    const int nz = sc.kshift > 0 ? 1 : 0;  // first tile with j0 >= 0
    auto full = [&](Band b, int* a, int* z) {
      const int lo_t = sc.tile_of(r0 + sc.rows + kBlockN - 1 - b.hi);  // j0 > r0 + R-1 - hi
      *a = lo_t > nz ? lo_t : nz;
      *z = sc.tile_of(r0 - (kBlockN - 1) - b.lo);                      // j0 <= r0 - 63 - lo
    };
    full(sc.p1, &f1a, &f1b);
    full(sc.p2, &f2a, &f2b);
  }

  // slot_action(sc, r0, tile_start(n), repeat), branch-free.
  TTCD_HD int act(int n, bool repeat) const {
    const bool in1 = (n >= n1a) & (n <= n1b);
    const bool in2 = (n >= n2a) & (n <= n2b);
    const int normal = in1 ? ((in2 | ((dual != 0) & (n <= nl))) ? kStudentLast : kBand1)
                           : (in2 ? kBand2 : kSkip);
    return repeat ? ((in1 & in2) ? kFar : kSkip) : normal;
  }
  // !wave_full(r0, band of action a, tile_start(n)) for an action that is not kSkip.
  TTCD_HD bool mask(int n, int a) const {
    const bool far = (a == kBand2) | (a == kFar);
    const int fa = far ? f2a : f1a, fz = far ? f2b : f1b;
    return !((n >= fa) & (n <= fz));
  }
};

// Slot words: everything the slot loop needs about slot k for one wave, in
// one 32-bit word. The kernel computes 64 consecutive slots at once (slot
// base + lane in each lane) and reads one word per slot back with
// v_readlane, so a slot costs a few scalar bit tests instead of evaluating
// the plan, the actions and the load bounds. Bits 0-5 are flags; bits 6+
// hold the tile index, so (word & ~63) is the tile's first key + kshift.
enum SlotWordBits : uint32_t {
  kWordLoad = 1u,      // slot exists: its K and V tiles are loaded
  kWordInterior = 2u,  // tile keys all inside [0, T): unclamped loads
  kWordActive = 4u,    // this wave folds keys (action != kSkip)
  kWordFar = 8u,       // ... of phase 2 (kBand2 or kFar), else of phase 1
  kWordLast = 16u,     // ... and it is kStudentLast (student output follows)
  kWordMask = 32u,     // ... and the scores need masking
};
constexpr int kWordTileShift = 6;
static_assert((1 << kWordTileShift) == kBlockN, "word & ~63 is the tile's key offset");

// Word of slot k of plan sp (nslot slots) for the wave described by ws
// (wave_valid false: a wave without rows, which only loads), keys [0, T).
TTCD_HD uint32_t slot_word(const Schedule& sc, const SlotPlan& sp, const WaveSlots& ws,
                           int nslot, bool wave_valid, int T, int k) {
  bool repeat;
  int n = sp.tile(k, &repeat);
  const bool load = (k >= 0) & (k < nslot);
  n = load ? n : 0;
  const int j0 = sc.tile_start(n);
  const int act = (load & wave_valid) ? ws.act(n, repeat) : (int)kSkip;
  const bool far = (act == kBand2) | (act == kFar);
  uint32_t w = (uint32_t)n << kWordTileShift;
  w |= load ? kWordLoad : 0u;
  w |= (load & (j0 >= 0) & (j0 + kBlockN <= T)) ? kWordInterior : 0u;
  w |= act != kSkip ? kWordActive : 0u;
  w |= far ? kWordFar : 0u;
  w |= act == kStudentLast ? kWordLast : 0u;
  w |= (act != kSkip && ws.mask(n, act)) ? kWordMask : 0u;
  return w;
}

TTCD_HD int word_tile(uint32_t w) { return (int)(w >> kWordTileShift); }
TTCD_HD int word_j0(const Schedule& sc, uint32_t w) { return (int)(w & ~63u) - sc.kshift; }
TTCD_HD Band word_band(const Schedule& sc, uint32_t w) { return (w & kWordFar) ? sc.p2 : sc.p1; }

// Query rows per wavefront for a GQA group size (see Geometry): 16 rows of
// each of two heads for an even group, else 32 rows of one head.
#ifndef TTCD_PAIR_WAVES
#define TTCD_PAIR_WAVES 1
#endif
TTCD_HD int wave_rows(int gqa_group) {
  return (TTCD_PAIR_WAVES && gqa_group % 2 == 0) ? kWaveRows / 2 : kWaveRows;
}

// Query tokens swept by one workgroup.
TTCD_HD int wg_span_tokens(int gqa_group) { return kWaves * wave_rows(gqa_group); }

// Schedules built by the C ABI entry points (windows already validated), for
// wavefronts of `rows` query rows.
TTCD_HD Schedule make_dual_schedule(int T, int ws, int wt, int rows) {
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
  s.rows = rows;
  return s;
}

TTCD_HD Schedule make_band_schedule(int T, int lo, int hi, int rows) {
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
  s.rows = rows;
  return s;
}

}  // namespace ttcd
