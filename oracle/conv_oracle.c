/*
 * conv_oracle.c - CPU restatement of the chunked causal depthwise conv.
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never by the product path.
 *
 * Follows profiling/fused_conv.py:39-48 (kernel body) and :56-58 (x made
 * contiguous, w = conv.weight.view(D, K)), with the semantics of
 * IPTTCDMLP._apply_ttt_conv (custom_models/ipttcd/modeling_ipttcdv9.py:203-211:
 * per-chunk left zero padding of K-1, depthwise, no bias):
 *   acc = +0.0f
 *   for j in 0..K-1: acc = fmaf(f32(x[n, c-(K-1)+j, d]) (0 if index < 0), f32(w[d, j]), acc)
 *   y[n, c, d] = round_to_nearest_even(acc) in x's dtype
 * fmaf is correctly rounded (one rounding per tap), so for bf16/f16 inputs,
 * whose products are exact in fp32, this equals mul-then-add as well.
 * dtype codes: 0 = bf16, 1 = f16, 2 = f32 (raw bit patterns in memory).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = h >> 15, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0)
    v = ldexpf((float)m, -24);
  else if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = ldexpf((float)(m | 0x400u), (int)e - 25);
  return sign ? -v : v;
}

static uint16_t f32_to_f16_rne(float f) {
  const uint32_t u = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;  /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
  if (a >= 0x38800000u) {                      /* normal half (>= 2^-14) */
    const uint32_t mant = a & 0x7fffffu;
    uint32_t r = ((uint32_t)((int)(a >> 23) - 127 + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  /* subnormal half: round a / 2^-24 to the nearest even integer */
  const float scaled = bits_to_f32(a) * 16777216.0f;
  return (uint16_t)(sign | (uint32_t)nearbyintf(scaled));
}

static float load(const void* p, int dt, int64_t i) {
  switch (dt) {
    case 0: return bf16_to_f32(((const uint16_t*)p)[i]);
    case 1: return f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static void store(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case 0: ((uint16_t*)p)[i] = f32_to_bf16_rne(v); break;
    case 1: ((uint16_t*)p)[i] = f32_to_f16_rne(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

/* Element-wise dtype round trip, exported so tests can pin the encoders. */
void ttcd_oracle_round(const float* src, void* dst, int dt, int64_t n) {
  for (int64_t i = 0; i < n; ++i) store(dst, dt, i, src[i]);
}

void ttcd_oracle_dwconv(const void* x, int x_dt, const void* w, int w_dt, void* y, int64_t N,
                        int C, int D, int K) {
  for (int64_t n = 0; n < N; ++n) {
    const int64_t base = n * (int64_t)C * D;
    for (int c = 0; c < C; ++c) {
      for (int d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < K; ++j) {
          const int src = c - (K - 1) + j;
          const float xv = src >= 0 ? load(x, x_dt, base + (int64_t)src * D + d) : 0.0f;
          acc = fmaf(xv, load(w, w_dt, (int64_t)d * K + j), acc);
        }
        store(y, x_dt, base + (int64_t)c * D + d, acc);
      }
    }
  }
}
