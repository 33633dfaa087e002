/*
 * kvx_oracle.c — CPU restatement of the reference's FP8 KV codec.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the oracle the tests, smoke() and
 * bench.py's CPU baseline compare libkvx against; no product code links or
 * loads it.
 *
 * Follows nanovllm/engine/cpu_prefix_cache.py (xxdydx/KV-Cache-Offloading):
 *   fp8_quantize   :20-24  scale = clamp_min(fp32(amax|x|) / 448, 1e-30) in the
 *                          scale dtype; payload = e4m3fn(clamp(fp32(x) /
 *                          fp32(scale), -448, 448))
 *   fp8_dequantize :27-28  target = bf16(fp32(payload) * fp32(scale))
 * with torch's conversions (torch/headeronly/util/Float8_e4m3fn.h,
 * BFloat16.h) restated from the formats' definitions: round to nearest, ties
 * to even, found by searching the table of representable values rather than
 * by bit manipulation, so it shares no code path with the kernels.
 * Division and multiplication are single IEEE-754 binary32 operations (SSE,
 * no flush-to-zero), as torch's CPU kernels perform them.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f32_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* e4m3fn magnitudes: value of code k (0..126) is (k < 8) ? k * 2^-9 :
 * (1 + (k & 7) / 8) * 2^((k >> 3) - 7). Code 127 (0x7F) is NaN; 480 = the
 * value it would have is the rounding boundary's upper neighbour. */
static double g_e4m3[128];
static int g_init = 0;

static void init_tables(void) {
  if (g_init) return;
  for (int k = 0; k < 128; ++k) {
    int e = k >> 3, m = k & 7;
    g_e4m3[k] = e == 0 ? m * ldexp(1.0, -9) : (1.0 + m / 8.0) * ldexp(1.0, e - 7);
  }
  g_init = 1;
}

/* Nearest e4m3fn code to f, ties to the even code; anything that rounds past
 * 448 (|f| > 464, and exactly 464 rounds to 448) and NaN give 0x7F | sign. */
uint8_t kvx_oracle_e4m3(float f) {
  init_tables();
  const uint8_t sign = (bits_of(f) >> 24) & 0x80;
  if (isnan(f)) return sign | 0x7F;
  const double a = fabs((double)f);
  if (a >= g_e4m3[127]) return sign | 0x7F;
  int lo = 0, hi = 127; /* invariant: g[lo] <= a < g[hi] */
  while (hi - lo > 1) {
    int mid = (lo + hi) / 2;
    if (g_e4m3[mid] <= a) lo = mid; else hi = mid;
  }
  const double dlo = a - g_e4m3[lo], dhi = g_e4m3[hi] - a;
  int k = dlo < dhi ? lo : dhi < dlo ? hi : ((lo & 1) ? hi : lo);
  return sign | (uint8_t)k; /* k == 127 is the NaN code: out of range */
}

float kvx_oracle_e4m3_decode(uint8_t c) {
  init_tables();
  const int k = c & 0x7F;
  if (k == 0x7F) return f32_of(((uint32_t)(c & 0x80) << 24) | 0x7FC00000u);
  const float v = (float)g_e4m3[k];
  return (c & 0x80) ? -v : v;
}

/* Nearest bf16 (8-bit significand) to f, ties to even; NaN -> 0x7FC0. */
uint16_t kvx_oracle_bf16(float f) {
  if (isnan(f)) return 0x7FC0;
  const uint32_t u = bits_of(f);
  const uint32_t sign = u & 0x80000000u;
  const uint32_t mag = u & 0x7FFFFFFFu;
  const uint32_t down = mag & 0xFFFF0000u; /* truncation toward zero */
  if (down == mag) return (uint16_t)((sign | down) >> 16);
  const uint32_t up = down + 0x10000u; /* next bf16 magnitude (0x7F800000 = inf) */
  const double a = (double)f32_of(mag), d = (double)f32_of(down);
  const double upv = up == 0x7F800000u ? ldexp(1.0, 128) : (double)f32_of(up);
  const double dd = a - d, du = upv - a;
  uint32_t r = dd < du ? down : du < dd ? up : (((down >> 16) & 1) ? up : down);
  return (uint16_t)((sign | r) >> 16);
}

static float bf16_value(uint16_t h) { return f32_of((uint32_t)h << 16); }

void kvx_oracle_e4m3_range(uint32_t first, uint32_t count, uint8_t* out) {
  init_tables();
  for (int64_t i = 0; i < (int64_t)count; ++i) out[i] = kvx_oracle_e4m3(f32_of(first + (uint32_t)i));
}

void kvx_oracle_bf16_range(uint32_t first, uint32_t count, uint16_t* out) {
  for (int64_t i = 0; i < (int64_t)count; ++i) out[i] = kvx_oracle_bf16(f32_of(first + (uint32_t)i));
}

/* cpu_prefix_cache.py:20-24 over `rows` rows of `hd` bf16 values (bit patterns). */
void kvx_oracle_quantize(const uint16_t* x, int64_t rows, int32_t hd, int32_t scale_fp32, uint8_t* codes,
                         void* scales) {
  init_tables();
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* row = x + r * hd;
    /* source.abs().amax(-1): NaN anywhere gives NaN. */
    float amax = 0.0f;
    int nan = 0;
    for (int32_t i = 0; i < hd; ++i) {
      const float a = fabsf(bf16_value(row[i]));
      if (isnan(a)) nan = 1;
      else if (a > amax) amax = a;
    }
    float s = (nan ? NAN : amax) / 448.0f; /* .float() / _FP8_MAX */
    if (s < 1e-30f) s = 1e-30f;            /* .clamp_min(1e-30); NaN passes */
    float used;
    if (scale_fp32) {
      ((float*)scales)[r] = s;
      used = s;
    } else {
      const uint16_t b = kvx_oracle_bf16(s); /* scale.copy_ into bf16 */
      ((uint16_t*)scales)[r] = b;
      used = bf16_value(b);
    }
    for (int32_t i = 0; i < hd; ++i) {
      float q = bf16_value(row[i]) / used; /* source.float() / scale.float() */
      if (q < -448.0f) q = -448.0f;        /* .clamp_(-448, 448); NaN passes */
      else if (q > 448.0f) q = 448.0f;
      codes[r * hd + i] = kvx_oracle_e4m3(q);
    }
  }
}

/* cpu_prefix_cache.py:27-28: torch.mul(payload.to(bf16), scale, out=bf16 target). */
void kvx_oracle_dequantize(const uint8_t* codes, const void* scales, int64_t rows, int32_t hd, int32_t scale_fp32,
                           uint16_t* out) {
  init_tables();
  for (int64_t r = 0; r < rows; ++r) {
    const float s = scale_fp32 ? ((const float*)scales)[r] : bf16_value(((const uint16_t*)scales)[r]);
    for (int32_t i = 0; i < hd; ++i) out[r * hd + i] = kvx_oracle_bf16(kvx_oracle_e4m3_decode(codes[r * hd + i]) * s);
  }
}

/*
 * The kernels divide by a row scale s as q0 = a*y, r = fma(-q0, s, a),
 * q = fma(r, y, q0) with y = RN(1/s). Away from overflow and underflow each
 * step scales exactly with the exponents of a and s, so the quotient is exact
 * for all inputs iff it is exact for every pair of significands. Counts the
 * pairs (bf16 significand of a) x (fp32 significand of s) where it differs
 * from IEEE division, for fp32 significands [first, first + count) of the
 * 2^23; 0 over all of them proves the method for the kernels' scale range.
 * Single-threaded: callers split the range across threads (ctypes releases
 * the GIL), which keeps a second OpenMP runtime out of the torch process.
 */
int64_t kvx_oracle_fastdiv_mismatches(uint32_t first, uint32_t count) {
  int64_t bad = 0;
  for (int64_t mb = first; mb < (int64_t)first + count && mb < (1 << 23); ++mb) {
    const float s = f32_of(0x3F800000u | (uint32_t)mb);
    volatile float one = 1.0f;
    const float y = one / s;
    for (uint32_t ma = 0; ma < 128; ++ma) {
      const float a = f32_of(0x3F800000u | (ma << 16));
      const float q0 = a * y;
      const float r = fmaf(-q0, s, a);
      const float q = fmaf(r, y, q0);
      bad += bits_of(q) != bits_of(a / s);
    }
  }
  return bad;
}
