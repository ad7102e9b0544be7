/*
 * fp8_quant.c -- C restatement of the reference's vblock32 checkpoint
 * quantiser, in integer arithmetic on IEEE-754 bit patterns.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): built by
 * oracle/build_oracle.py into oracle/_build/liboracle_fp8.so and loaded by
 * oracle/fp8_quant.py from tests/, smoke() and bench.py's cpu_baseline.
 *
 * Restates prototype/gdn_replay_fp8_reference.py:36-37 (_safe_scale) and
 * :40-106 (quantize_checkpoint, vblock branch :71-87 and :91-99):
 *   amax  = max |x| over a 32 x K block (NaN propagates),
 *   s32   = amax / 448 if amax > 0 else 1        (IEEE fp32 divide),
 *   scale = fp16(s32)                              (stored, round-nearest-even),
 *   code  = e4m3fn(clamp(x / s32, -448, 448))      (divide by the UNROUNDED s32),
 * and :109-134 (dequantize_checkpoint): x = float(code) * float(scale).
 * The conversions are written from the IEEE-754 / OCP-FP8 definitions, not
 * from any library; tests pin them against torch's CPU casts.
 *
 * Must be compiled without fast-math and with -ffp-contract=off so every
 * float operation is a single correctly rounded IEEE operation.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* Round-to-nearest-even right shift of a non-negative integer. */
static uint64_t rne_shift(uint64_t value, int shift) {
  if (shift <= 0) return value << (-shift);
  if (shift >= 64) return 0;
  uint64_t kept = value >> shift;
  uint64_t rem = value & ((UINT64_C(1) << shift) - 1);
  uint64_t half = UINT64_C(1) << (shift - 1);
  if (rem > half || (rem == half && (kept & 1))) kept += 1;
  return kept;
}

/* fp32 -> OCP e4m3fn code, round-to-nearest-even. Like torch's cast:
 * |x| > 464, inf and NaN give 0x7F | sign. */
uint8_t oracle_e4m3fn_encode(float x) {
  uint32_t u = f32_bits(x);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  uint32_t exp32 = (u >> 23) & 0xFF;
  uint32_t man32 = u & 0x7FFFFF;
  if (exp32 == 0xFF) return (uint8_t)(sign | 0x7F);           /* inf, NaN */
  if (exp32 == 0) return sign;                                  /* fp32 subnormal: < 2^-126 */
  uint64_t significand = (UINT64_C(1) << 23) | man32;           /* value = sig * 2^(exp32-150) */
  int e8 = (int)exp32 - 127 + 7;
  uint32_t code;
  if (e8 >= 1) {
    uint64_t m = rne_shift(significand, 20);                    /* 4-bit significand 8..16 */
    if (m == 16) { m = 8; e8 += 1; }
    if (e8 > 15 || (e8 == 15 && (m - 8) == 7)) return (uint8_t)(sign | 0x7F);
    code = ((uint32_t)e8 << 3) | (uint32_t)(m - 8);
  } else {
    /* subnormal e4m3fn: units of 2^-9; sig * 2^(exp32-150) / 2^-9 = sig * 2^(exp32-141) */
    int shift = 141 - (int)exp32;
    code = (uint32_t)rne_shift(significand, shift);             /* 0..8; 8 == min normal 0x08 */
  }
  return (uint8_t)(sign | code);
}

float oracle_e4m3fn_decode(uint8_t code) {
  int sign = code & 0x80;
  int exponent = (code >> 3) & 0xF;
  int mantissa = code & 0x7;
  float value;
  if (exponent == 0xF && mantissa == 0x7) return bits_f32(sign ? 0xFFC00000u : 0x7FC00000u);
  if (exponent == 0) value = ldexpf((float)mantissa, -9);
  else value = ldexpf((float)(8 + mantissa), exponent - 10);
  return sign ? -value : value;
}

/* fp32 -> IEEE binary16 bits, round-to-nearest-even, subnormals kept. */
uint16_t oracle_f16_bits(float x) {
  uint32_t u = f32_bits(x);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  uint32_t exp32 = (u >> 23) & 0xFF;
  uint32_t man32 = u & 0x7FFFFF;
  if (exp32 == 0xFF) return (uint16_t)(sign | 0x7C00 | (man32 ? 0x200 | (man32 >> 13) : 0));
  if (exp32 == 0) return sign;                                  /* < 2^-126: rounds to 0 */
  uint64_t significand = (UINT64_C(1) << 23) | man32;
  int e16 = (int)exp32 - 127 + 15;
  if (e16 >= 1) {
    uint64_t m = rne_shift(significand, 13);                    /* 11-bit significand */
    if (m == 2048) { m = 1024; e16 += 1; }
    if (e16 >= 31) return (uint16_t)(sign | 0x7C00);            /* overflow -> inf */
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | (uint32_t)(m - 1024));
  }
  /* subnormal binary16: units of 2^-24; sig * 2^(exp32-150) / 2^-24 = sig * 2^(exp32-126) */
  int shift = 126 - (int)exp32;
  uint32_t m = (uint32_t)rne_shift(significand, shift);         /* 0..1024; 1024 == min normal */
  return (uint16_t)(sign | m);
}

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t e = (h >> 10) & 0x1F;
  uint32_t m = h & 0x3FF;
  if (e == 0x1F) return bits_f32(sign | 0x7F800000u | (m << 13));
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

void oracle_e4m3fn_encode_array(const float* x, int64_t n, uint8_t* codes) {
  for (int64_t i = 0; i < n; ++i) codes[i] = oracle_e4m3fn_encode(x[i]);
}

void oracle_f16_bits_array(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_bits(x[i]);
}

/* Quantise n_blocks contiguous blocks of block_elems floats (a vblock32 of a
 * [.., V, K] state is 32*K contiguous floats). saturated may be NULL. */
void oracle_quantize_blocks(const float* state, int64_t n_blocks, int64_t block_elems,
                            uint8_t* codes, uint16_t* scale_bits, int32_t* saturated) {
  for (int64_t blk = 0; blk < n_blocks; ++blk) {
    const float* x = state + blk * block_elems;
    uint8_t* c = codes + blk * block_elems;
    uint32_t amax_bits = 0;                       /* max over |x| bit patterns: NaN wins */
    for (int64_t i = 0; i < block_elems; ++i) {
      uint32_t a = f32_bits(x[i]) & 0x7FFFFFFFu;
      if (a > amax_bits) amax_bits = a;
    }
    float amax = bits_f32(amax_bits);
    float s32 = (amax > 0.0f) ? amax / 448.0f : 1.0f;   /* NaN amax compares false -> 1 */
    scale_bits[blk] = oracle_f16_bits(s32);
    int32_t sat = 0;
    for (int64_t i = 0; i < block_elems; ++i) {
      float n = x[i] / s32;
      if (fabsf(n) > 448.0f) sat += 1;
      if (!isnan(n)) n = n > 448.0f ? 448.0f : (n < -448.0f ? -448.0f : n);
      c[i] = oracle_e4m3fn_encode(n);
    }
    if (saturated) saturated[blk] = sat;
  }
}

void oracle_dequantize_blocks(const uint8_t* codes, const uint16_t* scale_bits, int64_t n_blocks,
                              int64_t block_elems, float* state) {
  for (int64_t blk = 0; blk < n_blocks; ++blk) {
    float s = oracle_f16_to_f32(scale_bits[blk]);
    for (int64_t i = 0; i < block_elems; ++i)
      state[blk * block_elems + i] = oracle_e4m3fn_decode(codes[blk * block_elems + i]) * s;
  }
}
