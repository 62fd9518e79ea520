/*
 * CPU oracle: plain-C restatement of the reference's quantized-weight matmul path.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the product library.
 * Citations are file:line in the dotstories/web-engine tree.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------ */
/* Decoders                                                                                         */
/* ------------------------------------------------------------------------------------------------ */

/* src/weights/fp8.ts:4-11 — float8_e4m3fn: bias 7, no infinity, 0x7f/0xff NaN, max 448. */
double or_e4m3(uint8_t b) {
  const double sign = (b & 0x80) ? -1.0 : 1.0;
  const int exp = (b >> 3) & 0xf;
  const int man = b & 0x7;
  if (exp == 0xf && man == 0x7) return NAN;
  if (exp == 0) return sign * (man / 8.0) * ldexp(1.0, -6);
  return sign * (1.0 + man / 8.0) * ldexp(1.0, exp - 7);
}

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

/* src/kernels/fp8.ts:12-20 — the shader decoder: rebias the exponent (7 -> 127), subnormals as
 * m * 2^-9, sign applied last. It has no NaN branch, so 0x7f / 0xff decode to +-480. */
float or_e4m3_gpu(uint8_t b) {
  const uint32_t e = (b >> 3) & 0xfu;
  const uint32_t m = b & 7u;
  const float normal = bits_to_f32(((e + 120u) << 23) | (m << 20));
  const float subnormal = (float)m * 0.001953125f;
  const float v = e == 0u ? subnormal : normal;
  return (b & 0x80u) ? -v : v;
}

/* src/weights/fp8.ts:14-21 — float8_e5m2: bias 15, IEEE infinity and NaN. */
double or_e5m2(uint8_t b) {
  const double sign = (b & 0x80) ? -1.0 : 1.0;
  const int exp = (b >> 2) & 0x1f;
  const int man = b & 0x3;
  if (exp == 0x1f) return man ? NAN : sign * INFINITY;
  if (exp == 0) return sign * (man / 4.0) * ldexp(1.0, -14);
  return sign * (1.0 + man / 4.0) * ldexp(1.0, exp - 15);
}

/* src/weights/fp8.ts:23-30 — IEEE half. */
double or_f16(uint16_t h) {
  const double sign = (h & 0x8000) ? -1.0 : 1.0;
  const int exp = (h >> 10) & 0x1f;
  const int man = h & 0x3ff;
  if (exp == 0x1f) return man ? NAN : sign * INFINITY;
  if (exp == 0) return sign * (man / 1024.0) * ldexp(1.0, -14);
  return sign * (1.0 + man / 1024.0) * ldexp(1.0, exp - 15);
}

/* src/weights/fp8.ts:43-44 — bf16 is the top half of an f32 (w << 16). */
float or_bf16(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* f32 -> bf16, round to nearest even. Used to build bf16 inputs; the reference builds its bf16 test
 * weights by truncation (tests/gpu/matmul.test.ts:121), which callers can do with a shift. */
uint16_t or_f32_to_bf16(float v) {
  uint32_t u = f32_to_bits(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* f32 -> IEEE half, round to nearest even, overflow to infinity, gradual underflow. */
uint16_t or_f32_to_f16(float v) {
  const uint32_t u = f32_to_bits(v);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                 /* below 2^-14: subnormal half */
    /* value = a_float; half subnormal unit = 2^-24. Round a_float / 2^-24 to nearest even. */
    const double x = (double)bits_to_f32(a) * 16777216.0;
    double r = nearbyint(x); /* default rounding mode: nearest even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  /* normal: rebias 127 -> 15, keep 10 mantissa bits with RNE on the 13 dropped bits */
  uint32_t rebased = a - ((127u - 15u) << 23);
  uint32_t mant = rebased >> 13;
  const uint32_t rest = rebased & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (mant & 1u))) mant += 1u;
  return (uint16_t)(sign | (uint16_t)mant);
}

/* src/kernels/fp8.ts:24-36 — out[i] = e4m3(byte i) * scale[0], f32 multiply. Bytes are little-endian
 * within each u32, so byte i is simply bytes[i]. */
void or_unpack_fp8(const uint8_t* bytes, size_t n, float scale, float* out) {
  for (size_t i = 0; i < n; i++) out[i] = or_e4m3_gpu(bytes[i]) * scale;
}

/* int4 (this project's format): nibble j of a LE u32 word is k = 8 * word + j, two's complement. */
float or_int4_value(uint32_t word, int nibble, uint16_t scale_f16) {
  int q = (int)((word >> (4 * nibble)) & 0xfu);
  if (q >= 8) q -= 16;
  return (float)q * (float)or_f16(scale_f16);
}

void or_dequant_int4(const uint32_t* words, const uint16_t* scales, size_t rows, size_t k, size_t group, float* out) {
  const size_t groups = k / group;
  for (size_t r = 0; r < rows; r++)
    for (size_t kk = 0; kk < k; kk++) {
      const size_t idx = r * k + kk;
      out[idx] = or_int4_value(words[idx / 8], (int)(idx % 8), scales[r * groups + kk / group]);
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* Seeded generators                                                                                */
/* ------------------------------------------------------------------------------------------------ */

/* tests/gpu/matmul.test.ts:10-12 — seed = (seed * 1664525 + 1013904223) mod 2^32; value = seed / 2^32. */
uint32_t or_lcg_next(uint32_t* state) {
  *state = *state * 1664525u + 1013904223u;
  return *state;
}
double or_lcg_uniform(uint32_t* state) { return or_lcg_next(state) / 4294967296.0; }

/* n consecutive draws of the generator above, as doubles in [0, 1). */
void or_lcg_fill(uint32_t seed, size_t n, double* out) {
  uint32_t s = seed;
  for (size_t i = 0; i < n; i++) out[i] = or_lcg_uniform(&s);
}

/* tests/gpu/matmul.test.ts:14-23 — x (f32) first, uniform in [-1, 1); then fp8 bytes, NaN codes moved
 * down by one. */
void or_matmul_test_data(uint32_t m, uint32_t n, uint32_t k, uint32_t seed, float* x, uint8_t* w) {
  uint32_t s = seed;
  for (size_t i = 0; i < (size_t)m * k; i++) x[i] = (float)(or_lcg_uniform(&s) * 2.0 - 1.0);
  for (size_t i = 0; i < (size_t)n * k; i++) {
    int b = (int)floor(or_lcg_uniform(&s) * 256.0);
    if ((b & 0x7f) == 0x7f) b -= 1;
    w[i] = (uint8_t)b;
  }
}

/* src/model/noise.ts:9-39 — MT19937 as torch seeds it (low 32 bits of the seed). */
void or_mt_seed(or_mt19937* mt, uint64_t seed) {
  mt->state[0] = (uint32_t)seed;
  for (uint32_t i = 1; i < 624; i++) {
    const uint32_t prev = mt->state[i - 1];
    mt->state[i] = 1812433253u * (prev ^ (prev >> 30)) + i;
  }
  mt->index = 624;
}

static void mt_twist(or_mt19937* mt) {
  uint32_t* s = mt->state;
  for (int i = 0; i < 624; i++) {
    const uint32_t y = (s[i] & 0x80000000u) | (s[(i + 1) % 624] & 0x7fffffffu);
    s[i] = s[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
  }
  mt->index = 0;
}

uint32_t or_mt_next(or_mt19937* mt) {
  if (mt->index >= 624) mt_twist(mt);
  uint32_t y = mt->state[mt->index++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

/* src/model/noise.ts:45-48 */
static float uniform24(or_mt19937* mt) { return (float)(or_mt_next(mt) & 0xffffffu) * (1.0f / 16777216.0f); }
static double uniform53(or_mt19937* mt) {
  const double hi = (double)(or_mt_next(mt) & 0x1fffffu);
  const double lo = (double)or_mt_next(mt);
  return (hi * 4294967296.0 + lo) * ldexp(1.0, -53);
}

/* src/model/noise.ts:51-59 — Box-Muller over 16 values, pairs (j, j + 8), f32 rounding at each step. */
static void fill16(float* d) {
  const float two_pi = (float)(2.0 * M_PI);
  for (int j = 0; j < 8; j++) {
    const float u1 = 1.0f - d[j];
    const float radius = (float)sqrt((double)(-2.0f * (float)log((double)u1)));
    const float theta = two_pi * d[j + 8];
    d[j] = radius * (float)cos((double)theta);
    d[j + 8] = radius * (float)sin((double)theta);
  }
}

/* src/model/noise.ts:62-84 — torch.manual_seed(seed); torch.randn(n) on the CPU, float32. */
void or_torch_randn(size_t n, uint64_t seed, float* out) {
  or_mt19937 mt;
  or_mt_seed(&mt, seed);
  if (n < 16) {
    for (size_t i = 0; i < n; i += 2) {
      const double u1 = uniform53(&mt);
      const double u2 = uniform53(&mt);
      const double r = sqrt(-2.0 * log1p(-u2));
      const double theta = 2.0 * M_PI * u1;
      out[i] = (float)(r * cos(theta));
      if (i + 1 < n) out[i + 1] = (float)(r * sin(theta));
    }
    return;
  }
  for (size_t i = 0; i < n; i++) out[i] = uniform24(&mt);
  for (size_t i = 0; i + 16 <= n; i += 16) fill16(out + i);
  if (n % 16) {
    for (size_t i = n - 16; i < n; i++) out[i] = uniform24(&mt);
    fill16(out + n - 16);
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* Matmul                                                                                           */
/* ------------------------------------------------------------------------------------------------ */

/* src/kernels/matmul.ts:198-212 — defaults (negative = default) and the multiple-of-4 checks, in the
 * reference's order K, xStride, wStride, xOffset, wOffset, with its message text. Returns 0 or -1. */
int or_matmul_params_make(uint32_t m, uint32_t n, uint32_t k, float scale, int64_t x_stride, int64_t w_stride,
                          int64_t y_stride, int64_t x_offset, int64_t w_offset, int64_t y_offset, int64_t k_split,
                          or_matmul_params* out, char* msg, size_t msg_len) {
  const int64_t xs = x_stride < 0 ? k : x_stride, ws = w_stride < 0 ? k : w_stride, ys = y_stride < 0 ? n : y_stride;
  const int64_t xo = x_offset < 0 ? 0 : x_offset, wo = w_offset < 0 ? 0 : w_offset, yo = y_offset < 0 ? 0 : y_offset;
  const int64_t ks = k_split < 1 ? 1 : k_split;
  const char* names[5] = {"K", "xStride", "wStride", "xOffset", "wOffset"};
  const int64_t vals[5] = {k, xs, ws, xo, wo};
  for (int i = 0; i < 5; i++)
    if (vals[i] % 4) {
      if (msg) snprintf(msg, msg_len, "%s must be a multiple of 4, got %lld", names[i], (long long)vals[i]);
      return -1;
    }
  out->m = m;
  out->n = n;
  out->k = k;
  out->scale = scale;
  out->x_stride = (uint32_t)xs;
  out->w_stride = (uint32_t)ws;
  out->y_stride = (uint32_t)ys;
  out->x_offset = (uint32_t)xo;
  out->w_offset = (uint32_t)wo;
  out->y_offset = (uint32_t)yo;
  out->width = 0;
  out->cin = 0;
  out->k_split = (uint32_t)ks;
  if (msg && msg_len) msg[0] = 0;
  return 0;
}

/* src/model/ops.ts:38-45 — BUSY = 256 workgroups, MIN_SLICE = 256, TILE = 128. */
/* src/kernels/matmul.ts:268-272 — conv3x3Params: M = height * width pixels, N = cout, K = 9 * cin, the conv
 * input fields set; "cin must be a multiple of 4, got <cin>". */
int or_conv3x3_params(uint32_t height, uint32_t width, uint32_t cin, uint32_t cout, or_matmul_params* out, char* msg,
                      size_t msg_len) {
  if (cin % 4) {
    if (msg) snprintf(msg, msg_len, "cin must be a multiple of 4, got %u", cin);
    return -1;
  }
  if (or_matmul_params_make(height * width, cout, 9 * cin, 1.0f, -1, -1, -1, -1, -1, -1, 1, out, msg, msg_len)) return -1;
  out->width = width;
  out->cin = cin;
  return 0;
}

uint32_t or_ksplit_for(uint32_t m, uint32_t n, uint32_t k) {
  const uint32_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
  uint32_t want = (256 + tiles - 1) / tiles;
  const uint32_t cap = k / 256;
  uint32_t s = want < cap ? want : cap;
  return s < 1 ? 1 : s;
}

/* src/kernels/matmul.ts:156 — K values per slice: ceil(ceil(K / split) / 16) * 16. */
uint32_t or_ksplit_chunk(uint32_t k, uint32_t k_split) { return ((k + k_split - 1) / k_split + 15) / 16 * 16; }

static double load_x(int dtype, const void* x, size_t i) {
  switch (dtype) {
    case OR_F16: return or_f16(((const uint16_t*)x)[i]);
    case OR_BF16: return or_bf16(((const uint16_t*)x)[i]);
    default: return ((const float*)x)[i];
  }
}

/* src/kernels/matmul.ts:74-83 — the conv3x3 input: x is a channel-last image [M / width, width, cin], row r is
 * pixel r, k runs over (tap, channel): tap = k / cin reads pixel (r / width + tap / 3 - 1, r % width + tap % 3 - 1),
 * zero outside the image. */
static double load_x_conv(const or_matmul_params* p, int dtype, const void* x, uint32_t r, uint32_t kk) {
  const uint32_t tap = kk / p->cin, c = kk % p->cin;
  const int px = (int)(r % p->width) + (int)(tap % 3u) - 1, py = (int)(r / p->width) + (int)(tap / 3u) - 1;
  if (px < 0 || py < 0 || px >= (int)p->width || py >= (int)(p->m / p->width)) return 0.0;
  return load_x(dtype, x, ((size_t)py * p->width + (size_t)px) * p->cin + c);
}

static double load_w(int dtype, const void* w, const uint16_t* scales, uint32_t scales_per_row, uint32_t group,
                     uint32_t row, uint32_t kk, size_t idx) {
  switch (dtype) {
    case OR_FP8: return or_e4m3(((const uint8_t*)w)[idx]);
    case OR_BF16: return or_bf16(((const uint16_t*)w)[idx]);
    case OR_F16: return or_f16(((const uint16_t*)w)[idx]);
    case OR_INT4:
      return or_int4_value(((const uint32_t*)w)[idx / 8], (int)(idx % 8),
                           scales[(size_t)row * scales_per_row + kk / group]);
    default: return ((const float*)w)[idx];
  }
}

/* tests/gpu/matmul.test.ts:26-35 (float64 triple loop) with the layout of src/kernels/matmul.ts:5-32:
 *   y[r * y_stride + c + y_offset] (= | +=) scale * sum_k x[x_offset + r * x_stride + k] * W[w_offset + c * w_stride + k]
 * flags bit 0: split-K partials (matmul.ts:155-159): slice z sums k in [z*kc, min(K, z*kc + kc)) into rows
 * z * M + r. flags bit 1: accumulate (matmul.ts:145): y += ... instead of y = ....
 * int4 weights: W values are nibbles, scales [N, w_stride / group] f16. Rows [row_begin, row_end) only. */
static void matmul_rows(const or_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                        const uint16_t* w_scales, uint32_t group, int flags, uint32_t row_begin, uint32_t row_end,
                        double* y) {
  const int split = flags & 1;
  const int accumulate = flags & 2;
  const uint32_t slices = split ? p->k_split : 1;
  const uint32_t kc = split ? or_ksplit_chunk(p->k, p->k_split) : p->k;
  const uint32_t spr = (w_dtype == OR_INT4 && group) ? p->w_stride / group : 0;
  for (uint32_t z = 0; z < slices; z++) {
    const uint32_t kb = split ? z * kc : 0;
    uint32_t ke = split ? kb + kc : p->k;
    if (ke > p->k) ke = p->k;
    for (uint32_t r = row_begin; r < row_end; r++)
      for (uint32_t c = 0; c < p->n; c++) {
        double s = 0.0;
        for (uint32_t kk = kb; kk < ke; kk++) {
          const double xv = p->width ? load_x_conv(p, x_dtype, x, r, kk)
                                     : load_x(x_dtype, x, (size_t)p->x_offset + (size_t)r * p->x_stride + kk);
          const size_t widx = (size_t)p->w_offset + (size_t)c * p->w_stride + kk;
          s += xv * load_w(w_dtype, w, w_scales, spr, group, c, kk, widx);
        }
        const size_t o = (size_t)p->y_offset + ((size_t)z * p->m + r) * p->y_stride + c;
        y[o] = (accumulate ? y[o] : 0.0) + s * (double)p->scale;
      }
  }
}

void or_matmul_f64(const or_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                   const uint16_t* w_scales, uint32_t group, int flags, double* y) {
  matmul_rows(p, x_dtype, x, w_dtype, w, w_scales, group, flags, 0, p->m, y);
}

void or_matmul_f64_rows(const or_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                        const uint16_t* w_scales, uint32_t group, uint32_t row_begin, uint32_t row_end, double* y) {
  matmul_rows(p, x_dtype, x, w_dtype, w, w_scales, group, 0, row_begin, row_end, y);
}

/* src/kernels/text.ts:67-84 — out[t, d] = sum_l w[l] * x[t, l, d]. */
void or_layer_sum(uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w, double* out) {
  for (uint32_t t = 0; t < tokens; t++)
    for (uint32_t d = 0; d < dim; d++) {
      double s = 0.0;
      for (uint32_t l = 0; l < layers; l++) s += (double)w[l] * x[((size_t)t * layers + l) * dim + d];
      out[(size_t)t * dim + d] = s;
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* RMSNorm, RoPE, elementwise                                                                       */
/* ------------------------------------------------------------------------------------------------ */

/* tests/gpu/rmsnorm.test.ts:10-20 and src/kernels/rmsnorm.ts:42-45:
 *   out = x / sqrt(mean(x^2) + eps) * (offset + w) * (1 + scale) + shift. scale/shift may be NULL (zeros). */
void or_rmsnorm_f64(size_t rows, size_t d, double eps, double offset, const float* x, const float* weight,
                    const float* scale, const float* shift, double* out) {
  for (size_t r = 0; r < rows; r++) {
    double sum = 0.0;
    for (size_t i = 0; i < d; i++) sum += (double)x[r * d + i] * x[r * d + i];
    const double inv = 1.0 / sqrt(sum / (double)d + eps);
    for (size_t i = 0; i < d; i++)
      out[r * d + i] = x[r * d + i] * inv * (offset + weight[i]) * (1.0 + (scale ? scale[i] : 0.0f)) +
                       (shift ? shift[i] : 0.0f);
  }
}

/* src/kernels/rope.ts:14-18 — text tokens at the origin, then image tokens row by row; the last two
 * axes are (row, column), leading axes 0. pos is [tokens, axes]. */
void or_rope_positions(uint32_t text_tokens, uint32_t rows, uint32_t columns, uint32_t axes, double* pos) {
  const size_t tokens = (size_t)text_tokens + (size_t)rows * columns;
  memset(pos, 0, tokens * axes * sizeof(double));
  for (size_t i = 0; i < (size_t)rows * columns; i++) {
    double* p = pos + (text_tokens + i) * axes;
    if (axes >= 2) {
      p[axes - 2] = (double)(i / columns);
      p[axes - 1] = (double)(i % columns);
    } else if (axes == 1) {
      p[0] = (double)i;
    }
  }
}

/* src/kernels/rope.ts:20-36 — per axis of dim D: angle = pos * theta^(-2j / D) in f64, stored as f32.
 * Returns -1 for an odd axis ("Every RoPE axis needs an even number of dims"), else the pair count. */
int or_rope_tables(const double* pos, uint32_t tokens, const uint32_t* axes, uint32_t naxes, double theta,
                   float* cos_out, float* sin_out) {
  uint32_t pairs = 0;
  for (uint32_t a = 0; a < naxes; a++) {
    if (axes[a] % 2) return -1;
    pairs += axes[a] / 2;
  }
  for (uint32_t t = 0; t < tokens; t++) {
    uint32_t pair = 0;
    for (uint32_t a = 0; a < naxes; a++)
      for (uint32_t j = 0; j < axes[a] / 2; j++, pair++) {
        const double angle = pos[(size_t)t * naxes + a] * pow(theta, -(2.0 * j) / (double)axes[a]);
        cos_out[(size_t)t * pairs + pair] = (float)cos(angle);
        sin_out[(size_t)t * pairs + pair] = (float)sin(angle);
      }
  }
  return (int)pairs;
}

/* src/kernels/rope.ts:45-57 — interleaved pairs (2j, 2j+1) or half pairs (j, j + pairs). */
void or_rope_rotate_f64(uint32_t tokens, uint32_t heads, uint32_t pairs, int half, const float* x,
                        const float* cos_t, const float* sin_t, double* out) {
  for (uint32_t t = 0; t < tokens; t++)
    for (uint32_t h = 0; h < heads; h++)
      for (uint32_t j = 0; j < pairs; j++) {
        const double c = cos_t[(size_t)t * pairs + j], s = sin_t[(size_t)t * pairs + j];
        if (!half) {
          const size_t i = ((size_t)t * heads + h) * pairs + j;
          const double a = x[2 * i], b = x[2 * i + 1];
          out[2 * i] = a * c - b * s;
          out[2 * i + 1] = b * c + a * s;
        } else {
          const size_t base = ((size_t)t * heads + h) * pairs * 2;
          const double a = x[base + j], b = x[base + j + pairs];
          out[base + j] = a * c - b * s;
          out[base + j + pairs] = b * c + a * s;
        }
      }
}

/* tests/gpu/attention.test.ts:9-32 (and src/kernels/attention.ts:9-18): per query head h (kv head
 * g = h / (heads / kv_heads)) and query i, s_j = q_i . k_j / sqrt(dim) over keys j (causal: j <= i),
 * p = exp(s - max s) / sum, out = sum_j p_j v_j. q [tokens, heads, dim], k/v [tokens, kv_heads, dim];
 * only query rows [q_begin, q_end) are computed, into out[(i - q_begin), heads, dim]. */
void or_attention_f64(uint32_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t dim, int causal, uint32_t q_begin,
                      uint32_t q_end, const double* q, const double* k, const double* v, double* out) {
  const uint32_t group = heads / kv_heads;
  const double rs = 1.0 / sqrt((double)dim);
  double* s = (double*)malloc(sizeof(double) * (tokens ? tokens : 1));
  for (uint32_t h = 0; h < heads; h++) {
    const uint32_t g = h / group;
    for (uint32_t i = q_begin; i < q_end; i++) {
      const uint32_t n = causal ? i + 1 : tokens;
      const double* qi = q + ((size_t)i * heads + h) * dim;
      double mx = -INFINITY;
      for (uint32_t j = 0; j < n; j++) {
        const double* kj = k + ((size_t)j * kv_heads + g) * dim;
        double dot = 0.0;
        for (uint32_t d = 0; d < dim; d++) dot += qi[d] * kj[d];
        s[j] = dot * rs;
        if (s[j] > mx) mx = s[j];
      }
      double sum = 0.0;
      for (uint32_t j = 0; j < n; j++) {
        s[j] = exp(s[j] - mx);
        sum += s[j];
      }
      double* o = out + ((size_t)(i - q_begin) * heads + h) * dim;
      for (uint32_t d = 0; d < dim; d++) o[d] = 0.0;
      for (uint32_t j = 0; j < n; j++) {
        const double p = s[j] / sum;
        const double* vj = v + ((size_t)j * kv_heads + g) * dim;
        for (uint32_t d = 0; d < dim; d++) o[d] += p * vj[d];
      }
    }
  }
  free(s);
}

/* ------------------------------------------------------------------------------------------------ */
/* Blocks                                                                                           */
/* ------------------------------------------------------------------------------------------------ */

/* tests/gpu/block.test.ts:26-35: y[m, n] = scale * x[m, k] . e4m3(W[n, k]) in f64. */
static double* blk_mm(const double* x, const or_linear* w, size_t m) {
  double* y = (double*)malloc(sizeof(double) * m * w->n);
  double tab[256];
  for (int b = 0; b < 256; b++) tab[b] = or_e4m3((uint8_t)b);
  for (size_t i = 0; i < m; i++)
    for (uint32_t j = 0; j < w->n; j++) {
      double s = 0.0;
      const uint8_t* wr = w->bytes + (size_t)j * w->k;
      const double* xr = x + i * w->k;
      for (uint32_t t = 0; t < w->k; t++) s += xr[t] * tab[wr[t]];
      y[i * w->n + j] = s * w->scale;
    }
  return y;
}

/* tests/gpu/block.test.ts:36-45: x / sqrt(mean x^2 + eps) * (offset + w) * (1 + scale) + shift, per row. */
static double* blk_rmsnorm(const double* x, const float* w, size_t rows, size_t d, double eps, double offset,
                           const double* scale, const double* shift) {
  double* y = (double*)malloc(sizeof(double) * rows * d);
  for (size_t r = 0; r < rows; r++) {
    double ss = 0.0;
    for (size_t i = 0; i < d; i++) ss += x[r * d + i] * x[r * d + i];
    const double inv = 1.0 / sqrt(ss / (double)d + eps);
    for (size_t i = 0; i < d; i++)
      y[r * d + i] = x[r * d + i] * inv * (offset + w[i]) * (1.0 + (scale ? scale[i] : 0.0)) + (shift ? shift[i] : 0.0);
  }
  return y;
}

/* tests/gpu/block.test.ts:46-58: interleaved pairs, in place; row t of cos/sin for token t. */
static void blk_rope(double* x, size_t tokens, size_t heads, size_t pairs, const float* c, const float* s) {
  for (size_t t = 0; t < tokens; t++)
    for (size_t h = 0; h < heads; h++)
      for (size_t j = 0; j < pairs; j++) {
        const size_t i = ((t * heads + h) * pairs + j) * 2;
        const double cc = c[t * pairs + j], ss = s[t * pairs + j];
        const double a = x[i], b = x[i + 1];
        x[i] = a * cc - b * ss;
        x[i + 1] = b * cc + a * ss;
      }
}

static double blk_sigmoid(double v) { return 1.0 / (1.0 + exp(-v)); }

/* tests/gpu/block.test.ts:60-100 (the composition of src/model/block.ts:91-105): Krea single-stream block. */
void or_krea_block_f64(const or_block_cfg* cfg, uint32_t tokens, const double* x, const or_linear* w,
                       const float* norm1, const float* norm2, const float* norm_q, const float* norm_k,
                       const float* table, const float* temb, const float* cos_t, const float* sin_t, double* out) {
  const size_t H = cfg->hidden, T = tokens, hd = cfg->head_dim;
  double* mod = (double*)malloc(sizeof(double) * 6 * H);
  for (size_t i = 0; i < 6 * H; i++) mod[i] = (double)temb[i] + (double)table[i];
  const double *prescale = mod, *preshift = mod + H, *pregate = mod + 2 * H, *postscale = mod + 3 * H,
               *postshift = mod + 4 * H, *postgate = mod + 5 * H;
  double* h = blk_rmsnorm(x, norm1, T, H, cfg->eps, 1.0, prescale, preshift);
  double* q0 = blk_mm(h, &w[0], T);
  double* q = blk_rmsnorm(q0, norm_q, T * cfg->heads, hd, cfg->eps, 1.0, NULL, NULL);
  blk_rope(q, T, cfg->heads, hd / 2, cos_t, sin_t);
  double* k0 = blk_mm(h, &w[1], T);
  double* k = blk_rmsnorm(k0, norm_k, T * cfg->kv_heads, hd, cfg->eps, 1.0, NULL, NULL);
  blk_rope(k, T, cfg->kv_heads, hd / 2, cos_t, sin_t);
  double* v = blk_mm(h, &w[2], T);
  double* g = blk_mm(h, &w[3], T);
  double* o = (double*)malloc(sizeof(double) * T * cfg->heads * hd);
  or_attention_f64(tokens, cfg->heads, cfg->kv_heads, cfg->head_dim, 0, 0, tokens, q, k, v, o);
  for (size_t i = 0; i < T * H; i++) o[i] = o[i] * blk_sigmoid(g[i]);
  double* a = blk_mm(o, &w[4], T);
  double* x1 = (double*)malloc(sizeof(double) * T * H);
  for (size_t i = 0; i < T * H; i++) x1[i] = x[i] + pregate[i % H] * a[i];
  double* h2 = blk_rmsnorm(x1, norm2, T, H, cfg->eps, 1.0, postscale, postshift);
  double* gg = blk_mm(h2, &w[5], T);
  double* uu = blk_mm(h2, &w[6], T);
  for (size_t i = 0; i < T * cfg->mlp; i++) gg[i] = gg[i] * blk_sigmoid(gg[i]) * uu[i];
  double* d = blk_mm(gg, &w[7], T);
  for (size_t i = 0; i < T * H; i++) out[i] = x1[i] + postgate[i % H] * d[i];
  double* bufs[] = {mod, h, q0, q, k0, k, v, g, o, a, x1, h2, gg, uu, d};
  for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) free(bufs[i]);
}

/* The double-stream block of the DiT configuration, composed from the same steps (src/model/block.ts:33-105
 * order) with one set of weights per stream (text, image) and one joint attention:
 *   mod_s = tvec + table_s (6 vectors, src/model/block.ts:30-37)
 *   h_s = rmsnorm(x_s, norm1_s) * (1 + prescale_s) + preshift_s
 *   [q_s | k_s | v_s] = h_s . qkv_s^T;  q_s, k_s: per-head rmsnorm (norm_q_s, norm_k_s); image q, k: RoPE
 *   o = attention([q_txt; q_img], [k_txt; k_img], [v_txt; v_img])   (text rows first)
 *   x1_s = x_s + pregate_s * (o_s . proj_s^T)
 *   out_s = x1_s + postgate_s * (gelu_tanh((rmsnorm(x1_s, norm2_s) * (1 + postscale_s) + postshift_s) . up_s^T)
 *           . down_s^T)
 * All norms use offset 1 and cfg->eps; heads == kv_heads. */
void or_double_block_f64(const or_block_cfg* cfg, uint32_t txt_tokens, uint32_t img_tokens, const double* x_txt,
                         const double* x_img, const or_stream_weights* txt, const or_stream_weights* img,
                         const float* tvec, const float* cos_img, const float* sin_img, double* out_txt,
                         double* out_img) {
  const size_t H = cfg->hidden, hd = cfg->head_dim, heads = cfg->heads, T = (size_t)txt_tokens + img_tokens;
  const or_stream_weights* ws[2] = {txt, img};
  const double* xs[2] = {x_txt, x_img};
  double* outs[2] = {out_txt, out_img};
  const size_t rows[2] = {txt_tokens, img_tokens}, row0[2] = {0, txt_tokens};
  double* q = (double*)malloc(sizeof(double) * T * H);
  double* k = (double*)malloc(sizeof(double) * T * H);
  double* v = (double*)malloc(sizeof(double) * T * H);
  double* mod[2];
  for (int s = 0; s < 2; s++) {
    mod[s] = (double*)malloc(sizeof(double) * 6 * H);
    for (size_t i = 0; i < 6 * H; i++) mod[s][i] = (double)tvec[i] + (double)ws[s]->table[i];
    double* h = blk_rmsnorm(xs[s], ws[s]->norm1, rows[s], H, cfg->eps, 1.0, mod[s], mod[s] + H);
    double* qkv = blk_mm(h, &ws[s]->qkv, rows[s]);
    double* qs = (double*)malloc(sizeof(double) * rows[s] * H);
    double* ks = (double*)malloc(sizeof(double) * rows[s] * H);
    for (size_t r = 0; r < rows[s]; r++)
      for (size_t i = 0; i < H; i++) {
        qs[r * H + i] = qkv[r * 3 * H + i];
        ks[r * H + i] = qkv[r * 3 * H + H + i];
        v[(row0[s] + r) * H + i] = qkv[r * 3 * H + 2 * H + i];
      }
    double* qn = blk_rmsnorm(qs, ws[s]->norm_q, rows[s] * heads, hd, cfg->eps, 1.0, NULL, NULL);
    double* kn = blk_rmsnorm(ks, ws[s]->norm_k, rows[s] * heads, hd, cfg->eps, 1.0, NULL, NULL);
    if (s == 1) {
      blk_rope(qn, rows[s], heads, hd / 2, cos_img, sin_img);
      blk_rope(kn, rows[s], heads, hd / 2, cos_img, sin_img);
    }
    memcpy(q + row0[s] * H, qn, sizeof(double) * rows[s] * H);
    memcpy(k + row0[s] * H, kn, sizeof(double) * rows[s] * H);
    free(h);
    free(qkv);
    free(qs);
    free(ks);
    free(qn);
    free(kn);
  }
  double* o = (double*)malloc(sizeof(double) * T * H);
  or_attention_f64((uint32_t)T, (uint32_t)heads, (uint32_t)heads, (uint32_t)hd, 0, 0, (uint32_t)T, q, k, v, o);
  for (int s = 0; s < 2; s++) {
    const double *pregate = mod[s] + 2 * H, *postscale = mod[s] + 3 * H, *postshift = mod[s] + 4 * H,
                 *postgate = mod[s] + 5 * H;
    double* a = blk_mm(o + row0[s] * H, &ws[s]->proj, rows[s]);
    double* x1 = (double*)malloc(sizeof(double) * rows[s] * H);
    for (size_t i = 0; i < rows[s] * H; i++) x1[i] = xs[s][i] + pregate[i % H] * a[i];
    double* h2 = blk_rmsnorm(x1, ws[s]->norm2, rows[s], H, cfg->eps, 1.0, postscale, postshift);
    double* u = blk_mm(h2, &ws[s]->up, rows[s]);
    for (size_t i = 0; i < rows[s] * cfg->mlp; i++) u[i] = or_gelu_tanh(u[i]);
    double* d = blk_mm(u, &ws[s]->down, rows[s]);
    for (size_t i = 0; i < rows[s] * H; i++) outs[s][i] = x1[i] + postgate[i % H] * d[i];
    free(a);
    free(x1);
    free(h2);
    free(u);
    free(d);
    free(mod[s]);
  }
  free(q);
  free(k);
  free(v);
  free(o);
}

/* tests/gpu/text.test.ts:58 — PyTorch's tanh GELU, textbook form. */
double or_gelu_tanh(double v) { return 0.5 * v * (1.0 + tanh(sqrt(2.0 / M_PI) * (v + 0.044715 * v * v * v))); }

/* src/kernels/elementwise.ts:25-29 — the shader's f32 form: tanh through exp with |u| clamped to 15. */
float or_gelu_tanh_shader(float v) {
  float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  if (u < -15.0f) u = -15.0f;
  if (u > 15.0f) u = 15.0f;
  const float e = expf(2.0f * u);
  return 0.5f * v * (1.0f + (e - 1.0f) / (e + 1.0f));
}

/* src/kernels/elementwise.ts:22 */
double or_sigmoid(double v) { return 1.0 / (1.0 + exp(-v)); }

/* src/kernels/elementwise.ts:38-84 — the per-value ops, in f64. d is the column count for the ops that
 * index a per-column vector (gatedAdd: x + g[i % d] * h; addBias: x + b[i % d]). */
void or_elementwise_f64(int op, size_t n, size_t d, const float* a, const float* b, const float* c, double* out) {
  for (size_t i = 0; i < n; i++) {
    switch (op) {
      case OR_SWIGLU: out[i] = a[i] * or_sigmoid(a[i]) * b[i]; break;
      case OR_SIGMOID_GATE: out[i] = a[i] * or_sigmoid(b[i]); break;
      case OR_GATED_ADD: out[i] = a[i] + (double)c[i % d] * b[i]; break;
      case OR_ADD_BIAS: out[i] = a[i] + (double)b[i % d]; break;
      case OR_GELU_TANH: out[i] = or_gelu_tanh(a[i]); break;
      case OR_ADD: out[i] = (double)a[i] + b[i]; break;
      case OR_SILU: out[i] = a[i] * or_sigmoid(a[i]); break;
      default: out[i] = NAN;
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* Comparisons                                                                                      */
/* ------------------------------------------------------------------------------------------------ */

/* tests/gpu/matmul.test.ts:38-46 — largest error relative to the largest reference value. */
double or_rel_error(const double* got, const double* ref, size_t n) {
  double err = 0.0, mx = 0.0;
  for (size_t i = 0; i < n; i++) {
    const double e = fabs(got[i] - ref[i]);
    if (e > err || isnan(e)) err = isnan(e) ? INFINITY : e;
    if (fabs(ref[i]) > mx) mx = fabs(ref[i]);
  }
  return err / mx;
}

/* src/model/compare.ts:2-17 — cosine similarity, max error, L2 relative error. */
void or_compare(const double* result, const double* reference, size_t n, double* cosine, double* max_error,
                double* relative_error) {
  double dot = 0.0, a2 = 0.0, b2 = 0.0, mx = 0.0, e2 = 0.0;
  for (size_t i = 0; i < n; i++) {
    const double a = result[i], b = reference[i];
    dot += a * b;
    a2 += a * a;
    b2 += b * b;
    if (fabs(a - b) > mx) mx = fabs(a - b);
    e2 += (a - b) * (a - b);
  }
  *cosine = dot / sqrt(a2 * b2);
  *max_error = mx;
  *relative_error = sqrt(e2 / b2);
}
