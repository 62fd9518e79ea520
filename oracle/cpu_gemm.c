/*
 * Strong CPU baseline of the quantized-weight matmul: y[m, n] = scale * sum_k x[m, k] * W[n, k] with f32
 * accumulation on every host thread given, AVX-512 where the host has it (runtime check), portable C elsewhere.
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it beside the faithful float64 loop of
 * tests/gpu/matmul.test.ts:26-35 (or_matmul_f64), and tests/test_cpu_baseline.py checks it against that loop.
 * The product library never links or calls it.
 *
 * Weights are decoded as or_matmul_f64 decodes them (fp8 e4m3fn by table, bf16, f16, f32, or this project's
 * int4: two's-complement nibbles times an f16 scale per group of K). Layout is the contiguous default of
 * src/kernels/matmul.ts:198-212 (x [M, K], W [N, K], y [M, N]).
 *
 * Blocking: a thread takes 64 output columns at a time; per 128-k block it decodes W into an f32 panel
 * [128][64] (32 KB, stays in L1) and runs every 6-row strip of x through a 6 x 64 register tile (24 zmm
 * accumulators), then scales and converts the finished columns.
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#if defined(__x86_64__)
#include <immintrin.h>
#define CB_X86 1
#else
#define CB_X86 0
#endif

enum { NB = 64, KB = 128, MR = 6 };

typedef struct {
  uint32_t m, n, k, group;
  float scale;
  int w_dtype, y_dtype, gelu;
  const float* a;  /* x as f32 [m, k] */
  const void* w;
  const uint16_t* scales;
  void* y;
  float table[256];  /* fp8 decode */
  float* half;       /* f16 decode, 65536 entries (f16 weights or activations only) */
  atomic_uint next;  /* next 64-column block */
  int use_avx512;
} job_t;

static float w_value(const job_t* j, uint32_t row, uint32_t kk) {
  const size_t idx = (size_t)row * j->k + kk;
  switch (j->w_dtype) {
    case OR_FP8: return j->table[((const uint8_t*)j->w)[idx]];
    case OR_BF16: return or_bf16(((const uint16_t*)j->w)[idx]);
    case OR_F16: return (float)or_f16(((const uint16_t*)j->w)[idx]);
    case OR_INT4:
      return or_int4_value(((const uint32_t*)j->w)[idx / 8], (int)(idx % 8),
                           j->scales[(size_t)row * (j->k / j->group) + kk / j->group]);
    default: return ((const float*)j->w)[idx];
  }
}

/* panel[kk][c] = W[n0 + c][k0 + kk] for c < cols (zeros beyond) */
static void pack(const job_t* j, uint32_t n0, uint32_t cols, uint32_t k0, uint32_t kb, float* panel) {
  if (cols < NB) memset(panel, 0, sizeof(float) * KB * NB);
  for (uint32_t c = 0; c < cols; c++) {
    const size_t row = (size_t)(n0 + c) * j->k + k0;
    switch (j->w_dtype) {
      case OR_FP8: {
        const uint8_t* src = (const uint8_t*)j->w + row;
        for (uint32_t kk = 0; kk < kb; kk++) panel[kk * NB + c] = j->table[src[kk]];
        break;
      }
      case OR_F16: {
        const uint16_t* src = (const uint16_t*)j->w + row;
        for (uint32_t kk = 0; kk < kb; kk++) panel[kk * NB + c] = j->half[src[kk]];
        break;
      }
      case OR_INT4: { /* k0 and kb are multiples of 8 here (K % group == 0, group % 8 == 0, KB % 8 == 0) */
        const uint32_t* words = (const uint32_t*)j->w + row / 8;
        const uint16_t* sc = j->scales + (size_t)(n0 + c) * (j->k / j->group);
        for (uint32_t kk = 0; kk < kb; kk += 8) {
          const float s = j->half[sc[(k0 + kk) / j->group]];
          const uint32_t word = words[kk / 8];
          for (int q = 0; q < 8; q++) panel[(kk + q) * NB + c] = (float)((int)((word >> (4 * q)) & 0xfu) ^ 8) - 8.0f;
          for (int q = 0; q < 8; q++) panel[(kk + q) * NB + c] *= s;
        }
        break;
      }
      default:
        for (uint32_t kk = 0; kk < kb; kk++) panel[kk * NB + c] = w_value(j, n0 + c, k0 + kk);
    }
  }
}

/* c[r][0..63] += sum_kk a[r][kk] * panel[kk][0..63] for R rows (portable form) */
static void strip_c(int R, uint32_t kb, const float* a, size_t lda, const float* panel, float* c) {
  for (int r = 0; r < R; r++) {
    float acc[NB];
    memcpy(acc, c + (size_t)r * NB, sizeof acc);
    for (uint32_t kk = 0; kk < kb; kk++) {
      const float av = a[(size_t)r * lda + kk];
      const float* p = panel + (size_t)kk * NB;
      for (int q = 0; q < NB; q++) acc[q] += av * p[q];
    }
    memcpy(c + (size_t)r * NB, acc, sizeof acc);
  }
}

#if CB_X86
__attribute__((target("avx512f"), always_inline)) static inline void strip_avx512_r(const int R, uint32_t kb,
                                                                                     const float* a, size_t lda,
                                                                                     const float* panel, float* c) {
  __m512 acc[MR][4];
  for (int r = 0; r < R; r++)
    for (int q = 0; q < 4; q++) acc[r][q] = _mm512_loadu_ps(c + (size_t)r * NB + 16 * q);
  for (uint32_t kk = 0; kk < kb; kk++) {
    const float* p = panel + (size_t)kk * NB;
    const __m512 b0 = _mm512_loadu_ps(p), b1 = _mm512_loadu_ps(p + 16), b2 = _mm512_loadu_ps(p + 32),
                 b3 = _mm512_loadu_ps(p + 48);
    for (int r = 0; r < R; r++) {
      const __m512 av = _mm512_set1_ps(a[(size_t)r * lda + kk]);
      acc[r][0] = _mm512_fmadd_ps(av, b0, acc[r][0]);
      acc[r][1] = _mm512_fmadd_ps(av, b1, acc[r][1]);
      acc[r][2] = _mm512_fmadd_ps(av, b2, acc[r][2]);
      acc[r][3] = _mm512_fmadd_ps(av, b3, acc[r][3]);
    }
  }
  for (int r = 0; r < R; r++)
    for (int q = 0; q < 4; q++) _mm512_storeu_ps(c + (size_t)r * NB + 16 * q, acc[r][q]);
}

__attribute__((target("avx512f"))) static void strip_avx512(int R, uint32_t kb, const float* a, size_t lda,
                                                             const float* panel, float* c) {
  switch (R) {
    case 6: strip_avx512_r(6, kb, a, lda, panel, c); break;
    case 5: strip_avx512_r(5, kb, a, lda, panel, c); break;
    case 4: strip_avx512_r(4, kb, a, lda, panel, c); break;
    case 3: strip_avx512_r(3, kb, a, lda, panel, c); break;
    case 2: strip_avx512_r(2, kb, a, lda, panel, c); break;
    default: strip_avx512_r(1, kb, a, lda, panel, c); break;
  }
}
#endif

static void* worker(void* arg) {
  job_t* j = (job_t*)arg;
  float* panel = (float*)aligned_alloc(64, sizeof(float) * KB * NB);
  float* acc = (float*)aligned_alloc(64, sizeof(float) * (size_t)((j->m + MR - 1) / MR * MR) * NB);
  if (!panel || !acc) {
    free(panel);
    free(acc);
    return (void*)1;
  }
  const uint32_t blocks = (j->n + NB - 1) / NB;
  for (;;) {
    const uint32_t b = atomic_fetch_add(&j->next, 1u);
    if (b >= blocks) break;
    const uint32_t n0 = b * NB, cols = j->n - n0 < NB ? j->n - n0 : NB;
    memset(acc, 0, sizeof(float) * (size_t)j->m * NB);
    for (uint32_t k0 = 0; k0 < j->k; k0 += KB) {
      const uint32_t kb = j->k - k0 < KB ? j->k - k0 : KB;
      pack(j, n0, cols, k0, kb, panel);
      for (uint32_t m0 = 0; m0 < j->m; m0 += MR) {
        const int R = (int)(j->m - m0 < MR ? j->m - m0 : MR);
        const float* a = j->a + (size_t)m0 * j->k + k0;
#if CB_X86
        if (j->use_avx512) {
          strip_avx512(R, kb, a, j->k, panel, acc + (size_t)m0 * NB);
          continue;
        }
#endif
        strip_c(R, kb, a, j->k, panel, acc + (size_t)m0 * NB);
      }
    }
    for (uint32_t r = 0; r < j->m; r++)
      for (uint32_t c = 0; c < cols; c++) {
        float v = acc[(size_t)r * NB + c] * j->scale;
        if (j->gelu) v = v / (1.0f + expf(-2.0f * 0.7978845608f * v * (1.0f + 0.044715f * v * v)));
        const size_t o = (size_t)r * j->n + n0 + c;
        switch (j->y_dtype) {
          case OR_F16: ((uint16_t*)j->y)[o] = or_f32_to_f16(v); break;
          case OR_BF16: ((uint16_t*)j->y)[o] = or_f32_to_bf16(v); break;
          default: ((float*)j->y)[o] = v;
        }
      }
  }
  free(panel);
  free(acc);
  return NULL;
}

/* Returns 0, or -1 for bad arguments / no memory. threads <= 0 means 1. avx512: 1 = use when the host has it,
 * 0 = portable C only. gelu: tanh GELU on the scaled sum, in the form v / (1 + e^(-2u)) (= 0.5 v (1 + tanh u)),
 * before the conversion to y's dtype. */
int cb_matmul(int threads, int avx512, uint32_t m, uint32_t n, uint32_t k, float scale, int x_dtype, const void* x,
              int w_dtype, const void* w, const uint16_t* scales, uint32_t group, int y_dtype, int gelu, void* y) {
  if (!m || !n || !k || !x || !w || !y) return -1;
  if (w_dtype == OR_INT4 && (!scales || !group || k % group || group % 8)) return -1;
  if (threads <= 0) threads = 1;
  job_t* j = (job_t*)calloc(1, sizeof *j);
  float* a = (float*)malloc(sizeof(float) * (size_t)m * k);
  pthread_t* tid = (pthread_t*)calloc((size_t)threads, sizeof *tid);
  if (!j || !a || !tid) {
    free(j);
    free(a);
    free(tid);
    return -1;
  }
  if (x_dtype == OR_F16 || w_dtype == OR_F16 || w_dtype == OR_INT4) {
    j->half = (float*)malloc(sizeof(float) * 65536);
    if (!j->half) {
      free(j);
      free(a);
      free(tid);
      return -1;
    }
    for (uint32_t h = 0; h < 65536; h++) j->half[h] = (float)or_f16((uint16_t)h);
  }
  for (size_t i = 0; i < (size_t)m * k; i++) {
    switch (x_dtype) {
      case OR_F16: a[i] = j->half[((const uint16_t*)x)[i]]; break;
      case OR_BF16: a[i] = or_bf16(((const uint16_t*)x)[i]); break;
      default: a[i] = ((const float*)x)[i];
    }
  }
  for (int b = 0; b < 256; b++) j->table[b] = (float)or_e4m3((uint8_t)b);
  j->m = m, j->n = n, j->k = k, j->group = group, j->scale = scale, j->w_dtype = w_dtype, j->y_dtype = y_dtype;
  j->gelu = gelu;
  j->a = a, j->w = w, j->scales = scales, j->y = y;
  atomic_init(&j->next, 0u);
#if CB_X86
  j->use_avx512 = avx512 && __builtin_cpu_supports("avx512f");
#else
  (void)avx512;
#endif
  int rc = 0, started = 0;
  for (int t = 0; t < threads; t++) {
    if (pthread_create(&tid[t], NULL, worker, j) != 0) break;
    started++;
  }
  if (started == 0) rc = -1;
  for (int t = 0; t < started; t++) {
    void* r = NULL;
    pthread_join(tid[t], &r);
    if (r) rc = -1;
  }
  free(tid);
  free(a);
  free(j->half);
  free(j);
  return rc;
}

/* 1 when cb_matmul(avx512 = 1) runs the AVX-512 strip on this host */
int cb_has_avx512(void) {
#if CB_X86
  return __builtin_cpu_supports("avx512f") ? 1 : 0;
#else
  return 0;
#endif
}
