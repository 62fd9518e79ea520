/*
 * CPU oracle for the quantized-weight matmul path (fp8 / bf16 / f32 / int4 weights, RMSNorm, RoPE,
 * elementwise epilogues, split-K). TEST INFRASTRUCTURE ONLY: the tests, the smoke check and the
 * bench's cpu_baseline leg load it to check results; the product library never links or calls it.
 *
 * Every function restates the reference's algorithm in plain C and cites the reference file:line it
 * follows (paths relative to the dotstories/web-engine tree). Accumulation that the reference's
 * tests do in float64 is done in double here as well.
 *
 * int4 weights have no counterpart in the reference (its matmul takes fp8 / bf16 / f32 only). Their
 * format is this project's definition: 8 two's-complement nibbles per little-endian u32 along K,
 * low nibble = lowest k, one f16 scale per `group` consecutive k of a row, value = q * s in f32.
 * Parity of int4 against the reference is therefore unpinned by the reference; the tests pin the
 * definition with closed forms (all 16 codes x scales) and a numpy brute force.
 */
#ifndef WE_ORACLE_H
#define WE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags, the same values as the product ABI uses */
enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2, OR_FP8 = 3, OR_INT4 = 4 };

/* ---- decoders ---- */
double or_e4m3(uint8_t b);          /* NaN for 0x7f / 0xff, -0 kept */
float or_e4m3_gpu(uint8_t b);       /* shader formula: no NaN branch, 0x7f -> 480 */
double or_e5m2(uint8_t b);
double or_f16(uint16_t h);
float or_bf16(uint16_t h);
uint16_t or_f32_to_bf16(float v);   /* round to nearest even (NaN kept quiet) */
uint16_t or_f32_to_f16(float v);    /* round to nearest even, overflow -> inf */
void or_unpack_fp8(const uint8_t* bytes, size_t n, float scale, float* out);
float or_int4_value(uint32_t word, int nibble, uint16_t scale_f16);
void or_dequant_int4(const uint32_t* words, const uint16_t* scales, size_t rows, size_t k, size_t group, float* out);

/* ---- seeded generators ---- */
uint32_t or_lcg_next(uint32_t* state);
double or_lcg_uniform(uint32_t* state);
void or_lcg_fill(uint32_t seed, size_t n, double* out);
void or_matmul_test_data(uint32_t m, uint32_t n, uint32_t k, uint32_t seed, float* x, uint8_t* w);
typedef struct { uint32_t state[624]; int index; } or_mt19937;
void or_mt_seed(or_mt19937* mt, uint64_t seed);
uint32_t or_mt_next(or_mt19937* mt);
void or_torch_randn(size_t n, uint64_t seed, float* out);

/* ---- matmul ---- */
typedef struct {
  uint32_t m, n, k;
  float scale;
  uint32_t x_stride, w_stride, y_stride, x_offset, w_offset, y_offset, width, cin, k_split;
} or_matmul_params;

int or_matmul_params_make(uint32_t m, uint32_t n, uint32_t k, float scale, int64_t x_stride, int64_t w_stride,
                          int64_t y_stride, int64_t x_offset, int64_t w_offset, int64_t y_offset, int64_t k_split,
                          or_matmul_params* out, char* msg, size_t msg_len);
uint32_t or_ksplit_for(uint32_t m, uint32_t n, uint32_t k);
int or_conv3x3_params(uint32_t height, uint32_t width, uint32_t cin, uint32_t cout, or_matmul_params* out, char* msg,
                      size_t msg_len);

/* ---- strong CPU baseline (cpu_gemm.c): y = scale * x . W^T (then tanh GELU when `gelu`), f32 accumulation,
 * `threads` host threads, AVX-512 when `avx512` and the host has it; contiguous layout, y dtype F32 / F16 / BF16.
 * 0 or -1. */
int cb_matmul(int threads, int avx512, uint32_t m, uint32_t n, uint32_t k, float scale, int x_dtype, const void* x,
              int w_dtype, const void* w, const uint16_t* scales, uint32_t group, int y_dtype, int gelu, void* y);
int cb_has_avx512(void);
uint32_t or_ksplit_chunk(uint32_t k, uint32_t k_split);
void or_matmul_f64(const or_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                   const uint16_t* w_scales, uint32_t group, int flags, double* y);
void or_matmul_f64_rows(const or_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                        const uint16_t* w_scales, uint32_t group, uint32_t row_begin, uint32_t row_end, double* y);
void or_layer_sum(uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w, double* out);

/* ---- norms, rope, elementwise ---- */
void or_rmsnorm_f64(size_t rows, size_t d, double eps, double offset, const float* x, const float* weight,
                    const float* scale, const float* shift, double* out);
void or_rope_positions(uint32_t text_tokens, uint32_t rows, uint32_t columns, uint32_t axes, double* pos);
int or_rope_tables(const double* pos, uint32_t tokens, const uint32_t* axes, uint32_t naxes, double theta,
                   float* cos_out, float* sin_out);
/* Blocks (f64 compositions of the primitives above). */
typedef struct {
  const uint8_t* bytes; /* fp8 e4m3fn [n, k] */
  float scale;
  uint32_t n, k;
} or_linear;
typedef struct {
  uint32_t hidden, mlp, heads, kv_heads, head_dim;
  double eps;
} or_block_cfg;
/* w: wq, wk, wv, gate, wo, mlpGate, mlpUp, mlpDown */
void or_krea_block_f64(const or_block_cfg* cfg, uint32_t tokens, const double* x, const or_linear* w,
                       const float* norm1, const float* norm2, const float* norm_q, const float* norm_k,
                       const float* table, const float* temb, const float* cos_t, const float* sin_t, double* out);
typedef struct {
  or_linear qkv, proj, up, down;
  const float *norm1, *norm2, *norm_q, *norm_k, *table;
} or_stream_weights;
void or_double_block_f64(const or_block_cfg* cfg, uint32_t txt_tokens, uint32_t img_tokens, const double* x_txt,
                         const double* x_img, const or_stream_weights* txt, const or_stream_weights* img,
                         const float* tvec, const float* cos_img, const float* sin_img, double* out_txt,
                         double* out_img);
void or_attention_f64(uint32_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t dim, int causal, uint32_t q_begin,
                      uint32_t q_end, const double* q, const double* k, const double* v, double* out);
void or_rope_rotate_f64(uint32_t tokens, uint32_t heads, uint32_t pairs, int half, const float* x,
                        const float* cos_t, const float* sin_t, double* out);
double or_gelu_tanh(double v);
float or_gelu_tanh_shader(float v);
double or_sigmoid(double v);
void or_elementwise_f64(int op, size_t n, size_t d, const float* a, const float* b, const float* c, double* out);
enum { OR_SWIGLU = 0, OR_SIGMOID_GATE = 1, OR_GATED_ADD = 2, OR_ADD_BIAS = 3, OR_GELU_TANH = 4, OR_ADD = 5, OR_SILU = 6 };

/* ---- comparisons ---- */
double or_rel_error(const double* got, const double* ref, size_t n);
void or_compare(const double* result, const double* reference, size_t n, double* cosine, double* max_error,
                double* relative_error);

#ifdef __cplusplus
}
#endif
#endif
