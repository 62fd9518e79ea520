// Memory-bound kernels around the matmul: buffer zeroing, the dequantization test kernels, the
// elementwise ops, the split-K layer sum, RMSNorm, RoPE and the fused per-head RMSNorm + RoPE of q/k.
// All math is f32; activations may be stored as f32, f16 or bf16.
#include "common.h"
#include "internal.h"

namespace we {

static inline unsigned grid_for(size_t n, unsigned threads, unsigned cap = 1u << 20) {
  size_t g = (n + threads - 1) / threads;
  if (g > cap) g = cap;
  return (unsigned)(g ? g : 1);
}

// ------------------------------------------------------------------ zero fill (Graph's zero shader, src/gpu/graph.ts:14-21)
// and the poison fill of freed buffers (every byte 0xff: NaN as f32, bf16, f16 and e4m3)
__global__ void fill_kernel(u32x4* p16, size_t n16, uint8_t* tail, size_t ntail, uint32_t byte) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const uint32_t word = byte * 0x01010101u;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    p16[i] = u32x4{word, word, word, word};
  if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = (uint8_t)byte;
}

hipError_t launch_fill(void* p, size_t bytes, uint8_t byte, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const size_t n16 = bytes / 16, tail = bytes % 16;
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n16 ? n16 : 1, 256, 4096)), dim3(256), 0, s, (u32x4*)p, n16,
                     (uint8_t*)p + n16 * 16, tail, (uint32_t)byte);
  return hipGetLastError();
}

hipError_t launch_zero(void* p, size_t bytes, hipStream_t s) { return launch_fill(p, bytes, 0, s); }

// ------------------------------------------------------------------ f32 activations as three bf16 planes
// out[r, p K + k] = plane p of x[r, k]: hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid). Each remainder is
// exact in f32 (at most 16, then 8 significant bits), so hi + mid + lo == x for every normal f32 value and a GEMM
// over the 3K planes against weights that repeat every K sums exact products of all 24 bits of x. One thread per 8
// consecutive values of a row (two 16-byte loads, three 16-byte stores); x rows 16-byte aligned, K % 8 == 0.
__global__ void __launch_bounds__(256) split_f32_planes_kernel(const float* __restrict__ x, uint32_t m, uint32_t k,
                                                              uint32_t xs, uint16_t* __restrict__ out) {
  const uint32_t groups = k / 8;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)m * groups) return;
  const uint32_t r = (uint32_t)(idx / groups), g = (uint32_t)(idx % groups);
  const float* src = x + (size_t)r * xs + (size_t)g * 8;
  const f32x4 a = *(const f32x4*)src, b = *(const f32x4*)(src + 4);
  const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  uint32_t h[3][8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    h[0][i] = f32_to_bf16(v[i]);
    const float r1 = v[i] - bf16_to_f32((uint16_t)h[0][i]);
    h[1][i] = f32_to_bf16(r1);
    h[2][i] = f32_to_bf16(r1 - bf16_to_f32((uint16_t)h[1][i]));
  }
  uint16_t* dst = out + (size_t)r * 3 * k + (size_t)g * 8;
#pragma unroll
  for (int p = 0; p < 3; p++)
    *(u32x4*)(dst + (size_t)p * k) = u32x4{h[p][0] | (h[p][1] << 16), h[p][2] | (h[p][3] << 16),
                                           h[p][4] | (h[p][5] << 16), h[p][6] | (h[p][7] << 16)};
}

hipError_t launch_split_f32_planes(const float* x, uint32_t m, uint32_t k, uint32_t x_stride, uint16_t* out,
                                   hipStream_t s) {
  const size_t n = (size_t)m * (k / 8);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(split_f32_planes_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, m, k, x_stride,
                     out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ unpackFp8 (src/kernels/fp8.ts:24-36)
__global__ void unpack_fp8_kernel(const uint8_t* packed, size_t n, const float* scale, float* out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const float sc = scale[0];
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = e4m3_shader(packed[i]) * sc;
}

hipError_t launch_unpack_fp8(const void* packed, size_t n, const float* scale, float* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(unpack_fp8_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, (const uint8_t*)packed, n, scale, out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ int4 dequant (q * s in f32, exact)
__global__ void dequant_int4_kernel(const uint32_t* w, const uint16_t* sc, uint32_t rows, uint32_t k, uint32_t group,
                                    float* out) {
  const size_t total = (size_t)rows * k;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const uint32_t gpr = k / group;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint32_t r = (uint32_t)(i / k), kk = (uint32_t)(i % k);
    const int q = ((int)(w[i / 8] << (28 - 4 * (i % 8)))) >> 28;
    out[i] = (float)q * f16_to_f32(sc[(size_t)r * gpr + kk / group]);
  }
}

hipError_t launch_dequant_int4(const uint32_t* w, const uint16_t* sc, uint32_t rows, uint32_t k, uint32_t group,
                               float* out, hipStream_t s) {
  const size_t n = (size_t)rows * k;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(dequant_int4_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, w, sc, rows, k, group, out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ elementwise (src/kernels/elementwise.ts:38-84)
// a, b, out: activations of dtype DT; per-column vectors (add_bias: b, gated_add: c) are f32.
template <int DT>
__global__ void elementwise_kernel(int op, size_t n, size_t d, const void* a, const void* b, const void* c, void* out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float x = load_as_f32<DT>(a, i);
    float r;
    switch (op) {
      case 0: r = x * sigmoid(x) * load_as_f32<DT>(b, i); break;         // swiglu
      case 1: r = x * sigmoid(load_as_f32<DT>(b, i)); break;             // sigmoidGate
      case 2: r = x + ((const float*)c)[i % d] * load_as_f32<DT>(b, i); break;  // gatedAdd
      case 3: r = x + ((const float*)b)[i % d]; break;                   // addBias
      case 4: r = gelu_tanh(x); break;                                   // geluTanh
      case 5: r = x + load_as_f32<DT>(b, i); break;                      // add
      default: r = x * sigmoid(x); break;                                // silu
    }
    store_from_f32<DT>(out, i, r);
  }
}

hipError_t launch_elementwise(int op, size_t n, size_t d, int dtype, const void* a, const void* b, const void* c,
                              void* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const dim3 g(grid_for(n, 256)), t(256);
  switch (dtype) {
    case F16: hipLaunchKernelGGL(elementwise_kernel<F16>, g, t, 0, s, op, n, d, a, b, c, out); break;
    case BF16: hipLaunchKernelGGL(elementwise_kernel<BF16>, g, t, 0, s, op, n, d, a, b, c, out); break;
    default: hipLaunchKernelGGL(elementwise_kernel<F32>, g, t, 0, s, op, n, d, a, b, c, out); break;
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ layerSum (src/kernels/text.ts:67-84)
__global__ void layer_sum_kernel(uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w,
                                 float* out) {
  const size_t n = (size_t)tokens * dim;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const size_t t = i / dim, d = i % dim;
    float sum = 0.0f;
    for (uint32_t l = 0; l < layers; l++) sum += w[l] * x[(t * layers + l) * dim + d];
    out[i] = sum;
  }
}

hipError_t launch_layer_sum(uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w, float* out,
                            hipStream_t s) {
  const size_t n = (size_t)tokens * dim;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(layer_sum_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, tokens, layers, dim, x, w, out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ RMSNorm (src/kernels/rmsnorm.ts:13-48)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// one wave per row (d <= 1024), several rows per block
// The modulation add of src/model/block.ts:33-37 folded into the norm that first consumes it: scale / shift are
// the timestep vector's parts and tscale / tshift the block table's, added per value as the separate add pass would
// (scale[i] + tscale[i], one f32 add, the same bits); the launch also writes mo = ma + mb (the six vectors, for the
// later consumers), spread over its threads. All NULL: plain norm.
struct NormMod {
  const float* tscale;
  const float* tshift;
  const float* ma;
  const float* mb;
  float* mo;
  uint32_t mn;
};

__device__ __forceinline__ void norm_mod_side(const NormMod& md) {
  if (!md.mo) return;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < md.mn; j += stride) md.mo[j] = md.ma[j] + md.mb[j];
}

__device__ __forceinline__ float mod_part(const float* p, const float* t, uint32_t i) {
  return p ? (t ? p[i] + t[i] : p[i]) : 0.0f;
}

template <int DT>
__global__ void __launch_bounds__(256) rmsnorm_wave_kernel(uint32_t rows, uint32_t d, float eps, float offset,
                                                          const void* x, const float* weight, const float* scale,
                                                          const float* shift, void* out, NormMod md) {
  norm_mod_side(md);
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const size_t base = (size_t)row * d;
  float v[16];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t i = lane + 64 * j;
    v[j] = i < d ? load_as_f32<DT>(x, base + i) : 0.0f;
    ss += v[j] * v[j];
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)d + eps);
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t i = lane + 64 * j;
    if (i < d) {
      const float sc = mod_part(scale, md.tscale, i), sh = mod_part(shift, md.tshift, i);
      store_from_f32<DT>(out, base + i, v[j] * inv * (offset + weight[i]) * (1.0f + sc) + sh);
    }
  }
}

// one 256-thread block per row (any d)
template <int DT>
__global__ void __launch_bounds__(256) rmsnorm_block_kernel(uint32_t rows, uint32_t d, float eps, float offset,
                                                           const void* x, const float* weight, const float* scale,
                                                           const float* shift, void* out, NormMod md) {
  norm_mod_side(md);
  __shared__ float part[4];
  const uint32_t row = blockIdx.x;
  const size_t base = (size_t)row * d;
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < d; i += 256) {
    const float v = load_as_f32<DT>(x, base + i);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = 1.0f / sqrtf(tot / (float)d + eps);
  for (uint32_t i = threadIdx.x; i < d; i += 256) {
    const float sc = mod_part(scale, md.tscale, i), sh = mod_part(shift, md.tshift, i);
    store_from_f32<DT>(out, base + i, load_as_f32<DT>(x, base + i) * inv * (offset + weight[i]) * (1.0f + sc) + sh);
  }
}

// 16-bit rows with d a multiple of 8 (up to 8 * 64 * NCH): one wave per row, 16-byte loads and stores, the
// row held in registers between the sum of squares and the scaling (x is read once). Same per-value
// expression as the kernels above; weight / scale / shift are read as f32x4.
template <int DT, int NCH>
__global__ void __launch_bounds__(256) rmsnorm_vec_kernel(uint32_t rows, uint32_t d, float eps, float offset,
                                                         const u32x4* x, const float* weight, const float* scale,
                                                         const float* shift, u32x4* out, NormMod md) {
  norm_mod_side(md);
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint32_t nc = d / 8;
  const u32x4* xr = x + (size_t)row * nc;
  u32x4* orow = out + (size_t)row * nc;
  float v[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < NCH; q++) {
    const uint32_t c = lane + 64 * q;
    const u32x4 r = c < nc ? xr[c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint16_t hbits = (uint16_t)(r[e / 2] >> (16 * (e % 2)));
      v[q][e] = DT == BF16 ? bf16_to_f32(hbits) : f16_to_f32(hbits);
      ss += v[q][e] * v[q][e];
    }
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)d + eps);
  const std::integral_constant<bool, DT == F16> tag;
#pragma unroll
  for (int q = 0; q < NCH; q++) {
    const uint32_t c = lane + 64 * q;
    if (c >= nc) continue;
    float w[8], sc[8], sh[8];
    *(f32x4*)&w[0] = *(const f32x4*)(weight + 8 * c);
    *(f32x4*)&w[4] = *(const f32x4*)(weight + 8 * c + 4);
#pragma unroll
    for (int e = 0; e < 8; e++) sc[e] = sh[e] = 0.0f;
    if (scale) {
      *(f32x4*)&sc[0] = *(const f32x4*)(scale + 8 * c);
      *(f32x4*)&sc[4] = *(const f32x4*)(scale + 8 * c + 4);
      if (md.tscale) {
        *(f32x4*)&sc[0] += *(const f32x4*)(md.tscale + 8 * c);
        *(f32x4*)&sc[4] += *(const f32x4*)(md.tscale + 8 * c + 4);
      }
    }
    if (shift) {
      *(f32x4*)&sh[0] = *(const f32x4*)(shift + 8 * c);
      *(f32x4*)&sh[4] = *(const f32x4*)(shift + 8 * c + 4);
      if (md.tshift) {
        *(f32x4*)&sh[0] += *(const f32x4*)(md.tshift + 8 * c);
        *(f32x4*)&sh[4] += *(const f32x4*)(md.tshift + 8 * c + 4);
      }
    }
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = v[q][e] * inv * (offset + w[e]) * (1.0f + sc[e]) + sh[e];
    orow[c] = u32x4{pack2(y[0], y[1], tag), pack2(y[2], y[3], tag), pack2(y[4], y[5], tag), pack2(y[6], y[7], tag)};
  }
}

// rmsnorm_vec_kernel with the per-column factors staged once per workgroup in LDS: offset + weight, 1 + scale
// (+ the modulation's scale) and shift (+ its shift), as f32 [d] each (12 * d bytes of dynamic LDS). In
// rmsnorm_vec_kernel every wave-row loads all five f32 parameter vectors (ten 16-byte loads per 8 values beside one
// of x), which made the texture addresser, not HBM, its limit (15.1 us for 4096 x 3072 bf16 with the modulation,
// against 9.7 us for the plain norm that moves the same bytes); here the WPG rows of a workgroup share one load of
// them. The per-value expression is the same (y = v * inv * (offset + w) * (1 + sc) + sh, sc and sh summed as there),
// so the results are bit for bit those of rmsnorm_vec_kernel. Wave w of the workgroup takes row WPG * blockIdx.x + w.
constexpr uint32_t RMS_LDS_MAXD = 4096;

template <int DT, int NCH, int WPG>
__global__ void __launch_bounds__(64 * WPG) rmsnorm_lds_kernel(uint32_t rows, uint32_t d, float eps, float offset,
                                                              const u32x4* x, const float* weight, const float* scale,
                                                              const float* shift, u32x4* out, NormMod md) {
  extern __shared__ f32x4 rms_lds[];
  f32x4* fw = rms_lds;
  f32x4* fs = rms_lds + d / 4;
  f32x4* fh = rms_lds + d / 2;
  norm_mod_side(md);
  const uint32_t row = blockIdx.x * WPG + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const uint32_t nc = d / 8;
  // the row's x first, so its loads are in flight while the factors are staged
  u32x4 r[NCH];
#pragma unroll
  for (int q = 0; q < NCH; q++) {
    const uint32_t c = lane + 64 * q;
    r[q] = row < rows && c < nc ? x[(size_t)row * nc + c] : u32x4{0u, 0u, 0u, 0u};
  }
  for (uint32_t j = threadIdx.x; j < d / 4; j += 64 * WPG) {
    const f32x4 w = *(const f32x4*)(weight + 4 * j);
    f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f}, sh = {0.0f, 0.0f, 0.0f, 0.0f};
    if (scale) {
      sc = *(const f32x4*)(scale + 4 * j);
      if (md.tscale) sc += *(const f32x4*)(md.tscale + 4 * j);
    }
    if (shift) {
      sh = *(const f32x4*)(shift + 4 * j);
      if (md.tshift) sh += *(const f32x4*)(md.tshift + 4 * j);
    }
    fw[j] = offset + w;
    fs[j] = 1.0f + sc;
    fh[j] = sh;
  }
  __syncthreads();
  if (row >= rows) return;
  float v[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < NCH; q++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint16_t hbits = (uint16_t)(r[q][e / 2] >> (16 * (e % 2)));
      v[q][e] = DT == BF16 ? bf16_to_f32(hbits) : f16_to_f32(hbits);
      ss += v[q][e] * v[q][e];
    }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)d + eps);
  const std::integral_constant<bool, DT == F16> tag;
  u32x4* orow = out + (size_t)row * nc;
#pragma unroll
  for (int q = 0; q < NCH; q++) {
    const uint32_t c = lane + 64 * q;
    if (c >= nc) continue;
    float y[8];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const f32x4 w = fw[2 * c + h], sc = fs[2 * c + h], sh = fh[2 * c + h];
#pragma unroll
      for (int e = 0; e < 4; e++) y[4 * h + e] = v[q][4 * h + e] * inv * w[e] * sc[e] + sh[e];
    }
    orow[c] = u32x4{pack2(y[0], y[1], tag), pack2(y[2], y[3], tag), pack2(y[4], y[5], tag), pack2(y[6], y[7], tag)};
  }
}

template <int DT>
static bool rmsnorm_vec(uint32_t rows, uint32_t d, float eps, float offset, const void* x, const float* w,
                        const float* sc, const float* sh, void* out, const NormMod& md, hipStream_t s) {
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (d % 8 || d > 8 * 64 * 12 || !a16(x) || !a16(out) || !a16(w) || !a16(sc) || !a16(sh) || !a16(md.tscale) ||
      !a16(md.tshift))
    return false;
  const dim3 g((rows + 3) / 4), t(256);
  const uint32_t nch = (d / 8 + 63) / 64;
  const u32x4 *xv = (const u32x4*)x;
  u32x4* ov = (u32x4*)out;
  if (d <= RMS_LDS_MAXD) {
    // 8 rows (waves) per workgroup; 16 once every CU gets a workgroup of 16 (10.4 vs 10.7 us at 4096 x 3072, while
    // at 512 rows the 16-row groups leave CUs idle: 6.2 vs 4.9 us)
    const uint32_t lds = 12 * d;
    const bool w16 = rows >= 4096;
    const dim3 gl(w16 ? (rows + 15) / 16 : (rows + 7) / 8), tl(w16 ? 1024 : 512);
    if (w16) {
      if (nch <= 4) hipLaunchKernelGGL((rmsnorm_lds_kernel<DT, 4, 16>), gl, tl, lds, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
      else if (nch <= 6) hipLaunchKernelGGL((rmsnorm_lds_kernel<DT, 6, 16>), gl, tl, lds, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
      else hipLaunchKernelGGL((rmsnorm_lds_kernel<DT, 8, 16>), gl, tl, lds, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
    } else {
      if (nch <= 4) hipLaunchKernelGGL((rmsnorm_lds_kernel<DT, 4, 8>), gl, tl, lds, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
      else if (nch <= 6) hipLaunchKernelGGL((rmsnorm_lds_kernel<DT, 6, 8>), gl, tl, lds, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
      else hipLaunchKernelGGL((rmsnorm_lds_kernel<DT, 8, 8>), gl, tl, lds, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
    }
    return true;
  }
  // 4096 < d <= 6144: the factors would not leave room in LDS for more than one or two workgroups per CU
  hipLaunchKernelGGL((rmsnorm_vec_kernel<DT, 12>), g, t, 0, s, rows, d, eps, offset, xv, w, sc, sh, ov, md);
  return true;
}

template <int DT>
static void rmsnorm_dt(uint32_t rows, uint32_t d, float eps, float offset, const void* x, const float* w,
                       const float* sc, const float* sh, void* out, const NormMod& md, hipStream_t s) {
  if constexpr (DT != F32) {
    if (d > 1024 && rmsnorm_vec<DT>(rows, d, eps, offset, x, w, sc, sh, out, md, s)) return;
  }
  if (d <= 1024)
    hipLaunchKernelGGL(rmsnorm_wave_kernel<DT>, dim3((rows + 3) / 4), dim3(256), 0, s, rows, d, eps, offset, x, w, sc, sh,
                       out, md);
  else
    hipLaunchKernelGGL(rmsnorm_block_kernel<DT>, dim3(rows), dim3(256), 0, s, rows, d, eps, offset, x, w, sc, sh, out,
                       md);
}

static hipError_t rmsnorm_any(uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                              const float* weight, const float* scale, const float* shift, void* out, const NormMod& md,
                              hipStream_t s) {
  if (rows == 0 || d == 0) return hipSuccess;
  switch (dtype) {
    case F16: rmsnorm_dt<F16>(rows, d, eps, offset, x, weight, scale, shift, out, md, s); break;
    case BF16: rmsnorm_dt<BF16>(rows, d, eps, offset, x, weight, scale, shift, out, md, s); break;
    default: rmsnorm_dt<F32>(rows, d, eps, offset, x, weight, scale, shift, out, md, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm(uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                          const float* weight, const float* scale, const float* shift, void* out, hipStream_t s) {
  return rmsnorm_any(rows, d, eps, offset, dtype, x, weight, scale, shift, out, NormMod{}, s);
}

// mod = tvec + table (mod_n values) and out = rmsnorm(x) modulated by (tvec + table)[0:d] / [d:2d], one launch
// (rows >= 1 and d >= 1: the caller checks)
hipError_t launch_rmsnorm_mod(uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                              const float* weight, const float* tvec, const float* table, uint32_t mod_n, float* mod,
                              void* out, hipStream_t s) {
  const NormMod md{table, table + d, tvec, table, mod, mod_n};
  return rmsnorm_any(rows, d, eps, offset, dtype, x, weight, tvec, tvec + d, out, md, s);
}

// ------------------------------------------------------------------ RoPE (src/kernels/rope.ts:45-77)
template <int DT>
__global__ void rope_kernel(uint32_t tokens, uint32_t heads, uint32_t pairs, int half, const void* x, const float* cs,
                            const float* sn, void* out) {
  const size_t total = (size_t)tokens * heads * pairs;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t j = i % pairs, th = i / pairs, t = th / heads;
    const float c = cs[t * pairs + j], s = sn[t * pairs + j];
    size_t ia, ib;
    if (!half) {
      ia = 2 * i;
      ib = 2 * i + 1;
    } else {
      ia = th * pairs * 2 + j;
      ib = ia + pairs;
    }
    const float a = load_as_f32<DT>(x, ia), b = load_as_f32<DT>(x, ib);
    store_from_f32<DT>(out, ia, a * c - b * s);
    store_from_f32<DT>(out, ib, b * c + a * s);
  }
}

hipError_t launch_rope(uint32_t tokens, uint32_t heads, uint32_t pairs, int half, int dtype, const void* x,
                       const float* c, const float* sn, void* out, hipStream_t s) {
  const size_t n = (size_t)tokens * heads * pairs;
  if (n == 0) return hipSuccess;
  const dim3 g(grid_for(n, 256)), t(256);
  switch (dtype) {
    case F16: hipLaunchKernelGGL(rope_kernel<F16>, g, t, 0, s, tokens, heads, pairs, half, x, c, sn, out); break;
    case BF16: hipLaunchKernelGGL(rope_kernel<BF16>, g, t, 0, s, tokens, heads, pairs, half, x, c, sn, out); break;
    default: hipLaunchKernelGGL(rope_kernel<F32>, g, t, 0, s, tokens, heads, pairs, half, x, c, sn, out); break;
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ fused per-head RMSNorm + RoPE
// One wave per (token, head) row of head_dim = 2 * pairs values (pairs <= 256): lane l owns pairs
// l, l + 64, ..., so both values of each of its pairs are in its registers (interleaved: 2j, 2j+1;
// half: j, j + pairs). Tokens below rope_from are only normalized; cos/sin row = token - rope_from.
// Token t's heads start at t * xs (input) and t * os (output) elements.
template <int DT>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(uint32_t tokens, uint32_t heads, uint32_t head_dim,
                                                          float eps, float offset, const float* weight,
                                                          uint32_t rope_from, int half, const float* cs,
                                                          const float* sn, const void* x, uint32_t xs, void* out,
                                                          uint32_t os) {
  const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (size_t)tokens * heads) return;
  const uint32_t t = (uint32_t)(row / heads), hh = (uint32_t)(row % heads);
  const uint32_t pairs = head_dim / 2;
  const size_t base = (size_t)t * xs + (size_t)hh * head_dim;
  const size_t obase = (size_t)t * os + (size_t)hh * head_dim;
  float va[4], vb[4];
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t j = lane + 64 * q;
    if (j < pairs) {
      const uint32_t ia = half ? j : 2 * j, ib = half ? j + pairs : 2 * j + 1;
      va[q] = load_as_f32<DT>(x, base + ia);
      vb[q] = load_as_f32<DT>(x, base + ib);
    } else {
      va[q] = vb[q] = 0.0f;
    }
    ss += va[q] * va[q] + vb[q] * vb[q];
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)head_dim + eps);
  const bool rot = t >= rope_from;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t j = lane + 64 * q;
    if (j >= pairs) continue;
    const uint32_t ia = half ? j : 2 * j, ib = half ? j + pairs : 2 * j + 1;
    const float a = va[q] * inv * (offset + weight[ia]);
    const float b = vb[q] * inv * (offset + weight[ib]);
    float ra = a, rb = b;
    if (rot) {
      const size_t ti = (size_t)(t - rope_from) * pairs + j;
      const float c = cs[ti], s = sn[ti];
      ra = a * c - b * s;
      rb = b * c + a * s;
    }
    store_from_f32<DT>(out, obase + ia, ra);
    store_from_f32<DT>(out, obase + ib, rb);
  }
}

// Head dim 128, interleaved pairs, 16-bit values, 16-byte aligned rows: 16 lanes per (token, head) row, lane
// l holding values 8l .. 8l + 7 (pairs 4l .. 4l + 3) in one 16-byte load; four rows per wave. Same per-value
// expressions as qk_norm_rope_kernel.
template <int DT>
__global__ void __launch_bounds__(256) qk_norm_rope_vec_kernel(uint32_t tokens, uint32_t heads, float eps, float offset,
                                                              const float* weight, uint32_t rope_from, const float* cs,
                                                              const float* sn, const uint16_t* x, uint32_t xs,
                                                              uint16_t* out, uint32_t os) {
  const size_t row = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  const bool valid = row < (size_t)tokens * heads;
  const uint32_t t = valid ? (uint32_t)(row / heads) : 0u, hh = valid ? (uint32_t)(row % heads) : 0u;
  const size_t base = (size_t)t * xs + (size_t)hh * 128 + 8 * l;
  const u32x4 r = valid ? *(const u32x4*)(x + base) : u32x4{0u, 0u, 0u, 0u};
  float v[8];
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const uint16_t hbits = (uint16_t)(r[e / 2] >> (16 * (e % 2)));
    v[e] = DT == BF16 ? bf16_to_f32(hbits) : f16_to_f32(hbits);
  }
#pragma unroll
  for (int p = 0; p < 4; p++) ss += v[2 * p] * v[2 * p] + v[2 * p + 1] * v[2 * p + 1];
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);  // the 16 lanes of the row
  if (!valid) return;
  const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
  float w[8];
  *(f32x4*)&w[0] = *(const f32x4*)(weight + 8 * l);
  *(f32x4*)&w[4] = *(const f32x4*)(weight + 8 * l + 4);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; e++) y[e] = v[e] * inv * (offset + w[e]);
  if (t >= rope_from) {
    const size_t ti = (size_t)(t - rope_from) * 64 + 4 * l;
    const f32x4 c4 = *(const f32x4*)(cs + ti), s4 = *(const f32x4*)(sn + ti);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const float a = y[2 * p], b = y[2 * p + 1];
      y[2 * p] = a * c4[p] - b * s4[p];
      y[2 * p + 1] = b * c4[p] + a * s4[p];
    }
  }
  const std::integral_constant<bool, DT == F16> tag;
  *(u32x4*)(out + (size_t)t * os + (size_t)hh * 128 + 8 * l) =
      u32x4{pack2(y[0], y[1], tag), pack2(y[2], y[3], tag), pack2(y[4], y[5], tag), pack2(y[6], y[7], tag)};
}

hipError_t launch_qk_norm_rope(uint32_t tokens, uint32_t heads, uint32_t head_dim, float eps, float offset,
                               const float* weight, uint32_t rope_from, int half, const float* c, const float* sn,
                               int dtype, const void* x, uint32_t xs, void* out, uint32_t os, hipStream_t s) {
  const size_t rows = (size_t)tokens * heads;
  if (rows == 0) return hipSuccess;
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if ((dtype == BF16 || dtype == F16) && head_dim == 128 && !half && xs % 8 == 0 && os % 8 == 0 && a16(x) &&
      a16(out) && a16(weight) && a16(c) && a16(sn)) {
    const dim3 g((unsigned)((rows + 15) / 16)), t(256);
    if (dtype == BF16)
      hipLaunchKernelGGL(qk_norm_rope_vec_kernel<BF16>, g, t, 0, s, tokens, heads, eps, offset, weight, rope_from, c, sn,
                         (const uint16_t*)x, xs, (uint16_t*)out, os);
    else
      hipLaunchKernelGGL(qk_norm_rope_vec_kernel<F16>, g, t, 0, s, tokens, heads, eps, offset, weight, rope_from, c, sn,
                         (const uint16_t*)x, xs, (uint16_t*)out, os);
    return hipGetLastError();
  }
  const dim3 g((unsigned)((rows + 3) / 4)), t(256);
  switch (dtype) {
    case F16:
      hipLaunchKernelGGL(qk_norm_rope_kernel<F16>, g, t, 0, s, tokens, heads, head_dim, eps, offset, weight, rope_from,
                         half, c, sn, x, xs, out, os);
      break;
    case BF16:
      hipLaunchKernelGGL(qk_norm_rope_kernel<BF16>, g, t, 0, s, tokens, heads, head_dim, eps, offset, weight, rope_from,
                         half, c, sn, x, xs, out, os);
      break;
    default:
      hipLaunchKernelGGL(qk_norm_rope_kernel<F32>, g, t, 0, s, tokens, heads, head_dim, eps, offset, weight, rope_from,
                         half, c, sn, x, xs, out, os);
      break;
  }
  return hipGetLastError();
}

}  // namespace we
