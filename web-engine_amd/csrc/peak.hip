// Peak probes: timePeak (src/bench/peak.ts:69-109) on gfx950, plus the two ceilings the matmul path is
// measured against: dense bf16 MFMA and a streaming HBM read.
//
// Math kinds follow the reference: every thread runs PEAK_CHAINS = 8 independent chains for `iters`
// iterations, 64 operations per thread per iteration:
//   F32: 8 chains x 4 fma (2 ops each) in f32 (scalar v_fma_f32: the library compiles without packed f32
//        math, so the probe reports the scalar-FMA ceiling, half the packed-FMA figure MI355X publishes);
//   F16: 8 chains x 2 packed fma (v_pk_fma_f16, 4 ops each);
//   I8:  8 chains x dot4 of int8 (v_dot4_i32_i8, 4 multiply-adds = 8 ops);
//   MFMA_BF16: per wave 8 chains of v_mfma_f32_32x32x16_bf16 (32768 FLOP each) per iteration, i.e. 4096 FLOP
//        per thread per iteration, on small constant operands;
//   MFMA_BF16_DATA: the same work on v_mfma_f32_16x16x32_bf16 (the shape of the GEMM's ping-pong tiles; two per
//        32x32x16 of the loop above) on operands with the fp8-weight GEMM's bit statistics: A as its activations
//        (bf16 of N(0,1)-like magnitude, every mantissa bit random), B as its weights (the bf16 images of random
//        finite e4m3fn codes, decoded by the hardware converter), 8 operand pairs per lane rotated so that
//        consecutive MFMAs of a chain see different data. The chip runs at its power limit under the GEMM, and
//        the power of an MFMA grows with the bits that toggle in its operands (and with the accumulator bits it
//        moves: 32x32x16 reaches about 10% less here): this is the ceiling of the matmul's MFMA loop on the data
//        it is measured with.
// The chains start from the thread id so no value is a compile-time constant, and every result is folded
// into out[thread] so nothing is removed. b = 0.5 and c = 0.25 keep the float chains exact (and finite).
#include "common.h"
#include "internal.h"

namespace we {
namespace {

constexpr int PEAK_CHAINS = 8;
typedef float f32x16_p __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(64) peak_f32(uint32_t iters, float b, float c, uint32_t* out) {
  const uint32_t id = blockIdx.x * 64 + threadIdx.x;
  float a[PEAK_CHAINS][4];
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) a[j][e] = (float)(id % 16u) + (float)j;
  for (uint32_t i = 0; i < iters; i++)
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) a[j][e] = __builtin_fmaf(a[j][e], b, c);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++) s += a[j][0] + a[j][1] + a[j][2] + a[j][3];
  out[id] = __float_as_uint(s);
}

__global__ void __launch_bounds__(64) peak_f16(uint32_t iters, float bf, float cf, uint32_t* out) {
  const uint32_t id = blockIdx.x * 64 + threadIdx.x;
  const f16x2 b = {(_Float16)bf, (_Float16)bf}, c = {(_Float16)cf, (_Float16)cf};
  f16x2 a[PEAK_CHAINS][2];
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
    for (int e = 0; e < 2; e++) a[j][e] = f16x2{(_Float16)((float)(id % 16u) + j), (_Float16)((float)(id % 16u) + j)};
  for (uint32_t i = 0; i < iters; i++)
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
      for (int e = 0; e < 2; e++) a[j][e] = __builtin_elementwise_fma(a[j][e], b, c);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++) s += (float)a[j][0].x + (float)a[j][0].y + (float)a[j][1].x + (float)a[j][1].y;
  out[id] = __float_as_uint(s);
}

__global__ void __launch_bounds__(64) peak_i8(uint32_t iters, uint32_t y, uint32_t* out) {
  const uint32_t id = blockIdx.x * 64 + threadIdx.x;
  int a[PEAK_CHAINS];
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++) a[j] = (int)(id % 16u) + j;
  for (uint32_t i = 0; i < iters; i++)
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) a[j] = __builtin_amdgcn_sdot4(a[j], (int)y, a[j], false);
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++) s += (uint32_t)a[j];
  out[id] = s;
}

__global__ void __launch_bounds__(256) peak_mfma_bf16(uint32_t iters, uint32_t* out) {
  const uint32_t id = blockIdx.x * 256 + threadIdx.x;
  // operands: small exact bf16 values from the lane id (0.5 .. 2), the same every iteration
  u32x4 ra, rb;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    ra[e] = 0x3f003f00u + ((id + e) & 7u) * 0x00100010u;
    rb[e] = 0x3f803f80u + ((id >> 3) & 3u) * 0x00100010u;
  }
  const bf16x8 a = __builtin_bit_cast(bf16x8, ra), b = __builtin_bit_cast(bf16x8, rb);
  f32x16_p acc[PEAK_CHAINS];
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++) acc[j] = f32x16_p{};
  for (uint32_t i = 0; i < iters; i++)
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) s += acc[j][v];
  out[id] = __float_as_uint(s);
}

__device__ __forceinline__ uint32_t peak_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  return x ^ (x >> 16);
}

__global__ void __launch_bounds__(256) peak_mfma_bf16_data(uint32_t iters, uint32_t* out) {
  const uint32_t id = blockIdx.x * 256 + threadIdx.x;
  u32x4 ra[PEAK_CHAINS], rb[PEAK_CHAINS];
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t h = peak_hash(id * 64u + (uint32_t)(j * 4 + e) * 2u);
      // two bf16: random sign and 7 mantissa bits, exponents 124 .. 127 (|v| in [0.125, 2))
      const uint32_t lo = (h & 0x807fu) | ((124u + ((h >> 7) & 3u)) << 7);
      const uint32_t hi = ((h >> 16) & 0x807fu) | ((124u + ((h >> 23) & 3u)) << 7);
      ra[j][e] = lo | (hi << 16);
    }
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      // four random finite e4m3fn codes (0x7f / 0xff, the NaN codes, become 0x7e / 0xfe) -> four bf16
      uint32_t w = peak_hash(id * 64u + (uint32_t)(j * 4 + e) * 2u + 1u);
#pragma unroll
      for (int b = 0; b < 4; b++)
        if (((w >> (8 * b)) & 0x7fu) == 0x7fu) w -= 1u << (8 * b);
      const auto lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
      const auto hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
      rb[j][e] = __builtin_bit_cast(uint32_t, lo);
      rb[j][e + 1] = __builtin_bit_cast(uint32_t, hi);
    }
  f32x4 acc[PEAK_CHAINS];
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++) acc[j] = f32x4{};
  uint32_t i = 0;
  // groups of 8 iterations: in sub-iteration s, half r, chain j multiplies A[j] with B[(j + s + r) % 8] (two
  // 16x16x32 MFMAs per chain and iteration: the 32768 FLOP of one 32x32x16)
  for (; i + PEAK_CHAINS <= iters; i += PEAK_CHAINS)
#pragma unroll
    for (int s8 = 0; s8 < PEAK_CHAINS; s8++)
#pragma unroll
      for (int r = 0; r < 2; r++)
#pragma unroll
        for (int j = 0; j < PEAK_CHAINS; j++)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ra[j]),
                                                           __builtin_bit_cast(bf16x8, rb[(j + s8 + r) % PEAK_CHAINS]),
                                                           acc[j], 0, 0, 0);
  for (; i < iters; i++)
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int j = 0; j < PEAK_CHAINS; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ra[j]),
                                                         __builtin_bit_cast(bf16x8, rb[(j + r) % PEAK_CHAINS]), acc[j], 0,
                                                         0, 0);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < PEAK_CHAINS; j++)
#pragma unroll
    for (int v = 0; v < 4; v++) s += acc[j][v];
  out[id] = __float_as_uint(s);
}

// Streaming read of n16 16-byte chunks in one shot: workgroup b reads the contiguous 32 KB block of chunks
// [b 256 U, (b + 1) 256 U), thread t the chunks t, t + 256, ... of it (each load instruction reads 1 KB of consecutive
// bytes), all in flight at once, no loop; the grid covers the buffer. It sums the words and each wave writes one sum.
// Measured on MI355X over one 34 MB buffer (graph replays, 10 rotating copies): this form 6.70 us, the same loads
// spaced by the whole grid 7.15 us, 2 or 4 times larger workgroups 7.9-8.2 us.
__global__ void __launch_bounds__(256) read_peak(const u32x4* __restrict__ p, uint64_t n16, uint32_t* out) {
  const uint64_t tid = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t base = (uint64_t)blockIdx.x * 256 * READ_PEAK_U + threadIdx.x;
  u32x4 v[READ_PEAK_U];
#pragma unroll
  for (int u = 0; u < READ_PEAK_U; u++) {
    const uint64_t i = base + (uint64_t)u * 256;
    v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
  }
  u32x4 t = v[0];
#pragma unroll
  for (int u = 1; u < READ_PEAK_U; u++) t += v[u];
  uint32_t s = t.x + t.y + t.z + t.w;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += (uint32_t)__shfl_xor((int)s, m, 64);
  if ((threadIdx.x & 63) == 0) out[tid >> 6] = s;
}

}  // namespace

hipError_t peak_launch(int kind, uint32_t workgroups, uint32_t iters, uint32_t* out, hipStream_t stream) {
  switch (kind) {
    case PEAK_F32: hipLaunchKernelGGL(peak_f32, dim3(workgroups), dim3(64), 0, stream, iters, 0.5f, 0.25f, out); break;
    case PEAK_F16: hipLaunchKernelGGL(peak_f16, dim3(workgroups), dim3(64), 0, stream, iters, 0.5f, 0.25f, out); break;
    case PEAK_I8: hipLaunchKernelGGL(peak_i8, dim3(workgroups), dim3(64), 0, stream, iters, 0x0302ff01u, out); break;
    case PEAK_MFMA_BF16_DATA:
      hipLaunchKernelGGL(peak_mfma_bf16_data, dim3(workgroups), dim3(256), 0, stream, iters, out);
      break;
    default: hipLaunchKernelGGL(peak_mfma_bf16, dim3(workgroups), dim3(256), 0, stream, iters, out); break;
  }
  return hipGetLastError();
}

hipError_t read_peak_launch(const void* buf, uint64_t bytes, uint32_t* out, hipStream_t stream) {
  const uint64_t n16 = bytes / 16;
  const uint64_t grid = (n16 + 256ull * READ_PEAK_U - 1) / (256ull * READ_PEAK_U);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(read_peak, dim3((unsigned)grid), dim3(256), 0, stream, (const u32x4*)buf, n16, out);
  return hipGetLastError();
}

}  // namespace we
