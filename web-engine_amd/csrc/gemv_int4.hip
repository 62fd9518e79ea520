// int4-weight GEMV / skinny GEMM on gfx950 (decode shapes, M <= 32 per launch row-block):
//   y[m, n] = scale * sum_g s[n, g] * sum_{k in g} x[m, k] * q[n, k]
// W: u32 [N, K/8], eight two's-complement nibbles per word along K (low nibble = lowest k);
// s: f16 [N, K/group]. The per-group scale multiplies the f32 partial sum of that group, so the
// dequantized value q * s is never rounded to 16 bits.
//
// Work split: a workgroup of 4 waves owns 32 output columns n and one block of 32 rows m; the four
// waves split K (a wavefront-level split-K) and their f32 partials are summed through LDS.
// Inside a wave the MFMA 32x32x16 runs with x as the A operand (rows m) and W as the B operand
// (columns n): lane l holds row n0 + l % 32 of W and, for each 64-k block, one 16-byte load of
// words [8b + 4h, 8b + 4h + 4) (h = l / 32). MFMA j of the block consumes word j, so its k-slot h
// maps to k = 64b + 32h + 8j .. +8; the x fragment is read from the same k. Every W byte is loaded
// exactly once, all loads of a wave are issued before the first MFMA needs them, and the 16 nibbles
// of a dword pair are unpacked in registers (f16: byte-permute + mask + one packed FMA per pair).
#include "common.h"
#include "internal.h"

namespace we {

struct Int4Args {
  const void* x;
  const uint32_t* w;
  const uint16_t* s;
  void* y;
  const float* bias;
  uint32_t m, n, k, group;
  float scale;
  uint32_t x_stride, y_stride, x_offset, y_offset;
  uint32_t flags, y_dtype;
};

// eight nibbles (one word) -> eight f16 in k order, exact
__device__ __forceinline__ u32x4 int4x8_to_f16(uint32_t w) {
  const uint32_t u = w ^ 0x88888888u;  // q + 8 in [0, 15] per nibble
  const f16x2 mul = {(_Float16)1.0f, (_Float16)0.0625f};
  const f16x2 add = {(_Float16)-1032.0f, (_Float16)-72.0f};
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    // byte p of u into bytes 0 and 2: lo half gets nibble 2p at bits 0-3, hi half nibble 2p+1 at bits 4-7
    const uint32_t sel = (uint32_t)p | (0x0cu << 8) | ((uint32_t)p << 16) | (0x0cu << 24);
    const uint32_t t = __builtin_amdgcn_perm(u, u, sel);
    const uint32_t v = (t & 0x00f0000fu) | 0x64006400u;  // lo: 1024 + u0, hi: 1024 + 16 u1
    const f16x2 h = __builtin_bit_cast(f16x2, v);
    const f16x2 q = __builtin_elementwise_fma(h, mul, add);  // lo: u0 - 8, hi: u1 - 8
    r[p] = __builtin_bit_cast(uint32_t, q);
  }
  return r;
}

// eight nibbles -> eight bf16 in k order, exact (small integers)
__device__ __forceinline__ u32x4 int4x8_to_bf16(uint32_t w) {
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const int lo = ((int)(w << (28 - 8 * p))) >> 28;
    const int hi = ((int)(w << (24 - 8 * p))) >> 28;
    const uint32_t a = __float_as_uint((float)lo), b = __float_as_uint((float)hi);
    r[p] = (a >> 16) | (b & 0xffff0000u);
  }
  return r;
}

template <int XT>
__device__ __forceinline__ void load_x_frag(const Int4Args& a, bool m_ok, size_t xrow, uint32_t k, u32x4 (&out)[4][2]) {
  // 32 consecutive k of one row: 4 fragments of 8 (one per MFMA j); f32 rows give hi + lo bf16 planes
  if (!m_ok) {
#pragma unroll
    for (int j = 0; j < 4; j++) out[j][0] = out[j][1] = u32x4{0, 0, 0, 0};
    return;
  }
  if constexpr (XT == F32) {
    const u32x4* p = (const u32x4*)((const float*)a.x + xrow + k);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const u32x4 v0 = p[2 * j], v1 = p[2 * j + 1];
      float f[8] = {__uint_as_float(v0.x), __uint_as_float(v0.y), __uint_as_float(v0.z), __uint_as_float(v0.w),
                    __uint_as_float(v1.x), __uint_as_float(v1.y), __uint_as_float(v1.z), __uint_as_float(v1.w)};
      uint32_t hi[8], lo[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        hi[e] = f32_to_bf16(f[e]);
        lo[e] = f32_to_bf16(f[e] - bf16_to_f32((uint16_t)hi[e]));
      }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        out[j][0][e] = hi[2 * e] | (hi[2 * e + 1] << 16);
        out[j][1][e] = lo[2 * e] | (lo[2 * e + 1] << 16);
      }
    }
  } else {
    const u32x4* p = (const u32x4*)((const uint16_t*)a.x + xrow + k);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      out[j][0] = p[j];
      out[j][1] = u32x4{0, 0, 0, 0};
    }
  }
}

constexpr int INT4_PF = 8;  // 64-k blocks of W prefetched per wave at a time

template <int XT>
__global__ void __launch_bounds__(256) int4_gemv_kernel(Int4Args a) {
  constexpr bool IS_F16 = XT == F16;
  constexpr int NA = XT == F32 ? 2 : 1;
  __shared__ float red[4][16][64];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const uint32_t n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  const uint32_t n = n0 + l32, m = m0 + l32;
  const bool n_ok = n < a.n, m_ok = m < a.m;
  const uint32_t nblk = a.k / 64;
  const uint32_t per = (nblk + 3) / 4;
  const uint32_t b0 = min(nblk, wave * per), b1 = min(nblk, b0 + per);
  const uint32_t words_per_row = a.k / 8, groups_per_row = a.k / a.group;
  const u32x4* wrow = (const u32x4*)(a.w + (size_t)(n_ok ? n : 0) * words_per_row) + h;  // + 2 per block
  const uint16_t* srow = a.s + (size_t)(n_ok ? n : 0) * groups_per_row;
  const size_t xrow = (size_t)a.x_offset + (size_t)(m_ok ? m : 0) * a.x_stride;

  f32x16 acc = {};
  u32x4 wq[INT4_PF];
  auto fetch = [&](uint32_t first) {
#pragma unroll
    for (int i = 0; i < INT4_PF; i++) {
      const uint32_t b = first + i;
      wq[i] = (n_ok && b < b1) ? __builtin_nontemporal_load(wrow + 2 * (size_t)b) : u32x4{0, 0, 0, 0};
    }
  };
  if (b0 < b1) fetch(b0);
  for (uint32_t c = b0; c < b1; c += INT4_PF) {
    u32x4 cur[INT4_PF];
#pragma unroll
    for (int i = 0; i < INT4_PF; i++) cur[i] = wq[i];
    if (c + INT4_PF < b1) fetch(c + INT4_PF);
#pragma unroll
    for (int i = 0; i < INT4_PF; i++) {
      const uint32_t b = c + i;
      if (b >= b1) break;
      const float s = n_ok ? f16_to_f32(srow[(b * 64) / a.group]) : 0.0f;
      u32x4 xf[4][2];
      load_x_frag<XT>(a, m_ok, xrow, b * 64 + h * 32, xf);
      f32x16 part = {};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const u32x4 wf = IS_F16 ? int4x8_to_f16(cur[i][j]) : int4x8_to_bf16(cur[i][j]);
#pragma unroll
        for (int p = 0; p < NA; p++) part = mfma_32x32x16<IS_F16>(xf[j][p], wf, part);
      }
#pragma unroll
      for (int v = 0; v < 16; v++) acc[v] += part[v] * s;
    }
  }

#pragma unroll
  for (int v = 0; v < 16; v++) red[wave][v][lane] = acc[v];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int idx = threadIdx.x * 4 + e;  // 0 .. 1023
    const int v = idx >> 6, ln = idx & 63;
    const float sum = red[0][v][ln] + red[1][v][ln] + red[2][v][ln] + red[3][v][ln];
    const uint32_t row = m0 + 8 * (v / 4) + 4 * (ln >> 5) + (v % 4);
    const uint32_t col = n0 + (ln & 31);
    if (row >= a.m || col >= a.n) continue;
    float val = sum * a.scale;
    if (a.flags & WE_EPI_BIAS_BIT) val += a.bias[col];
    if (a.flags & WE_EPI_GELU_BIT) val = gelu_tanh(val);
    const size_t o = (size_t)a.y_offset + (size_t)row * a.y_stride + col;
    if (a.y_dtype == F32) {
      float* y = (float*)a.y;
      y[o] = (a.flags & WE_EPI_ACCUMULATE_BIT) ? y[o] + val : val;
    } else if (a.y_dtype == BF16) {
      uint16_t* y = (uint16_t*)a.y;
      y[o] = f32_to_bf16((a.flags & WE_EPI_ACCUMULATE_BIT) ? bf16_to_f32(y[o]) + val : val);
    } else {
      uint16_t* y = (uint16_t*)a.y;
      y[o] = f32_to_f16((a.flags & WE_EPI_ACCUMULATE_BIT) ? f16_to_f32(y[o]) + val : val);
    }
  }
}

hipError_t int4_launch(const Int4Launch& L, hipStream_t stream) {
  Int4Args a{};
  a.x = L.x;
  a.w = L.w;
  a.s = L.scales;
  a.y = L.y;
  a.bias = L.bias;
  a.m = L.m;
  a.n = L.n;
  a.k = L.k;
  a.group = L.group;
  a.scale = L.scale;
  a.x_stride = L.x_stride;
  a.y_stride = L.y_stride;
  a.x_offset = L.x_offset;
  a.y_offset = L.y_offset;
  a.flags = L.flags;
  a.y_dtype = (uint32_t)L.y_dtype;
  dim3 grid((L.n + 31) / 32, (L.m + 31) / 32);
  switch (L.x_dtype) {
    case F16: hipLaunchKernelGGL(int4_gemv_kernel<F16>, grid, dim3(256), 0, stream, a); break;
    case BF16: hipLaunchKernelGGL(int4_gemv_kernel<BF16>, grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(int4_gemv_kernel<F32>, grid, dim3(256), 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace we
