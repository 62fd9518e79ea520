// Fast path of the gfx950 GEMM for the hot dtypes: 16-bit activations (bf16 or f16) times fp8 e4m3fn or
// 16-bit weights, fp32 accumulation on MFMA 32x32x16, y = x . W^T * scale (+ bias, gelu, accumulate,
// split-K) with the semantics of matmulWgsl (src/kernels/matmul.ts:118-178).
//
// Differences from the general kernel (gemm.hip), all about keeping the main loop straight-line:
//  * global loads are buffer loads through a buffer resource whose size is the operand's extent: a row
//    past M / N or a chunk past the K range gets an out-of-range offset and reads 0 in hardware, so no
//    lane ever branches; the k advance is the scalar offset of the load;
//  * LDS fragments of MFMA step s + 1 are read while the MFMAs of step s run;
//  * the fp8 NaN-code fix-up (the reference shader decodes 0x7f / 0xff to +-480) is decided once per
//    stage for the whole wave, so the common path has no branch between MFMAs.
// Requirements (checked on the host): rows 16-byte aligned, K and the split-K slice multiples of 16,
// operand extents below 2^31 bytes.
#include "common.h"
#include "internal.h"

namespace we {

namespace {

constexpr int BK = 64;
constexpr uint32_t kInvalid = 0x80000000u;  // a byte offset past every extent: the load returns 0
constexpr int kRsrcWord3 = 0x00020000;      // raw buffer, 32-bit data format (gfx9 family)

struct FastArgs {
  const void* x;
  const void* w;
  void* y;
  const float* bias;
  uint32_t x_bytes, w_bytes;  // readable bytes from x / w (their extents)
  uint32_t m, n, k;
  float scale;
  uint32_t x_stride, w_stride, y_stride, y_offset;  // x / w already point at their offsets
  uint32_t kc;
  uint32_t tiles_m, tiles_n;
  uint32_t flags, y_dtype;
};

__device__ __forceinline__ uint32_t xcd_remap_f(uint32_t pid, uint32_t total) {
  const uint32_t xcd = pid & 7u, idx = pid >> 3;
  const uint32_t base = total >> 3, rem = total & 7u;
  return xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
}

__device__ __forceinline__ void store_y(const FastArgs& a, size_t o, float val) {
  const bool acc = (a.flags & WE_EPI_ACCUMULATE_BIT) != 0;
  if (a.y_dtype == F32) {
    float* y = (float*)a.y;
    y[o] = acc ? y[o] + val : val;
  } else if (a.y_dtype == BF16) {
    uint16_t* y = (uint16_t*)a.y;
    y[o] = f32_to_bf16(acc ? bf16_to_f32(y[o]) + val : val);
  } else {
    uint16_t* y = (uint16_t*)a.y;
    y[o] = f32_to_f16(acc ? f16_to_f32(y[o]) + val : val);
  }
}

// fp8 word -> 4 x 16-bit without the NaN-code check (the caller decides that per stage)
template <bool IS_F16>
__device__ __forceinline__ u32x2 cvt_fp8x4(uint32_t w) {
  u32x2 r;
  if constexpr (IS_F16) {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
  } else {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  }
  return r;
}

}  // namespace

template <int BM, int BN, int WAVES_M, int WAVES_N, bool IS_F16, int BT>
__global__ void __launch_bounds__(WAVES_M* WAVES_N * 64) gemm_fast_kernel(FastArgs a) {
  constexpr int T = WAVES_M * WAVES_N * 64;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr bool B8 = BT == FP8;
  constexpr int A_STAGE = BM * 8;                // u32x4 chunks per stage
  constexpr int B_STAGE = B8 ? BN * 4 : BN * 8;  // u32x4 chunks per stage
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int A_IT = A_STAGE / T, B_IT = B_STAGE / T;
  static_assert(A_STAGE % T == 0 && B_STAGE % T == 0, "tile / thread mismatch");
  __shared__ u32x4 lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int half = lane >> 5, l32 = lane & 31;

  const uint32_t pid = xcd_remap_f(blockIdx.x, gridDim.x);
  constexpr uint32_t GROUP_M = 4;
  const uint32_t per_group = GROUP_M * a.tiles_n;
  const uint32_t first_m = (pid / per_group) * GROUP_M;
  const uint32_t gsize = min(a.tiles_m - first_m, GROUP_M);
  const uint32_t in_group = pid % per_group;
  const uint32_t row0 = (first_m + in_group % gsize) * BM, col0 = (in_group / gsize) * BN;

  const uint32_t z = blockIdx.y;
  const uint32_t k_begin = z * a.kc;
  const uint32_t k_end = min(a.k, k_begin + a.kc);
  const int nk = k_end > k_begin ? (int)((k_end - k_begin + BK - 1) / BK) : 0;

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)a.w_bytes, kRsrcWord3);

  // per-lane byte offsets of the chunks this thread stages (k = 0 of the row), invalid past M / N
  uint32_t offa[A_IT], offb[B_IT];
  int kca[A_IT], kcb[B_IT];  // k of the chunk inside the 64-k block
#pragma unroll
  for (int i = 0; i < A_IT; i++) {
    const int idx = i * T + tid, r = idx >> 3, c = idx & 7;
    const uint32_t row = row0 + r;
    offa[i] = row < a.m ? (row * a.x_stride + c * 8) * 2 : kInvalid;
    kca[i] = c * 8;
  }
#pragma unroll
  for (int i = 0; i < B_IT; i++) {
    const int idx = i * T + tid;
    const int r = B8 ? idx >> 2 : idx >> 3, c = B8 ? idx & 3 : idx & 7;
    const uint32_t col = col0 + r;
    offb[i] = col < a.n ? (B8 ? col * a.w_stride + c * 16 : (col * a.w_stride + c * 8) * 2) : kInvalid;
    kcb[i] = B8 ? c * 16 : c * 8;
  }

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = f32x16{};

  u32x4 ra[A_IT], rb[B_IT];
  auto load_global = [&](uint32_t kb) {
    const bool full = kb + BK <= k_end;  // uniform: only the last block of a slice can be partial
    const int sa = (int)(kb * 2), sb = (int)(B8 ? kb : kb * 2);
#pragma unroll
    for (int i = 0; i < A_IT; i++) {
      const uint32_t o = (full || kb + kca[i] < k_end) ? offa[i] : kInvalid;
      ra[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, sa, 0));
    }
#pragma unroll
    for (int i = 0; i < B_IT; i++) {
      const uint32_t o = (full || kb + kcb[i] < k_end) ? offb[i] : kInvalid;
      rb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, o, sb, 0));
    }
  };

  auto store_lds = [&](int stage) {
    u32x4* sa = lds + stage * STAGE;
    u32x4* sb = sa + A_STAGE;
#pragma unroll
    for (int i = 0; i < A_IT; i++) {
      const int idx = i * T + tid, r = idx >> 3, c = idx & 7;
      sa[r * 8 + (c ^ (r & 7))] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_IT; i++) {
      const int idx = i * T + tid;
      if constexpr (B8) {
        const int r = idx >> 2, c = idx & 3;
        sb[r * 4 + (c ^ ((r >> 1) & 3))] = rb[i];
      } else {
        const int r = idx >> 3, c = idx & 7;
        sb[r * 8 + (c ^ (r & 7))] = rb[i];
      }
    }
  };

  // LDS row indices and swizzle terms of this lane's fragments
  int arow[TM], brow[TN];
#pragma unroll
  for (int i = 0; i < TM; i++) arow[i] = wm * WTM + i * 32 + l32;
#pragma unroll
  for (int j = 0; j < TN; j++) brow[j] = wn * WTN + j * 32 + l32;

  auto compute = [&](int stage) {
    const u32x4* sa = lds + stage * STAGE;
    const u32x4* sb = sa + A_STAGE;
    u32x4 af[2][TM];
    u32x4 braw[B8 ? TN : 1][2];
    u32x4 bf[TN];
    if constexpr (B8) {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int r = brow[j], sw = (r >> 1) & 3;
        braw[j][0] = sb[r * 4 + ((2 * half) ^ sw)];
        braw[j][1] = sb[r * 4 + ((2 * half + 1) ^ sw)];
      }
    }
#pragma unroll
    for (int i = 0; i < TM; i++) af[0][i] = sa[arow[i] * 8 + ((half * 4) ^ (arow[i] & 7))];
    bool nan_codes = false;
    if constexpr (B8) {
      uint32_t any = 0;
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
          for (int e = 0; e < 4; e++) any |= ((braw[j][q][e] & 0x7f7f7f7fu) + 0x01010101u);
      nan_codes = __ballot((any & 0x80808080u) != 0u) != 0;
    }
    static_for<0, 4>([&](auto S) {
      constexpr int s = decltype(S)::value;
      if constexpr (s < 3) {
#pragma unroll
        for (int i = 0; i < TM; i++)
          af[(s + 1) & 1][i] = sa[arow[i] * 8 + ((half * 4 + s + 1) ^ (arow[i] & 7))];
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        if constexpr (B8) {
          const u32x4 q = braw[j][s >> 1];
          const uint32_t w0 = q[(s & 1) * 2], w1 = q[(s & 1) * 2 + 1];
          u32x2 lo, hi;
          if (nan_codes) {
            lo = fp8x4_to_16<IS_F16>(w0);
            hi = fp8x4_to_16<IS_F16>(w1);
          } else {
            lo = cvt_fp8x4<IS_F16>(w0);
            hi = cvt_fp8x4<IS_F16>(w1);
          }
          bf[j] = u32x4{lo.x, lo.y, hi.x, hi.y};
        } else {
          bf[j] = sb[brow[j] * 8 + ((half * 4 + s) ^ (brow[j] & 7))];
        }
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = mfma_32x32x16<IS_F16>(af[s & 1][i], bf[j], acc[i][j]);
    });
  };

  if (nk > 0) {
    load_global(k_begin);
    store_lds(0);
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
      const int cur = it & 1;
      if (it + 1 < nk) load_global(k_begin + (uint32_t)(it + 1) * BK);
      compute(cur);
      if (it + 1 < nk) store_lds(cur ^ 1);
      __syncthreads();
    }
  }

  const size_t zrow = (a.flags & WE_EPI_SPLIT_K_BIT) ? (size_t)z * a.m : 0;
  static_for<0, TM>([&](auto I) {
    static_for<0, TN>([&](auto J) {
      constexpr int i = decltype(I)::value, j = decltype(J)::value;
      const uint32_t col = col0 + wn * WTN + j * 32 + l32;
      const bool col_ok = col < a.n;
      const float b = (col_ok && (a.flags & WE_EPI_BIAS_BIT)) ? a.bias[col] : 0.0f;
      static_for<0, 16>([&](auto V) {
        constexpr int v = decltype(V)::value;
        const uint32_t row = row0 + wm * WTM + i * 32 + 8 * (v / 4) + 4 * half + (v % 4);
        if (col_ok && row < a.m) {
          float val = acc[i][j][v] * a.scale + b;
          if (a.flags & WE_EPI_GELU_BIT) val = gelu_tanh(val);
          store_y(a, (size_t)a.y_offset + (zrow + row) * (size_t)a.y_stride + col, val);
        }
      });
    });
  });
}

template <int BM, int BN, int WM, int WN, bool IS_F16, int BT>
static hipError_t launch_fast_cfg(FastArgs a, uint32_t splits, hipStream_t s) {
  a.tiles_m = (a.m + BM - 1) / BM;
  a.tiles_n = (a.n + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_fast_kernel<BM, BN, WM, WN, IS_F16, BT>), dim3(a.tiles_m * a.tiles_n, splits),
                     dim3(WM * WN * 64), 0, s, a);
  return hipGetLastError();
}

template <bool IS_F16, int BT>
static hipError_t launch_fast_types(const FastArgs& a, uint32_t splits, int cfg, hipStream_t s) {
  switch (cfg) {
    case GEMM_CFG_256x256: return launch_fast_cfg<256, 256, 2, 2, IS_F16, BT>(a, splits, s);
    case GEMM_CFG_256x128: return launch_fast_cfg<256, 128, 2, 2, IS_F16, BT>(a, splits, s);
    case GEMM_CFG_128x128: return launch_fast_cfg<128, 128, 2, 2, IS_F16, BT>(a, splits, s);
    case GEMM_CFG_64x64: return launch_fast_cfg<64, 64, 2, 2, IS_F16, BT>(a, splits, s);
    default: return launch_fast_cfg<32, 64, 1, 2, IS_F16, BT>(a, splits, s);
  }
}

// Returns hipErrorNotSupported when the shape / dtypes / alignment are not for this path.
hipError_t gemm_fast_launch(const GemmLaunch& L, hipStream_t stream) {
  const bool f16 = L.x_dtype == F16;
  if (!(L.x_dtype == BF16 || L.x_dtype == F16)) return hipErrorNotSupported;
  if (!(L.w_dtype == FP8 || (f16 ? L.w_dtype == F16 : L.w_dtype == BF16))) return hipErrorNotSupported;
  const uint32_t splits = L.splits < 1 ? 1 : L.splits;
  const uint32_t kc = splits > 1 ? L.kc : L.k;
  const int wb = L.w_dtype == FP8 ? 1 : 2;
  if (L.k % 16 || kc % 16) return hipErrorNotSupported;
  if (((uintptr_t)L.x + (uint64_t)L.x_offset * 2) % 16 || ((uintptr_t)L.w + (uint64_t)L.w_offset * wb) % 16 ||
      (L.x_stride * 2) % 16 || (L.w_stride * wb) % 16)
    return hipErrorNotSupported;
  const uint64_t xb = L.k ? ((uint64_t)(L.m - 1) * L.x_stride + L.k) * 2 : 0;
  const uint64_t wbytes = L.k ? ((uint64_t)(L.n - 1) * L.w_stride + L.k) * wb : 0;
  if (xb >= kInvalid || wbytes >= kInvalid) return hipErrorNotSupported;
  FastArgs a{};
  a.x = (const char*)L.x + (uint64_t)L.x_offset * 2;
  a.w = (const char*)L.w + (uint64_t)L.w_offset * wb;
  a.y = L.y;
  a.bias = L.bias;
  a.x_bytes = (uint32_t)xb;
  a.w_bytes = (uint32_t)wbytes;
  a.m = L.m;
  a.n = L.n;
  a.k = L.k;
  a.scale = L.scale;
  a.x_stride = L.x_stride;
  a.w_stride = L.w_stride;
  a.y_stride = L.y_stride;
  a.y_offset = L.y_offset;
  a.kc = kc;
  a.flags = L.flags;
  a.y_dtype = (uint32_t)L.y_dtype;
  const int cfg = L.cfg >= 0 ? L.cfg : pick_gemm_cfg(L.m, L.n, splits);
  if (f16) {
    if (L.w_dtype == FP8) return launch_fast_types<true, FP8>(a, splits, cfg, stream);
    return launch_fast_types<true, F16>(a, splits, cfg, stream);
  }
  if (L.w_dtype == FP8) return launch_fast_types<false, FP8>(a, splits, cfg, stream);
  return launch_fast_types<false, BF16>(a, splits, cfg, stream);
}

}  // namespace we
