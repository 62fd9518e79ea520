// Tiled GEMM on gfx950 MFMA: y[M, N] = x[M, K] . W[N, K]^T * scale, with W as stored (fp8 e4m3fn, bf16,
// f16 or f32) and fp32 accumulation. The math follows matmulWgsl (src/kernels/matmul.ts:118-178):
// strided / offset rows, scale applied to the f32 sum in the epilogue, split-K partials and accumulate
// mode, plus fused bias and tanh-GELU epilogues.
//
// Layout in LDS (per pipeline stage, two stages):
//   A: NA planes x BM rows x 64 k of 16-bit values = 128 B per row, eight 16-B chunks; chunk c of row r
//      lives at chunk (c ^ (r & 7)) so that the 32 rows an MFMA fragment reads hit distinct banks.
//   B fp8: BN rows x 64 B (raw bytes, unpacked in registers); chunk c of row r at (c ^ ((r >> 1) & 3)).
//   B 16-bit / f32: NB planes laid out like A.
// K order inside a 64-k block: lane half h (lane / 32) owns k in [32h, 32h + 32); MFMA step s uses
// [32h + 8s, 32h + 8s + 8). The same permutation is used for A and B, so the sum is unchanged and
// each lane reads 32 contiguous fp8 bytes (two ds_read_b128) per 32-column block.
// f32 operands are split into hi + mid + lo bf16 planes (f16 under a bf16 MFMA into hi + lo) when they
// are written to LDS; the product sums the plane pairs whose indices add up to at most 2, so the
// result carries the full 24-bit f32 mantissa of the inputs (dropped terms are below 2^-24).
#include "common.h"
#include "internal.h"

namespace we {

constexpr int BK = 64;

struct GemmArgs {
  const void* x;
  const void* w;
  void* y;
  const float* bias;
  const float* gate;  // gated residual: y = res + gate[col] * v (res may be y; NULL: none)
  const void* res;
  uint32_t m, n, k;
  float scale;
  uint32_t x_stride, w_stride, y_stride, x_offset, w_offset, y_offset;
  uint32_t kc;        // k values per split-K slice (= k when not split)
  uint32_t tiles_m, tiles_n;
  uint32_t flags;
  uint32_t y_dtype;
  uint32_t aligned;   // 1: every 16-B chunk of x / W rows is 16-B aligned
  uint32_t mul;       // product epilogue with res (GemmLaunch::mul), 0: none
  // 3x3 convolution input (conv_width > 0): x is a channel-last image [m / conv_width rows, conv_width, conv_cin],
  // row m of the GEMM is a pixel and k runs over (tap, channel) (src/kernels/matmul.ts:74-83)
  uint32_t conv_width, conv_cin;
};

// Planes per operand: 1 when the stored type is exact in the MFMA type; f16 under a bf16 MFMA needs
// hi + lo (exact: 11 bits <= 8 + 8); f32 needs hi + mid + lo (exact: 24 bits = 3 x 8).
template <int AT, int BT>
struct GemmTypes {
  static constexpr bool CT_F16 = (AT == F16) && (BT == FP8 || BT == F16);
  static constexpr int NA = AT == F32 ? 3 : ((AT == F16 && !CT_F16) ? 2 : 1);
  static constexpr int NB = BT == FP8 ? 1 : (BT == F32 ? 3 : ((BT == F16 && !CT_F16) ? 2 : 1));
  static constexpr int a_bytes = AT == F32 ? 4 : 2;
  static constexpr int b_bytes = BT == F32 ? 4 : (BT == FP8 ? 1 : 2);
};

// Hardware dispatches workgroup i to XCD i % 8. Renumber so that each XCD gets a contiguous range of
// tiles (which then share A rows / B columns in that XCD's L2).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t pid, uint32_t total) {
  const uint32_t xcd = pid & 7u, idx = pid >> 3;
  const uint32_t base = total >> 3, rem = total & 7u;
  return xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
}

// Split a value into 16-bit terms of the compute type (hi, then the rounded remainders).
template <bool CT_F16>
__device__ __forceinline__ uint32_t to_ct_bits(float v) {
  if constexpr (CT_F16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}
template <bool CT_F16>
__device__ __forceinline__ float ct_bits_to_f32(uint32_t h) {
  if constexpr (CT_F16) return f16_to_f32((uint16_t)h);
  else return bf16_to_f32((uint16_t)h);
}

// Eight consecutive source values (raw) -> one 16-B chunk per plane.
template <int SRC, bool CT_F16, int NP>
struct Chunk8 {
  // raw storage: f32 -> 8 floats (2 x u32x4); 16-bit -> 8 halves (1 x u32x4)
  static constexpr int RAW = SRC == F32 ? 2 : 1;
  __device__ static void convert(const u32x4 (&raw)[RAW], u32x4 (&out)[NP]) {
    if constexpr (NP == 1) {
      out[0] = raw[0];  // already the compute type
    } else {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if constexpr (SRC == F32) v[i] = __uint_as_float(raw[i / 4][i % 4]);
        else {
          const uint32_t h = (raw[0][i / 2] >> (16 * (i & 1))) & 0xffffu;
          v[i] = SRC == F16 ? f16_to_f32((uint16_t)h) : bf16_to_f32((uint16_t)h);
        }
      }
      uint32_t t[NP][8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        float rest = v[i];
#pragma unroll
        for (int p = 0; p < NP; p++) {
          t[p][i] = to_ct_bits<CT_F16>(rest);
          rest -= ct_bits_to_f32<CT_F16>(t[p][i]);
        }
      }
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[p][i] = t[p][2 * i] | (t[p][2 * i + 1] << 16);
    }
  }
};

template <int SRC>
__device__ __forceinline__ uint32_t raw_bits(const void* p, size_t i) {
  if constexpr (SRC == F32) return ((const uint32_t*)p)[i];
  else if constexpr (SRC == FP8) return ((const uint8_t*)p)[i];
  else return ((const uint16_t*)p)[i];
}

// Loads the chunk [k, k + VALS) of one row into raw registers; elements outside [.., k_end) or past the
// last row read as 0 (the reference pads partial tiles with zeros, src/kernels/matmul.ts:43,73).
template <int SRC, int VALS>
__device__ __forceinline__ void load_chunk(const void* base, size_t row_off, bool row_ok, uint32_t k, uint32_t k_end,
                                           bool aligned, u32x4* raw) {
  constexpr int BYTES = SRC == F32 ? 4 : (SRC == FP8 ? 1 : 2);
  constexpr int NV = VALS * BYTES / 16;  // u32x4 count
  if (row_ok && aligned && k + VALS <= k_end) {
    const u32x4* p = (const u32x4*)((const char*)base + (row_off + k) * BYTES);
#pragma unroll
    for (int i = 0; i < NV; i++) raw[i] = __builtin_nontemporal_load(p + i);
  } else {
    uint32_t words[NV * 4];
#pragma unroll
    for (int i = 0; i < NV * 4; i++) words[i] = 0;
    if (row_ok) {
#pragma unroll
      for (int e = 0; e < VALS; e++) {
        if (k + e < k_end) {
          const uint32_t b = raw_bits<SRC>(base, row_off + k + e);
          constexpr int PER = 4 / BYTES;  // values per dword
          words[e / PER] |= b << (8 * BYTES * (e % PER));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NV; i++) raw[i] = u32x4{words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]};
  }
}

// Eight k values [k, k + 8) of pixel `row` for the 3x3 convolution input, as load_chunk packs them: k runs over
// (tap, channel) with K = 9 * cin, tap t reads pixel (py + t / 3 - 1, px + t % 3 - 1), zeros outside the image
// (src/kernels/matmul.ts:74-83). cin is a multiple of 4, so each group of 4 values lies inside one tap.
template <int SRC>
__device__ __forceinline__ void load_conv8(const GemmArgs& a, uint32_t row, bool row_ok, uint32_t k, uint32_t k_end,
                                           u32x4* raw) {
  constexpr int BYTES = SRC == F32 ? 4 : 2;
  uint32_t words[8 * BYTES / 4];
#pragma unroll
  for (int i = 0; i < 8 * BYTES / 4; i++) words[i] = 0;
  const uint32_t width = a.conv_width, height = a.m / a.conv_width;
#pragma unroll
  for (int g = 0; g < 2; g++) {
    const uint32_t kk = k + 4u * g;
    if (!row_ok || kk >= k_end) continue;
    const uint32_t tap = kk / a.conv_cin, ch = kk % a.conv_cin;
    const int px = (int)(row % width) + (int)(tap % 3u) - 1, py = (int)(row / width) + (int)(tap / 3u) - 1;
    if (px < 0 || py < 0 || px >= (int)width || py >= (int)height) continue;
    const size_t e = ((size_t)py * width + (size_t)px) * a.conv_cin + ch;
    if constexpr (SRC == F32) {
      const u32x4 v = *(const u32x4*)((const float*)a.x + e);
#pragma unroll
      for (int i = 0; i < 4; i++) words[4 * g + i] = v[i];
    } else {
      const u32x2 v = *(const u32x2*)((const uint16_t*)a.x + e);
      words[2 * g] = v.x;
      words[2 * g + 1] = v.y;
    }
  }
#pragma unroll
  for (int i = 0; i < 2 * BYTES / 4; i++) raw[i] = u32x4{words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]};
}

// One output value: y = val, y += val (accumulate), y = res + val (gated residual) or the product epilogue with
// res, in the output dtype.
__device__ __forceinline__ void store_out(const GemmArgs& a, size_t o, float val) {
  if (a.mul) {
    const float aux = a.y_dtype == F32    ? ((const float*)a.res)[o]
                      : a.y_dtype == BF16 ? bf16_to_f32(((const uint16_t*)a.res)[o])
                                          : f16_to_f32(((const uint16_t*)a.res)[o]);
    val = mul_epilogue(a.mul, aux, val);
  }
  const void* add = a.mul ? nullptr : a.res ? a.res : ((a.flags & WE_EPI_ACCUMULATE_BIT) ? a.y : nullptr);
  if (a.y_dtype == F32) {
    ((float*)a.y)[o] = add ? ((const float*)add)[o] + val : val;
  } else if (a.y_dtype == BF16) {
    ((uint16_t*)a.y)[o] = f32_to_bf16(add ? bf16_to_f32(((const uint16_t*)add)[o]) + val : val);
  } else {
    ((uint16_t*)a.y)[o] = f32_to_f16(add ? f16_to_f32(((const uint16_t*)add)[o]) + val : val);
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int AT, int BT>
struct GemmCfg {
  using Ty = GemmTypes<AT, BT>;
  static constexpr int T = WAVES_M * WAVES_N * 64;
  static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int A_PLANE = BM * 128;  // bytes
  static constexpr int B_PLANE = BT == FP8 ? BN * 64 : BN * 128;
  static constexpr int STAGE = Ty::NA * A_PLANE + Ty::NB * B_PLANE;
  static constexpr int A_CHUNKS = BM * 8;                          // 8-value chunks per stage
  static constexpr int B_CHUNKS = BT == FP8 ? BN * 4 : BN * 8;     // 16 fp8 or 8 values per chunk
  static constexpr int A_ITERS = A_CHUNKS / T;
  static constexpr int B_ITERS = B_CHUNKS / T;
  static constexpr int A_RAW = AT == F32 ? 2 : 1;
  static constexpr int B_RAW = BT == F32 ? 2 : 1;
  static_assert(A_CHUNKS % T == 0 && B_CHUNKS % T == 0, "tile / thread mismatch");
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-aligned");
};

template <int BM, int BN, int WAVES_M, int WAVES_N, int AT, int BT>
__global__ void __launch_bounds__(WAVES_M* WAVES_N * 64)
gemm_kernel(GemmArgs a) {
  using C = GemmCfg<BM, BN, WAVES_M, WAVES_N, AT, BT>;
  using Ty = typename C::Ty;
  constexpr bool CT_F16 = Ty::CT_F16;
  constexpr int NA = Ty::NA, NB = Ty::NB;
  __shared__ u32x4 lds[2 * C::STAGE / 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // tile coordinates: XCD-contiguous ranges, then GROUP_M-swizzled so neighbours share W columns
  const uint32_t total = gridDim.x;
  const uint32_t pid = xcd_remap(blockIdx.x, total);
  constexpr uint32_t GROUP_M = 4;
  const uint32_t per_group = GROUP_M * a.tiles_n;
  const uint32_t group = pid / per_group;
  const uint32_t first_m = group * GROUP_M;
  const uint32_t gsize = min(a.tiles_m - first_m, GROUP_M);
  const uint32_t in_group = pid % per_group;
  const uint32_t tile_m = first_m + in_group % gsize;
  const uint32_t tile_n = in_group / gsize;
  const uint32_t row0 = tile_m * BM, col0 = tile_n * BN;

  const uint32_t z = blockIdx.y;
  const uint32_t k_begin = z * a.kc;
  const uint32_t k_end = min(a.k, k_begin + a.kc);
  const int nk = k_end > k_begin ? (int)((k_end - k_begin + BK - 1) / BK) : 0;
  const bool aligned = a.aligned != 0;

  f32x16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; i++)
#pragma unroll
    for (int j = 0; j < C::TN; j++) acc[i][j] = f32x16{};

  u32x4 ra[C::A_ITERS][C::A_RAW];
  u32x4 rb[C::B_ITERS][C::B_RAW];

  auto load_global = [&](uint32_t kb) {
#pragma unroll
    for (int i = 0; i < C::A_ITERS; i++) {
      const int idx = i * C::T + tid;
      const int r = idx >> 3, c = idx & 7;
      const uint32_t row = row0 + r;
      if (a.conv_width)
        load_conv8<AT>(a, row, row < a.m, kb + c * 8, k_end, ra[i]);
      else
        load_chunk<AT, 8>(a.x, (size_t)a.x_offset + (size_t)row * a.x_stride, row < a.m, kb + c * 8, k_end, aligned,
                          ra[i]);
    }
#pragma unroll
    for (int i = 0; i < C::B_ITERS; i++) {
      const int idx = i * C::T + tid;
      if constexpr (BT == FP8) {
        const int r = idx >> 2, c = idx & 3;
        const uint32_t col = col0 + r;
        load_chunk<FP8, 16>(a.w, (size_t)a.w_offset + (size_t)col * a.w_stride, col < a.n, kb + c * 16, k_end, aligned,
                            rb[i]);
      } else {
        const int r = idx >> 3, c = idx & 7;
        const uint32_t col = col0 + r;
        load_chunk<BT, 8>(a.w, (size_t)a.w_offset + (size_t)col * a.w_stride, col < a.n, kb + c * 8, k_end, aligned,
                          rb[i]);
      }
    }
  };

  auto store_lds = [&](int stage) {
    u32x4* sa = lds + stage * (C::STAGE / 16);
    u32x4* sb = sa + NA * (C::A_PLANE / 16);
#pragma unroll
    for (int i = 0; i < C::A_ITERS; i++) {
      const int idx = i * C::T + tid;
      const int r = idx >> 3, c = idx & 7;
      u32x4 planes[NA];
      Chunk8<AT, CT_F16, NA>::convert(ra[i], planes);
#pragma unroll
      for (int p = 0; p < NA; p++) sa[p * (C::A_PLANE / 16) + r * 8 + (c ^ (r & 7))] = planes[p];
    }
#pragma unroll
    for (int i = 0; i < C::B_ITERS; i++) {
      const int idx = i * C::T + tid;
      if constexpr (BT == FP8) {
        const int r = idx >> 2, c = idx & 3;
        sb[r * 4 + (c ^ ((r >> 1) & 3))] = rb[i][0];
      } else {
        const int r = idx >> 3, c = idx & 7;
        u32x4 planes[NB];
        Chunk8<BT, CT_F16, NB>::convert(rb[i], planes);
#pragma unroll
        for (int p = 0; p < NB; p++) sb[p * (C::B_PLANE / 16) + r * 8 + (c ^ (r & 7))] = planes[p];
      }
    }
  };

  const int half = lane >> 5, l32 = lane & 31;

  auto compute = [&](int stage) {
    const u32x4* sa = lds + stage * (C::STAGE / 16);
    const u32x4* sb = sa + NA * (C::A_PLANE / 16);
    u32x4 braw[BT == FP8 ? C::TN : 1][2];
    if constexpr (BT == FP8) {
#pragma unroll
      for (int j = 0; j < C::TN; j++) {
        const int r = wn * C::WTN + j * 32 + l32;
        const int sw = (r >> 1) & 3;
        braw[j][0] = sb[r * 4 + ((2 * half) ^ sw)];
        braw[j][1] = sb[r * 4 + ((2 * half + 1) ^ sw)];
      }
    }
#pragma unroll
    for (int s = 0; s < 4; s++) {
      u32x4 af[C::TM][NA];
#pragma unroll
      for (int i = 0; i < C::TM; i++) {
        const int r = wm * C::WTM + i * 32 + l32;
        const int c = half * 4 + s;
#pragma unroll
        for (int p = 0; p < NA; p++) af[i][p] = sa[p * (C::A_PLANE / 16) + r * 8 + (c ^ (r & 7))];
      }
      u32x4 bf[C::TN][NB];
#pragma unroll
      for (int j = 0; j < C::TN; j++) {
        if constexpr (BT == FP8) {
          const u32x4 q = braw[j][s >> 1];
          const uint32_t w0 = q[(s & 1) * 2], w1 = q[(s & 1) * 2 + 1];
          const u32x2 lo = fp8x4_to_16<CT_F16>(w0), hi = fp8x4_to_16<CT_F16>(w1);
          bf[j][0] = u32x4{lo.x, lo.y, hi.x, hi.y};
        } else {
          const int r = wn * C::WTN + j * 32 + l32;
          const int c = half * 4 + s;
#pragma unroll
          for (int p = 0; p < NB; p++) bf[j][p] = sb[p * (C::B_PLANE / 16) + r * 8 + (c ^ (r & 7))];
        }
      }
#pragma unroll
      for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
#pragma unroll
          for (int pa = 0; pa < NA; pa++)
#pragma unroll
            for (int pb = 0; pb < NB; pb++)
              if (pa + pb <= 2) acc[i][j] = mfma_32x32x16<CT_F16>(af[i][pa], bf[j][pb], acc[i][j]);
        }
    }
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

  // epilogue: lane holds column l32 of each 32x32 block, rows 8*(v/4) + 4*half + v%4
  const size_t zrow = (a.flags & WE_EPI_SPLIT_K_BIT) ? (size_t)z * a.m : 0;
  static_for<0, C::TM>([&](auto I) {
    static_for<0, C::TN>([&](auto J) {
      constexpr int i = decltype(I)::value, j = decltype(J)::value;
      const uint32_t col = col0 + wn * C::WTN + j * 32 + l32;
      const bool col_ok = col < a.n;
      const float b = (col_ok && (a.flags & WE_EPI_BIAS_BIT)) ? a.bias[col] : 0.0f;
      const float gt = (col_ok && a.gate) ? a.gate[col] : 1.0f;
      static_for<0, 16>([&](auto V) {
        constexpr int v = decltype(V)::value;
        const uint32_t row = row0 + wm * C::WTM + i * 32 + 8 * (v / 4) + 4 * half + (v % 4);
        if (col_ok && row < a.m) {
          float val = acc[i][j][v] * a.scale + b;
          if (a.flags & WE_EPI_GELU_BIT) val = gelu_tanh(val);
          if (a.gate) val *= gt;
          store_out(a, (size_t)a.y_offset + (zrow + row) * (size_t)a.y_stride + col, val);
        }
      });
    });
  });
}

// ---------------------------------------------------------------------------------------------------
// host-side dispatch

template <int BM, int BN, int WAVES_M, int WAVES_N, int AT, int BT>
static hipError_t launch_cfg(const GemmArgs& a0, uint32_t splits, hipStream_t stream) {
  GemmArgs a = a0;
  a.tiles_m = (a.m + BM - 1) / BM;
  a.tiles_n = (a.n + BN - 1) / BN;
  dim3 grid(a.tiles_m * a.tiles_n, splits);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WAVES_M, WAVES_N, AT, BT>), grid, dim3(WAVES_M * WAVES_N * 64), 0, stream, a);
  return hipGetLastError();
}

template <int AT, int BT>
static hipError_t launch_types(const GemmArgs& a, uint32_t splits, int cfg, hipStream_t stream) {
  using Ty = GemmTypes<AT, BT>;
  constexpr bool big_ok = Ty::NA == 1 && Ty::NB == 1;
  if constexpr (Ty::NA + Ty::NB > 4) {  // three-plane operands: only the small tiles fit in LDS
    if (cfg == GEMM_CFG_32x64) return launch_cfg<32, 64, 1, 2, AT, BT>(a, splits, stream);
    return launch_cfg<64, 64, 2, 2, AT, BT>(a, splits, stream);
  } else {
    switch (cfg) {
      case GEMM_CFG_256x256:
        if constexpr (big_ok) return launch_cfg<256, 256, 2, 2, AT, BT>(a, splits, stream);
        else return launch_cfg<128, 128, 2, 2, AT, BT>(a, splits, stream);
      case GEMM_CFG_256x192:  // no 192-column tile here: 256 x 128
      case GEMM_CFG_256x128:
        if constexpr (big_ok) return launch_cfg<256, 128, 2, 2, AT, BT>(a, splits, stream);
        else return launch_cfg<128, 128, 2, 2, AT, BT>(a, splits, stream);
      case GEMM_CFG_128x128: return launch_cfg<128, 128, 2, 2, AT, BT>(a, splits, stream);
      case GEMM_CFG_64x64: return launch_cfg<64, 64, 2, 2, AT, BT>(a, splits, stream);
      default: return launch_cfg<32, 64, 1, 2, AT, BT>(a, splits, stream);
    }
  }
}

template <int AT>
static hipError_t launch_w(int bt, const GemmArgs& a, uint32_t splits, int cfg, hipStream_t s) {
  switch (bt) {
    case FP8: return launch_types<AT, FP8>(a, splits, cfg, s);
    case BF16: return launch_types<AT, BF16>(a, splits, cfg, s);
    case F16: return launch_types<AT, F16>(a, splits, cfg, s);
    default: return launch_types<AT, F32>(a, splits, cfg, s);
  }
}

static bool aligned16(const void* p, uint64_t elems_offset, uint64_t stride, int bytes) {
  return (((uintptr_t)p) % 16 == 0) && ((elems_offset * bytes) % 16 == 0) && ((stride * bytes) % 16 == 0);
}

int pick_gemm_cfg(uint32_t m, uint32_t n, uint32_t splits) {
  if (m <= 32) return GEMM_CFG_32x64;
  if (m <= 64) return GEMM_CFG_64x64;
  const uint64_t big = (uint64_t)((m + 255) / 256) * ((n + 255) / 256) * splits;
  if (m >= 256 && n >= 256 && big >= 512) return GEMM_CFG_256x256;
  const uint64_t mid = (uint64_t)((m + 255) / 256) * ((n + 127) / 128) * splits;
  if (m >= 256 && mid >= 256) return GEMM_CFG_256x128;
  return GEMM_CFG_128x128;
}

hipError_t gemm_launch(const GemmLaunch& L, hipStream_t stream) {
  if (!L.generic && !L.conv_width) {
    const hipError_t e = gemm_fast_launch(L, stream);
    if (e != hipErrorNotSupported || L.k_wrap) return e;  // planes of x (k_wrap) exist for the fast path only
  }
  GemmArgs a{};
  a.x = L.x;
  a.w = L.w;
  a.y = L.y;
  a.bias = L.bias;
  a.gate = L.gate;
  a.res = L.res;
  a.m = L.m;
  a.n = L.n;
  a.k = L.k;
  a.scale = L.scale;
  a.x_stride = L.x_stride;
  a.w_stride = L.w_stride;
  a.y_stride = L.y_stride;
  a.x_offset = L.x_offset;
  a.w_offset = L.w_offset;
  a.y_offset = L.y_offset;
  a.flags = L.flags;
  a.y_dtype = (uint32_t)L.y_dtype;
  a.mul = (uint32_t)L.mul;
  a.conv_width = L.conv_width;
  a.conv_cin = L.conv_cin;
  const uint32_t splits = L.splits < 1 ? 1 : L.splits;
  a.kc = splits > 1 ? L.kc : L.k;
  const int xb = L.x_dtype == F32 ? 4 : 2;
  const int wb = L.w_dtype == F32 ? 4 : (L.w_dtype == FP8 ? 1 : 2);
  a.aligned = aligned16(L.x, L.x_offset, L.x_stride, xb) && aligned16(L.w, L.w_offset, L.w_stride, wb) &&
              ((uint64_t)a.kc * xb) % 16 == 0 && ((uint64_t)a.kc * wb) % 16 == 0;
  const int cfg = L.cfg >= 0 ? L.cfg : pick_gemm_cfg(L.m, L.n, splits);
  switch (L.x_dtype) {
    case BF16: return launch_w<BF16>(L.w_dtype, a, splits, cfg, stream);
    case F16: return launch_w<F16>(L.w_dtype, a, splits, cfg, stream);
    default: return launch_w<F32>(L.w_dtype, a, splits, cfg, stream);
  }
}

}  // namespace we
