// Fast path of the gfx950 GEMM for the hot dtypes: 16-bit activations (bf16 or f16) times fp8 e4m3fn or
// 16-bit weights, fp32 accumulation on MFMA (16x16x32 in the ping-pong tiles, 32x32x16 in the others),
// y = x . W^T * scale (+ bias, gelu, accumulate, split-K) with the semantics of matmulWgsl
// (src/kernels/matmul.ts:118-178).
//
// Structure (one workgroup per BM x BN output tile, 64 k per pipeline stage, S stages in LDS):
//  * Operands move HBM -> LDS with direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds): each load
//    instruction of a wave fills 1 KB of LDS (lane i writes bytes [16 i, 16 i + 16)), no VGPR staging.
//    The source address of each lane is chosen so that the LDS image is XOR-swizzled: 16-byte chunk c of
//    row r sits at chunk position c ^ swz(r), which makes the MFMA fragment reads bank-conflict free.
//    Rows past M / N and k past the slice read through an out-of-range buffer offset and land as zeros.
//  * Loads run S - 1 stages ahead of the MFMAs. The 256 x 256 tiles (8 waves, two per SIMD) use a
//    ping-pong schedule: the two waves of a SIMD alternate between a phase of MFMAs only and a phase of
//    fragment reads / unpack / loads, one phase apart, separated by workgroup barriers (details at the
//    loop). Smaller tiles use one workgroup barrier per 64-k block, placed before the last MFMA step of
//    the block: after it the block's stage is free for the load S blocks ahead, and the next block's
//    stage is complete, so its first fragments are read while the last MFMAs still run.
//  * The weight tile is the MFMA's A operand and the activation tile its B operand, so the fp32
//    accumulators hold runs of 4 consecutive output columns per lane: the epilogue stores 8 or 16 bytes
//    per lane instead of 2.
//  * fp8 weights stay 1 byte per value in LDS and are unpacked to bf16 / f16 in registers by the
//    hardware converter (OCP e4m3fn). That converter turns the two NaN codes 0x7f / 0xff into NaN, where
//    the reference shader decodes them as +-480 (src/kernels/fp8.ts:12-20). The main loop does not look
//    at the codes; a NaN in a wave's accumulators (which finite weights and inputs never produce) sends
//    that wave through an exact recompute that decodes every byte with the shader's formula.
// Requirements (checked on the host): x / W rows 16-byte aligned, K and the split-K slice multiples of
// 16, operand extents below 2^31 bytes.
// f32 activations arrive as three exact bf16 planes along K (x [M, 3K], split by a pass before the GEMM); the kernel
// walks k over all 3K while the weights are read at k mod K (K a multiple of 64, so no 64-k block spans two
// planes): one GEMM of exact products, so every epilogue applies to the f32-exact sum.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "internal.h"

namespace we {

namespace {

constexpr int BK = 64;

constexpr uint32_t kInvalid = 0x80000000u;  // a byte offset past every extent: the load returns 0
constexpr int kRsrcWord3 = 0x00020000;      // raw buffer, 32-bit data format (gfx9 family)
constexpr int kCpolNt = 2;                  // buffer-load cache policy: nt (non-temporal)

typedef __attribute__((address_space(3))) void lds_ptr_t;

struct FastArgs {
  const void* x;
  const void* w;
  void* y;
  const float* bias;
  const float* gate;  // gated residual: y = res + gate[col] * v (res may be y; NULL: none)
  const void* res;
  uint32_t x_bytes, w_bytes;  // readable bytes from x / w (their extents)
  uint32_t m, n, k;
  // weights read at k - kwrap (k >= kwrap) and k - kwrap2 (k >= kwrap2): x holds k / kwrap planes of kwrap values per
  // row (GemmLaunch::k_wrap); 0xffffffff: no wrap
  uint32_t kwrap, kwrap2;
  float scale;
  uint32_t x_stride, w_stride, y_stride, y_offset;  // x / w already point at their offsets
  uint32_t kc;
  uint32_t tiles_m, tiles_n;
  uint32_t flags, y_dtype;
  uint32_t vec_store;  // 1: y rows and y_offset allow 4-value vector stores
  uint32_t store16;    // 1: y, y_offset and y rows are 16-byte aligned (whole-row staging of 16-bit outputs)
  // split-K partial sums (rsplits > 1): slice z stores its raw sums at part + z * m * n (dense rows of n);
  // splitk_reduce_kernel adds the slices and runs the epilogue
  float* part;
  uint32_t rsplits;
  uint32_t mul;  // product epilogue with res (GemmLaunch::mul), 0: none
  // fused per-head RMSNorm + RoPE of the q / k columns (GemmLaunch::qk_*), qk_cols 0: none
  uint32_t qk_cols, q_cols, qk_rope_from;
  float qk_eps, qk_offset;
  const float* qk_norm_q;
  const float* qk_norm_k;
  const float* qk_cos;
  const float* qk_sin;
  // A second GEMM in the same launch (gemm_fast_launch_pair): the same N, K, types, flags and product epilogue,
  // operands of its own. Tiles from grp_first on (after the XCD renumbering) compute it; grp_first 0: none.
  struct Second {
    const void* x;
    const void* w;
    void* y;
    const float* bias;
    const float* gate;
    const void* res;
    uint32_t x_bytes, w_bytes, m, x_stride, w_stride, y_stride, y_offset, tiles_m, vec_store, store16;
    float scale;
  } g;
  uint32_t grp, grp_first;
};

__device__ __forceinline__ uint32_t xcd_remap_f(uint32_t pid, uint32_t total) {
  const uint32_t xcd = pid & 7u, idx = pid >> 3;
  const uint32_t base = total >> 3, rem = total & 7u;
  return xcd < rem ? xcd * (base + 1) + idx : rem * (base + 1) + (xcd - rem) * base + idx;
}

// Chunk position of logical 16-byte chunk c in row r: rows of 128 B (8 chunks) and rows of 64 B
// (4 chunks). Both keep any 8 (and any 16) consecutive rows reading one logical chunk on distinct banks.
__device__ __forceinline__ int swz128(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz64(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// fp8 word -> 4 x 16-bit through the hardware converter
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

// y[o .. o + 3] = v, or addend[o ..] + v (addend: the residual, or y itself to accumulate; NULL: none)
template <int YT>
__device__ __forceinline__ void store4(const FastArgs& a, size_t o, const float (&v)[4], const void* addend) {
  if constexpr (YT == F32) {
    f32x4* p = (f32x4*)((float*)a.y + o);
    f32x4 r = {v[0], v[1], v[2], v[3]};
    if (addend) r += *(const f32x4*)((const float*)addend + o);
    *p = r;
  } else {
    u32x2* p = (u32x2*)((uint16_t*)a.y + o);
    float t[4] = {v[0], v[1], v[2], v[3]};
    if (addend) {
      const u32x2 old = *(const u32x2*)((const uint16_t*)addend + o);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t h = ((e < 2 ? old.x : old.y) >> (16 * (e & 1))) & 0xffffu;
        t[e] += YT == BF16 ? bf16_to_f32((uint16_t)h) : f16_to_f32((uint16_t)h);
      }
    }
    const std::integral_constant<bool, YT == F16> tag;
    *p = u32x2{pack2(t[0], t[1], tag), pack2(t[2], t[3], tag)};
  }
}

// one value of a y-typed operand (the product epilogue's aux) as f32
template <int YT>
__device__ __forceinline__ float load1(const void* p, size_t o) {
  if constexpr (YT == F32) return ((const float*)p)[o];
  else if constexpr (YT == BF16) return bf16_to_f32(((const uint16_t*)p)[o]);
  else return f16_to_f32(((const uint16_t*)p)[o]);
}

template <int YT>
__device__ __forceinline__ void store1(const FastArgs& a, size_t o, float v, const void* addend) {
  if constexpr (YT == F32) {
    ((float*)a.y)[o] = addend ? ((const float*)addend)[o] + v : v;
  } else {
    if (addend) {
      const uint16_t h = ((const uint16_t*)addend)[o];
      v += YT == BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    }
    ((uint16_t*)a.y)[o] = YT == BF16 ? f32_to_bf16(v) : f32_to_f16(v);
  }
}

}  // namespace

template <int BM, int BN, int WAVES_M, int WAVES_N, bool IS_F16, int BT, int S, int YT, bool PP>
__global__ void __launch_bounds__(WAVES_M* WAVES_N * 64) gemm_lds_kernel(FastArgs a) {
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  // The ping-pong tiles multiply on 16x16x32 MFMAs (more work per watt at the chip's power limit: 4096 x 12288 x 3072
  // up-projection 245 -> 232 us, down-projection 235 -> 224 us, bf16 4096 x 9216 x 3072 200 -> 186 us, same box,
  // against 32x32x16), the other tiles on 32x32x16. Accumulator block (ri, rc)
  // of a lane holds rows ri * RS + lrow and the 4 columns ccol(rc) + lcol .. + 3 of the wave tile: 32x32 blocks give
  // lane (l32, h) row l32 and, per block, 4 runs (8 q + 4 h); 16x16 blocks give lane (r16, g) row r16 and one run 4 g.
  constexpr int RS = PP ? 16 : 32;          // rows of an accumulator block
  constexpr int RR = WTM / RS;              // accumulator block rows per wave
  constexpr int TN16 = WTN / 16;            // 16x16 blocks per wave row (ping-pong tiles)
  constexpr int RC = PP ? TN16 : 4 * TN;    // 4-column runs per row and lane
  using AccT = std::conditional_t<PP, f32x4, f32x16>;
  constexpr bool B8 = BT == FP8;
  constexpr int WB = B8 ? 1 : 2;                  // weight bytes per value
  constexpr int A_BYTES = BM * 128;               // x: BM rows x 64 k x 2 B
  constexpr int B_ROW = 64 * WB;                  // weight row bytes per stage
  // the weight area is rounded up to whole load rounds of the workgroup; rows past BN load zeros (a
  // 192-column tile fills 12 of 16 loads)
  constexpr int B_INS = (BN * B_ROW / 1024 + NW - 1) / NW * NW;
  constexpr int B_BYTES = B_INS * 1024;
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int A_INS = A_BYTES / 1024;
  static_assert(A_INS % NW == 0 && (BN * B_ROW) % 1024 == 0, "stage loads must split evenly over the waves");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0 && WTM >= 32, "wave tile");
  static_assert(!PP || NW * 32 * (WTN * 2 + 16) <= S * STAGE, "the epilogue's row staging fits the stages");
  // Load schedule of the ping-pong tiles (LM, details at the loop). 16-bit weights (two ring stages): 1, the waves of
  // group 1 issue every load, between the MFMAs of their compute phase, one block further ahead than a memory-phase
  // load could be (4096 x 9216 x 3072 bf16, 256 x 192 tiles: 211 -> 199-205 us, same box). fp8 weights (three
  // stages): 0, every wave issues its share in its memory phase; loads in the compute phases held the MFMAs back (1:
  // 243 -> 279 us, 2, each group its own share in its compute phase: 247 -> 291 us, up-projection, same box).
  // Other tiles: every wave loads its share in the memory phase.
  constexpr int LM = PP ? (B8 ? 0 : 1) : 0;
  constexpr int NL = LM == 1 ? NW / 2 : NW;                               // waves that issue loads
  static_assert(A_INS % NL == 0 && B_INS % NL == 0, "stage loads split evenly over the loading waves");
  constexpr int A_PW = A_INS / NL, B_PW = B_INS / NL, L = A_PW + B_PW;  // loads per loading wave per stage
  constexpr int B_RPI = 1024 / B_ROW;                                     // weight rows per load
  constexpr int B_CPR = B_ROW / 16;                                       // 16-B chunks per weight row
  __shared__ __attribute__((aligned(1024))) char lds[S * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int lw = wave % NL;  // this wave's share of the loads (LM 1: group 1's waves 0 .. NW / 2 - 1)
  const int h = lane >> 5, l32 = lane & 31;

  uint32_t pid = xcd_remap_f(blockIdx.x, gridDim.x);
  if (a.grp_first && pid >= a.grp_first) {  // a tile of the second GEMM of a paired launch
    pid -= a.grp_first;
    a.x = a.g.x;
    a.w = a.g.w;
    a.y = a.g.y;
    a.bias = a.g.bias;
    a.gate = a.g.gate;
    a.res = a.g.res;
    a.x_bytes = a.g.x_bytes;
    a.w_bytes = a.g.w_bytes;
    a.m = a.g.m;
    a.x_stride = a.g.x_stride;
    a.w_stride = a.g.w_stride;
    a.y_stride = a.g.y_stride;
    a.y_offset = a.g.y_offset;
    a.tiles_m = a.g.tiles_m;
    a.vec_store = a.g.vec_store;
    a.store16 = a.g.store16;
    a.scale = a.g.scale;
  }
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

  // ---- per-lane source offsets of the direct-to-LDS loads (k = 0 of the block), invalid past M / N
  // The rows of a lane's successive loads are 8 NL (x) and B_RPI NL (weights) apart, multiples of 16 (swz128) and of 32
  // (swz64), so its chunk, and the first k of that chunk inside the 64-k block (ka, kb8), is the same for every load.
  static_assert((8 * NL) % 16 == 0 && (B_RPI * NL) % (B8 ? 32 : 16) == 0, "one swizzled chunk per lane");
  uint32_t offa[A_PW], offb[B_PW];
  int ka, kb8;
#pragma unroll
  for (int i = 0; i < A_PW; i++) {
    const int ins = lw + i * NL;
    const int r = ins * 8 + (lane >> 3);
    const int c = (lane & 7) ^ swz128(r);
    const uint32_t row = row0 + r;
    offa[i] = row < a.m ? (row * a.x_stride + c * 8) * 2 : kInvalid;
    if (i == 0) ka = c * 8;
  }
#pragma unroll
  for (int j = 0; j < B_PW; j++) {
    const int ins = lw + j * NL;
    const int r = ins * B_RPI + lane / B_CPR;
    const int c = (lane % B_CPR) ^ (B8 ? swz64(r) : swz128(r));
    const uint32_t col = col0 + r;
    offb[j] = r < BN && col < a.n ? (col * a.w_stride * WB + c * 16) : kInvalid;
    if (j == 0) kb8 = c * 16 / WB;
  }

  // With one row of tiles (M <= BM) every weight byte is read once per call: its loads take the non-temporal cache
  // policy (64 x 3072 x 3072 with the weights streamed from HBM: 11.24 -> 10.78 us; with the weights left in the
  // caches between calls 9.28 -> 9.37 us). Where M-tiles share the weights it costs L2 reuse (the 4096 x 12288 x 3072
  // up-projection 232 -> 244 us). Not in the ping-pong tiles, whose memory phase the branch reorders (the
  // up-projection 232 -> 241-246 us with it).
  const bool w_once = !PP && a.tiles_m == 1;
  // load q (0 .. L - 1) of this wave's share of the 64-k block starting at kb, into stage st
  auto issue_one = [&](auto Q, uint32_t kb, int st) {
    constexpr int q = decltype(Q)::value;
    const bool full = kb + BK <= k_end;  // only the last block of a slice can be partial
    char* base = lds + st * STAGE;
    if constexpr (q < A_PW) {
      const uint32_t o = (full || kb + ka < k_end) ? offa[q] : kInvalid;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t*)(base + (lw + q * NL) * 1024), 16, o, (int)(kb * 2), 0,
                                               0);
    } else {
      constexpr int j = q - A_PW;
      const uint32_t o = (full || kb + kb8 < k_end) ? offb[j] : kInvalid;
      const uint32_t kbw = kb >= a.kwrap2 ? kb - a.kwrap2 : kb >= a.kwrap ? kb - a.kwrap : kb;  // weights' k
      lds_ptr_t* dst = (lds_ptr_t*)(base + A_BYTES + (lw + j * NL) * 1024);
      if constexpr (!PP) {
        if (w_once) __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 16, o, (int)(kbw * WB), 0, kCpolNt);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 16, o, (int)(kbw * WB), 0, 0);
      } else {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 16, o, (int)(kbw * WB), 0, 0);
      }
    }
  };
  // issue this wave's share of the loads of the 64-k block starting at kb into stage st
  auto issue = [&](uint32_t kb, int st) { static_for<0, L>([&](auto Q) { issue_one(Q, kb, st); }); };

  // ---- per-lane LDS read offsets of the MFMA fragments (within a stage)
  // k order inside a 64-k block: MFMA step s, lane half h uses the 8 k of logical chunk 4h + s for both
  // operands (a permutation of k shared by x and W, so the sum is unchanged).
  uint32_t rda[4], rdb[B8 ? 2 : 4];
  {
    const int sa = (4 * h) ^ swz128(l32);
#pragma unroll
    for (int s = 0; s < 4; s++) rda[s] = (uint32_t)((wm * WTM + l32) * 128 + ((sa ^ s) * 16));
    if constexpr (B8) {
      const int sb = (2 * h) ^ swz64(l32);  // 16-B chunk 2h + t holds the 16 k of steps 2t, 2t + 1
#pragma unroll
      for (int t = 0; t < 2; t++) rdb[t] = (uint32_t)(A_BYTES + (wn * WTN + l32) * 64 + ((sb ^ t) * 16));
    } else {
#pragma unroll
      for (int s = 0; s < 4; s++) rdb[s] = (uint32_t)(A_BYTES + (wn * WTN + l32) * 128 + ((sa ^ s) * 16));
    }
  }
  // 16x16x32 (ping-pong tiles): 2 MFMA steps per 64-k block; step s, lane group g uses the 8 k of logical chunk
  // 2 g + s of both operands (k 16 g + 8 s ..), so an fp8 weight lane reads the 16 bytes of both steps at once.
  // x: row wm WTM + 16 i + r16; fp8 weights: row wn WTN + 16 j + r16, whose swizzle (bits 1-4 of the row) depends on
  // the parity of j; 16-bit weights: per step, as x.
  const int r16 = lane & 15, g16 = lane >> 4;
  uint32_t rx16[2], rw16[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    rx16[t] = (uint32_t)((wm * WTM + r16) * 128 + (((2 * g16 + t) ^ swz128(r16)) * 16));
    if constexpr (B8)
      rw16[t] = (uint32_t)(A_BYTES + (wn * WTN + 16 * t + r16) * 64 + ((g16 ^ swz64(16 * t + r16)) * 16));
    else
      rw16[t] = (uint32_t)(A_BYTES + (wn * WTN + r16) * 128 + (((2 * g16 + t) ^ swz128(r16)) * 16));
  }
  auto rd = [&](uint32_t off) { return *(const u32x4*)(lds + off); };

  AccT acc[RR][PP ? TN16 : TN];
#pragma unroll
  for (int i = 0; i < RR; i++)
#pragma unroll
    for (int j = 0; j < (PP ? TN16 : TN); j++) acc[i][j] = AccT{};

  u32x4 xf[2][TM];           // x fragments, double-buffered over steps
  u32x4 wr[2][TN];           // fp8: raw 16-B chunks (t = 0, 1); 16-bit: fragments double-buffered over steps
  auto read_x = [&](uint32_t st_off, int s, u32x4 (&d)[TM]) {
#pragma unroll
    for (int i = 0; i < TM; i++) d[i] = rd(st_off + rda[s] + i * 32 * 128);
  };
  auto read_w = [&](uint32_t st_off, int q, u32x4 (&d)[TN]) {
#pragma unroll
    for (int j = 0; j < TN; j++) d[j] = rd(st_off + rdb[q] + j * 32 * B_ROW);
  };

  if constexpr (PP) {
    // ---- ping-pong schedule. Waves w and w + NW / 2 share a SIMD (waves of a workgroup go round-robin
    // over the 4 SIMDs); group grp = w / (NW / 2). Each wave alternates a memory phase (all fragment
    // reads of one 64-k block, and the loads of the block S - 1 ahead) with a compute phase (the block's
    // 4 x TM x TN MFMAs, the fp8 unpack interleaved between them). Group 1 runs one phase behind group 0,
    // so in every interval between two workgroup barriers one wave of each SIMD issues MFMAs while the
    // other prepares its next operands: the MFMA pipe does not wait on LDS latency or on a barrier that
    // both waves of the SIMD sit at.
    // Interval j: group 0 runs phase j (even = memory of block j / 2, odd = compute), group 1 phase
    // j - 1. Block t is first read in interval 2t (group 0), so every wave waits for its own loads of
    // block t before the barrier that ends interval 2t - 1. The loads of block t + S - 1 go into the stage
    // of block t - 1, whose last read (group 1) was in interval 2t - 1, and are issued at the start of the
    // memory phase of block t: interval 2t or 2t + 1.
    static_assert(NW % 2 == 0 && S >= 2, "ping-pong needs two wave groups");
    const int grp = wave / (NW / 2);
    u32x4 xb[2][RR];                // x fragments of the 2 MFMA steps of a block
    u32x4 wb[B8 ? 1 : 2][TN16];     // fp8: raw 16-byte chunks (both steps); 16-bit: fragments per step
    auto pp_barrier = [&]() {
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    };
    // fp8 with 8 x 4 MFMAs per step (the 128 x 64 wave tile): the weight fragments of the block are unpacked at the
    // end of the memory phase, which is shorter than the compute phase, so the compute phase issues its MFMAs back
    // to back (2-3% off the 4096 x 12288 x 3072 and 4096 x 3072 x 12288 projections). The 64 x 96 wave tile (4 x 6
    // MFMAs per step) unpacks only its first step there (1.7% off 4096 x 9216 x 3072) and the second between its
    // MFMAs: unpacking more there made its memory phase the longer one.
    constexpr int PRE = !B8 ? 0 : RR >= 8 ? 2 : 1;  // steps unpacked in the memory phase
    constexpr bool PRE_CVT = PRE > 0;
    u32x4 wcv[PRE_CVT ? PRE : 1][TN16];
    auto unpack = [&](const u32x4& r, int q) {
      const u32x2 lo = cvt_fp8x4<IS_F16>(r[2 * q]), hi = cvt_fp8x4<IS_F16>(r[2 * q + 1]);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    };
    auto memory_block = [&](uint32_t st_off) {
#pragma unroll
      for (int q = 0; q < 2; q++)
#pragma unroll
        for (int i = 0; i < RR; i++) xb[q][i] = rd(st_off + rx16[q] + i * 16 * 128);
#pragma unroll
      for (int q = 0; q < (B8 ? 1 : 2); q++)
#pragma unroll
        for (int j = 0; j < TN16; j++)
          wb[q][j] = B8 ? rd(st_off + rw16[j & 1] + (j >> 1) * 32 * 64) : rd(st_off + rw16[q] + j * 16 * 128);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if constexpr (PRE_CVT) {
#pragma unroll
        for (int q = 0; q < PRE; q++)
#pragma unroll
          for (int j = 0; j < TN16; j++) wcv[q][j] = unpack(wb[0][j], q);
      }
    };
    // LD: issue this wave's L loads of the block at kb into stage st between the MFMAs (half of them per step)
    auto compute_block = [&](bool ld, uint32_t kb, int st) {
      static_for<0, 2>([&](auto Q) {
        constexpr int q = decltype(Q)::value;
        if (LM && ld) {  // wave-uniform
          constexpr int PER = (L + 1) / 2, Q0 = q * PER, Q1 = Q0 + PER < L ? Q0 + PER : L;
          static_for<Q0, Q1>([&](auto QQ) { issue_one(QQ, kb, st); });
        }
        u32x4 w[TN16];
#pragma unroll
        for (int j = 0; j < TN16; j++) {
          if constexpr (PRE_CVT && q < PRE) {
            w[j] = wcv[q < PRE ? q : 0][j];
          } else if constexpr (B8) {
            w[j] = unpack(wb[0][j], q);
          } else {
            w[j] = wb[q][j];
          }
        }
#pragma unroll
        for (int i = 0; i < RR; i++)
#pragma unroll
          for (int j = 0; j < TN16; j++) acc[i][j] = mfma_16x16x32<IS_F16>(w[j], xb[q][i], acc[i][j]);
      });
    };
    // own loads of block t + 1 complete; blocks issued after it (up to S - 2 of them) may be in flight
    auto wait_next = [&](int t) {
      if (t + 1 >= nk) return;
      if (S >= 3 && t + 2 < nk) wait_vmcnt<(S >= 3 ? (S - 2) * L : 0)>();
      else wait_vmcnt<0>();
    };
    if (nk > 0 && LM == 1) {
      // Group 1 issues every load of the ring. Prologue: blocks 0 .. S - 1 into stages 0 .. S - 1. In its compute
      // phase of block t (interval 2t + 2) a group-1 wave loads block t + S into block t's stage, which both groups
      // have read by then (group 0 in interval 2t, group 1 in 2t + 1). A group-1 wave's loads of block t + 1 must
      // land before the barrier that ends interval 2t + 1 (group 0 reads block t + 1 in interval 2t + 2): it waits
      // for them after its memory phase of block t, when at most the blocks up to t + S - 1 have been issued.
      if (grp == 1) {
#pragma unroll
        for (int p = 0; p < S; p++)
          if (p < nk) issue(k_begin + (uint32_t)p * BK, p);
        if (nk >= S) wait_vmcnt<(S - 1) * L>();
        else wait_vmcnt<0>();
      }
      lds_barrier();
      if (grp == 1) pp_barrier();  // group 1 sits out interval 0
      int cur = 0;
      for (int t = 0; t < nk; ++t) {
        memory_block((uint32_t)(cur * STAGE));
        if (grp == 1 && t + 1 < nk) {
          if (S >= 3 && t + S - 1 < nk) wait_vmcnt<(S >= 3 ? (S - 2) * L : 0)>();
          else wait_vmcnt<0>();
        }
        pp_barrier();
        compute_block(grp == 1 && t + S < nk, k_begin + (uint32_t)(t + S) * BK, cur);
        if (!(grp == 1 && t + 1 == nk)) pp_barrier();  // both groups pass the same number of barriers
        cur = cur + 1 == S ? 0 : cur + 1;
      }
    } else if (nk > 0) {
#pragma unroll
      for (int p = 0; p < S - 1; p++)
        if (p < nk) issue(k_begin + (uint32_t)p * BK, p);
      if (S >= 3 && nk >= 2) wait_vmcnt<(S >= 3 ? (S - 2) * L : 0)>();
      else wait_vmcnt<0>();
      lds_barrier();
      if (grp == 1) pp_barrier();  // group 1 sits out interval 0
      int cur = 0;
      for (int t = 0; t < nk; ++t) {
        const uint32_t cur_off = (uint32_t)(cur * STAGE);
        const int ahead = cur + S - 1 >= S ? cur - 1 : cur + S - 1;  // stage of block t + S - 1
        if (t + S - 1 < nk) issue(k_begin + (uint32_t)(t + S - 1) * BK, ahead);
        memory_block(cur_off);
        wait_next(t);
        pp_barrier();
        compute_block(false, 0u, 0);
        wait_next(t);
        if (!(grp == 1 && t + 1 == nk)) pp_barrier();  // both groups pass the same number of barriers
        cur = cur + 1 == S ? 0 : cur + 1;
      }
    }
  } else if (nk > 0) {
    // prologue: the first S blocks (or all of them)
#pragma unroll
    for (int p = 0; p < S; p++)
      if (p < nk) issue(k_begin + (uint32_t)p * BK, p);
    if (nk >= S) wait_vmcnt<(S - 1) * L>();
    else wait_vmcnt<0>();
    lds_barrier();
    read_x(0, 0, xf[0]);
    read_w(0, 0, wr[0]);

    int cur = 0;
    for (int it = 0; it < nk; ++it) {
      const uint32_t cur_off = (uint32_t)(cur * STAGE);
      const int nxt = cur + 1 == S ? 0 : cur + 1;
      const uint32_t nxt_off = (uint32_t)(nxt * STAGE);
      static_for<0, 4>([&](auto SI) {
        constexpr int s = decltype(SI)::value;
        if constexpr (s < 3) {
          read_x(cur_off, s + 1, xf[(s + 1) & 1]);
          if constexpr (B8) {
            if constexpr (s == 1) read_w(cur_off, 1, wr[1]);
          } else {
            read_w(cur_off, s + 1, wr[(s + 1) & 1]);
          }
        } else {
          // every wave has its last fragments of this block; block it + 1 must be complete
          if (it + S - 1 < nk) wait_vmcnt<(S - 2) * L>();
          else wait_vmcnt<0>();
          lds_barrier();
          if (it + S < nk) issue(k_begin + (uint32_t)(it + S) * BK, cur);
          if (it + 1 < nk) {
            read_x(nxt_off, 0, xf[0]);
            read_w(nxt_off, 0, wr[0]);
          }
        }
        u32x4 wf[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
          if constexpr (B8) {
            const u32x4 q = wr[s >> 1][j];
            const u32x2 lo = cvt_fp8x4<IS_F16>(q[(s & 1) * 2]), hi = cvt_fp8x4<IS_F16>(q[(s & 1) * 2 + 1]);
            wf[j] = u32x4{lo.x, lo.y, hi.x, hi.y};
          } else {
            wf[j] = wr[s & 1][j];
          }
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++) acc[i][j] = mfma_32x32x16<IS_F16>(wf[j], xf[s & 1][i], acc[i][j]);
      });
      cur = nxt;
    }
  }

  if constexpr (B8) {
    // NaN in the accumulators: only a NaN weight code (or a non-finite input) makes one. Recompute this
    // wave's tile with the shader's decoding of every byte (0x7f / 0xff -> +-480).
    float probe = 0.0f;
#pragma unroll
    for (int i = 0; i < RR; i++)
#pragma unroll
      for (int j = 0; j < (PP ? TN16 : TN); j++)
#pragma unroll
        for (int v = 0; v < (PP ? 4 : 16); v++) probe += acc[i][j][v] * 0.0f;
    if (__ballot(probe != probe) != 0) {
#pragma unroll
      for (int i = 0; i < RR; i++)
#pragma unroll
        for (int j = 0; j < (PP ? TN16 : TN); j++) acc[i][j] = AccT{};
      if constexpr (PP) {
        // 16x16x32 steps of 32 k: lane group g takes k0 + 8 g; the last step of a slice may hold only 16 k
        for (uint32_t k0 = k_begin; k0 < k_end; k0 += 32) {
          const uint32_t kk = k0 + 8 * g16;
          const bool in = kk < k_end;
          const uint32_t kkw = kk >= a.kwrap2 ? kk - a.kwrap2 : kk >= a.kwrap ? kk - a.kwrap : kk;  // weights' k
          u32x4 xr[RR];
          u32x4 wv[TN16];
#pragma unroll
          for (int i = 0; i < RR; i++) {
            const uint32_t row = row0 + wm * WTM + i * 16 + r16;
            const uint32_t o = row < a.m && in ? (row * a.x_stride + kk) * 2 : kInvalid;
            xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
          }
#pragma unroll
          for (int j = 0; j < TN16; j++) {
            const uint32_t col = col0 + wn * WTN + j * 16 + r16;
            const uint32_t o = col < a.n && in ? col * a.w_stride + kkw : kInvalid;
            const u32x2 raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, 0));
            const u32x2 lo = fp8x4_to_16<IS_F16>(raw.x), hi = fp8x4_to_16<IS_F16>(raw.y);
            wv[j] = u32x4{lo.x, lo.y, hi.x, hi.y};
          }
#pragma unroll
          for (int i = 0; i < RR; i++)
#pragma unroll
            for (int j = 0; j < TN16; j++) acc[i][j] = mfma_16x16x32<IS_F16>(wv[j], xr[i], acc[i][j]);
        }
      } else {
        for (uint32_t k0 = k_begin; k0 < k_end; k0 += 16) {
          const uint32_t kk = k0 + 8 * h;  // 8 k per lane half; k_end - k0 >= 16 (multiples of 16)
          const uint32_t kkw = kk >= a.kwrap2 ? kk - a.kwrap2 : kk >= a.kwrap ? kk - a.kwrap : kk;  // weights' k
          u32x4 xr[TM];
          u32x4 wv[TN];
#pragma unroll
          for (int i = 0; i < TM; i++) {
            const uint32_t row = row0 + wm * WTM + i * 32 + l32;
            const uint32_t o = row < a.m ? (row * a.x_stride + kk) * 2 : kInvalid;
            xr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
          }
#pragma unroll
          for (int j = 0; j < TN; j++) {
            const uint32_t col = col0 + wn * WTN + j * 32 + l32;
            const uint32_t o = col < a.n ? col * a.w_stride + kkw : kInvalid;
            const u32x2 raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, 0));
            const u32x2 lo = fp8x4_to_16<IS_F16>(raw.x), hi = fp8x4_to_16<IS_F16>(raw.y);
            wv[j] = u32x4{lo.x, lo.y, hi.x, hi.y};
          }
#pragma unroll
          for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = mfma_32x32x16<IS_F16>(wv[j], xr[i], acc[i][j]);
        }
      }
    }
  }

  // the accumulators as runs of 4 consecutive columns: block row ri (row ri * RS + lrow of the wave tile), run rc
  // (columns ccol(rc) + lcol .. + 3)
  const int lrow = PP ? r16 : l32, lcol = PP ? 4 * g16 : 4 * h;
  auto ccol = [](int rc) { return PP ? rc * 16 : (rc >> 2) * 32 + 8 * (rc & 3); };
  auto av = [&](int ri, int rc) -> f32x4 {
    if constexpr (PP) {
      return acc[ri][rc];
    } else {
      const int j = rc >> 2, q = rc & 3;
      return f32x4{acc[ri][j][4 * q], acc[ri][j][4 * q + 1], acc[ri][j][4 * q + 2], acc[ri][j][4 * q + 3]};
    }
  };

  if (a.rsplits > 1) {
    // ---- split-K slice: raw sums (no scale) to the partial-sum plane of this slice
    const size_t plane = (size_t)a.m * a.n;
    const bool vec = (a.n & 3u) == 0u;
#pragma unroll
    for (int i = 0; i < RR; i++) {
      const uint32_t row = row0 + wm * WTM + i * RS + lrow;
      if (row >= a.m) continue;
#pragma unroll
      for (int rc = 0; rc < RC; rc++) {
        const uint32_t c0 = col0 + wn * WTN + ccol(rc) + lcol;
        float* p = a.part + z * plane + (size_t)row * a.n + c0;
        const f32x4 v = av(i, rc);
        if (vec && c0 + 3 < a.n) {
          *(f32x4*)p = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (c0 + e < a.n) p[e] = v[e];
        }
      }
    }
    return;
  }

  // ---- fused q/k epilogue (the q/k path of attend(), src/model/block.ts:53-56): a head of 128 columns is
  // the 64 columns of waves wn and wn ^ 1 (WTN = 64, the tile aligned to heads), so each row's sum of squares
  // is the two waves' partial sums, exchanged through LDS. Every wave of the workgroup takes this branch (the
  // tile lies wholly inside the q/k columns), so the barriers below are uniform. Not in the ping-pong kernels:
  // their 128 accumulators and double operand sets leave no registers for it (it made them spill).
  if constexpr (WTN == 64 && WAVES_N % 2 == 0 && !PP) {
    if (a.qk_cols && col0 < a.qk_cols) {
      const bool has_bias_qk = (a.flags & WE_EPI_BIAS_BIT) != 0;
      float ss[TM];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        ss[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int v = 0; v < 16; v++) {
            float t = acc[i][j][v] * a.scale;
            if (has_bias_qk) t += a.bias[col0 + wn * WTN + j * 32 + 8 * (v >> 2) + 4 * h + (v & 3)];
            acc[i][j][v] = t;
            ss[i] += t * t;
          }
        ss[i] += __shfl_xor(ss[i], 32, 64);  // lanes l32 and l32 + 32 hold the same row
      }
      float* red = (float*)lds;  // [BM rows][WAVES_N] partial sums; every wave is done with the stages
      lds_barrier();
      if (h == 0) {
#pragma unroll
        for (int i = 0; i < TM; i++) red[(wm * WTM + i * 32 + l32) * WAVES_N + wn] = ss[i];
      }
      lds_barrier();
      const uint32_t hcol0 = (uint32_t)(wn & 1) * 64;  // this wave's first column inside its head
      const float* nw = (col0 + wn * WTN < a.q_cols ? a.qk_norm_q : a.qk_norm_k) + hcol0;
      const std::integral_constant<bool, YT == F16> tag;
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const uint32_t rloc = wm * WTM + i * 32 + l32;
        const float tot = red[rloc * WAVES_N + (wn & ~1)] + red[rloc * WAVES_N + (wn | 1)];
        const float inv = 1.0f / sqrtf(tot / 128.0f + a.qk_eps);
        const uint32_t row = row0 + rloc;
        // padding rows of the last M tile (row >= M) form no table address: the checked span of cos / sin
        // ends at row M - 1
        const bool rot = a.qk_cos && row >= a.qk_rope_from && row < a.m;
        const size_t trow = rot ? (size_t)(row - a.qk_rope_from) * 64 : 0;
        const size_t yrow = (size_t)a.y_offset + (size_t)row * a.y_stride + col0 + wn * WTN;
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const uint32_t cl = j * 32 + 8 * q + 4 * h;  // column inside the wave's 64 (and in the head: + hcol0)
            const f32x4 wv = *(const f32x4*)(nw + cl);
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = acc[i][j][4 * q + e] * inv * (a.qk_offset + wv[e]);
            if (rot) {
              const uint32_t pr = (hcol0 + cl) / 2;  // pairs (y0, y1) and (y2, y3)
              const f32x2 c2 = *(const f32x2*)(a.qk_cos + trow + pr), s2 = *(const f32x2*)(a.qk_sin + trow + pr);
#pragma unroll
              for (int p = 0; p < 2; p++) {
                const float u = y[2 * p], v = y[2 * p + 1];
                y[2 * p] = u * c2[p] - v * s2[p];
                y[2 * p + 1] = v * c2[p] + u * s2[p];
              }
            }
            if (row < a.m) {
              if constexpr (YT == F32) {
                *(f32x4*)((float*)a.y + yrow + cl) = f32x4{y[0], y[1], y[2], y[3]};
              } else {
                *(u32x2*)((uint16_t*)a.y + yrow + cl) = u32x2{pack2(y[0], y[1], tag), pack2(y[2], y[3], tag)};
              }
            }
          }
      }
      return;
    }
  }

  // ---- epilogue over the runs of 4 columns (av, ccol, lcol, lrow above)
  const bool accum = (a.flags & WE_EPI_ACCUMULATE_BIT) != 0;
  const bool has_bias = (a.flags & WE_EPI_BIAS_BIT) != 0;
  const bool gelu = (a.flags & WE_EPI_GELU_BIT) != 0;
  const size_t zrow = (a.flags & WE_EPI_SPLIT_K_BIT) ? (size_t)z * a.m : 0;  // the reference's partial rows
  const void* aux = a.mul ? a.res : nullptr;  // the product epilogue's second operand
  const void* addend = a.mul ? nullptr : a.res ? a.res : (accum ? a.y : nullptr);
  // Fast path (uniform branch): the wave's whole sub-tile lies inside y, 4-value stores are allowed, and
  // there is no bias; plain stores, the gated residual (gate and addend both present) or a product epilogue:
  // per row one base pointer, stores at constant offsets from it, GELU, gating and the product chosen outside
  // the loops (the general path below computes every case per value).
  const uint32_t wrow0 = row0 + wm * WTM, wcol0 = col0 + wn * WTN;
  const bool plain = !addend && !a.gate && !aux, gated = addend && a.gate;
  if (a.vec_store && !has_bias && (plain || gated || aux) && wrow0 + WTM <= a.m && wcol0 + WTN <= a.n) {
    // MODE 0 plain, 1 gated residual, 2 swiglu product, 3 sigmoidGate product
    auto fast = [&](auto GELU, auto MODE) {
      constexpr int MD = decltype(MODE)::value;
      constexpr bool GT = MD == 1;
      const void* other = MD == 1 ? addend : aux;  // the operand read beside the accumulators
      f32x4 gv[RC];  // the lane's gate values, the same for every row
      if constexpr (GT) {
#pragma unroll
        for (int rc = 0; rc < RC; rc++) gv[rc] = *(const f32x4*)(a.gate + wcol0 + lcol + ccol(rc));
      }
#pragma unroll
      for (int i = 0; i < RR; i++) {
        const size_t yrow = (size_t)a.y_offset + (zrow + wrow0 + i * RS + lrow) * (size_t)a.y_stride + wcol0 + lcol;
        if constexpr (YT == F32) {
          float* p = (float*)a.y + yrow;
          const float* r0 = MD ? (const float*)other + yrow : nullptr;
#pragma unroll
          for (int rc = 0; rc < RC; rc++) {
            const f32x4 v = av(i, rc);
            f32x4 r;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const float t = v[e] * a.scale;
              r[e] = decltype(GELU)::value ? gelu_tanh(t) : t;
            }
            if constexpr (GT) r = *(const f32x4*)(r0 + ccol(rc)) + gv[rc] * r;
            if constexpr (MD >= 2) {
              const f32x4 ax = *(const f32x4*)(r0 + ccol(rc));
#pragma unroll
              for (int e = 0; e < 4; e++) r[e] = mul_epilogue(MD - 1, ax[e], r[e]);
            }
            *(f32x4*)(p + ccol(rc)) = r;
          }
        } else if (PP && MD == 0 && a.store16) {
          // Whole rows through LDS. In the MFMA layout one store instruction covers 16 rows with 32 bytes each (4
          // lanes of 8 bytes per row); staged RS rows at a time in the wave's own LDS region (every wave is past
          // its last fragment read: the ping-pong loop ends on a barrier that follows the other group's last
          // memory phase), the stores become 16 bytes per lane over whole row segments. Measured with 32x32 blocks:
          // 3% off the 4096 x 12288 x 3072 up-projection. Rows are padded by 16 bytes, which puts the rows of a
          // write on distinct banks.
          constexpr int P = WTN * 2 + 16, CPR = WTN / 8;  // row pitch in bytes, 16-byte chunks per row
          static_assert((RS * CPR) % 64 == 0, "whole rounds of 64 lanes");
          char* reg = lds + wave * (32 * P);
          const std::integral_constant<bool, YT == F16> tag;
#pragma unroll
          for (int rc = 0; rc < RC; rc++) {
            const f32x4 v = av(i, rc);
            float t[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
              t[e] = v[e] * a.scale;
              if constexpr (decltype(GELU)::value) t[e] = gelu_tanh(t[e]);
            }
            *(u32x2*)(reg + lrow * P + (ccol(rc) + lcol) * 2) = u32x2{pack2(t[0], t[1], tag), pack2(t[2], t[3], tag)};
          }
          uint16_t* yb = (uint16_t*)a.y + (size_t)a.y_offset + (zrow + wrow0 + i * RS) * (size_t)a.y_stride + wcol0;
#pragma unroll
          for (int s = 0; s < RS * CPR / 64; s++) {  // RS rows x CPR chunks in rounds of 64 lanes
            const int idx = s * 64 + lane, r = idx / CPR, c = idx % CPR;
            *(u32x4*)(yb + (size_t)r * a.y_stride + c * 8) = *(const u32x4*)(reg + r * P + c * 16);
          }
        } else {
          uint16_t* p = (uint16_t*)a.y + yrow;
          const uint16_t* r0 = MD ? (const uint16_t*)other + yrow : nullptr;
          const std::integral_constant<bool, YT == F16> tag;
#pragma unroll
          for (int rc = 0; rc < RC; rc++) {
            const f32x4 v = av(i, rc);
            float t[4];
            u32x2 old = {0u, 0u};
            if constexpr (MD != 0) old = *(const u32x2*)(r0 + ccol(rc));
#pragma unroll
            for (int e = 0; e < 4; e++) {
              t[e] = v[e] * a.scale;
              if constexpr (decltype(GELU)::value) t[e] = gelu_tanh(t[e]);
              if constexpr (MD != 0) {
                const uint32_t hb = ((e < 2 ? old.x : old.y) >> (16 * (e & 1))) & 0xffffu;
                const float o = YT == BF16 ? bf16_to_f32((uint16_t)hb) : f16_to_f32((uint16_t)hb);
                t[e] = GT ? o + gv[rc][e] * t[e] : mul_epilogue(MD - 1, o, t[e]);
              }
            }
            *(u32x2*)(p + ccol(rc)) = u32x2{pack2(t[0], t[1], tag), pack2(t[2], t[3], tag)};
          }
        }
      }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if (aux) {  // the runtime refuses GELU with a product epilogue
      if (a.mul == 1u) fast(std::false_type{}, std::integral_constant<int, 2>{});
      else fast(std::false_type{}, std::integral_constant<int, 3>{});
    } else if (gated) {
      if (gelu) fast(std::true_type{}, I1{});
      else fast(std::false_type{}, I1{});
    } else {
      if (gelu) fast(std::true_type{}, I0{});
      else fast(std::false_type{}, I0{});
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < RR; i++) {
    const uint32_t row = row0 + wm * WTM + i * RS + lrow;
    if (row >= a.m) continue;
    const size_t yrow = (size_t)a.y_offset + (zrow + row) * (size_t)a.y_stride;
#pragma unroll
    for (int rc = 0; rc < RC; rc++) {
      {
        const uint32_t c0 = col0 + wn * WTN + ccol(rc) + lcol;
        const f32x4 av4 = av(i, rc);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float t = av4[e] * a.scale;
          if (has_bias) t += a.bias[c0 + e < a.n ? c0 + e : 0];
          if (gelu) t = gelu_tanh(t);
          if (a.gate) t *= a.gate[c0 + e < a.n ? c0 + e : 0];
          if (aux && c0 + e < a.n) t = mul_epilogue(a.mul, load1<YT>(aux, yrow + c0 + e), t);
          v[e] = t;
        }
        if (a.vec_store && c0 + 3 < a.n) {
          store4<YT>(a, yrow + c0, v, addend);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (c0 + e < a.n) store1<YT>(a, yrow + c0 + e, v[e], addend);
        }
      }
    }
  }
}

// Sum of the split-K partial planes, then the epilogue of the GEMM (scale, bias, GELU, accumulate, output
// type): one thread per 4 consecutive outputs of a row, slices added in slice order.
// XCD (BM, BN > 0): the slices of a tile ran on one XCD (workgroups go round-robin over the 8 XCDs, and the slice
// index adds a multiple of 8 tiles to the workgroup id), so each reduce workgroup takes a part of a tile of its own
// XCD and reads the slices there. Otherwise one thread per 4 consecutive outputs in row-major order.
template <int YT, int BM = 0, int BN = 0>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(FastArgs a) {
  uint32_t row, c0;
  if constexpr (BM > 0) {
    constexpr uint32_t ITEMS = BM * BN / 4, Q = ITEMS / 256;  // reduce workgroups per tile
    const uint32_t b = blockIdx.x, j = b >> 3;
    const uint32_t pid = (b & 7u) * (a.tiles_m * a.tiles_n / 8) + j / Q;  // a tile the GEMM ran on this XCD
    const uint32_t i = (j % Q) * 256 + threadIdx.x;
    constexpr uint32_t GROUP_M = 4;
    const uint32_t per_group = GROUP_M * a.tiles_n, first_m = (pid / per_group) * GROUP_M;
    const uint32_t gsize = min(a.tiles_m - first_m, GROUP_M), in_group = pid % per_group;
    row = (first_m + in_group % gsize) * BM + i / (BN / 4);
    c0 = (in_group / gsize) * BN + (i % (BN / 4)) * 4;
    if (row >= a.m || c0 >= a.n) return;
  } else {
    const uint32_t groups = (a.n + 3) / 4;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)a.m * groups) return;
    row = (uint32_t)(idx / groups);
    c0 = (uint32_t)(idx % groups) * 4;
  }
  const size_t plane = (size_t)a.m * a.n;
  const float* p = a.part + (size_t)row * a.n + c0;
  const bool full = c0 + 3 < a.n;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (full && (a.n & 3u) == 0u) {
    // up to 8 slices' loads in flight at once, added in slice order
    for (uint32_t z0 = 0; z0 < a.rsplits; z0 += 8) {
      f32x4 t[8];
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (z0 + u < a.rsplits) t[u] = *(const f32x4*)(p + (z0 + u) * plane);
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (z0 + u < a.rsplits)
#pragma unroll
          for (int e = 0; e < 4; e++) v[e] += t[u][e];
    }
  } else {
    for (uint32_t z = 0; z < a.rsplits; z++, p += plane)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (c0 + e < a.n) v[e] += p[e];
  }
  const bool accum = (a.flags & WE_EPI_ACCUMULATE_BIT) != 0;
  const bool has_bias = (a.flags & WE_EPI_BIAS_BIT) != 0;
  const bool gelu = (a.flags & WE_EPI_GELU_BIT) != 0;
  const void* aux = a.mul ? a.res : nullptr;
  const void* addend = a.mul ? nullptr : a.res ? a.res : (accum ? a.y : nullptr);
  const size_t yrow = (size_t)a.y_offset + (size_t)row * a.y_stride;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float t = v[e] * a.scale;
    if (has_bias) t += a.bias[c0 + e < a.n ? c0 + e : 0];
    if (gelu) t = gelu_tanh(t);
    if (a.gate) t *= a.gate[c0 + e < a.n ? c0 + e : 0];
    if (aux && c0 + e < a.n) t = mul_epilogue(a.mul, load1<YT>(aux, yrow + c0 + e), t);
    v[e] = t;
  }
  if (a.vec_store && full) {
    store4<YT>(a, yrow + c0, v, addend);
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (c0 + e < a.n) store1<YT>(a, yrow + c0 + e, v[e], addend);
  }
}

// Does the split-K reduce pass read each tile's partial sums from the L2 of the XCD that computed them? With a
// multiple of 8 tiles and at most 16 MiB of weights (2 MiB per XCD, so the weight stream does not push the sums
// out). `on` 0 (Tuning::gemm_reduce_xcd): never (measurements).
static bool reduce_in_l2(uint64_t tiles, uint64_t weight_bytes, int on) {
  return on && tiles % 8 == 0 && weight_bytes <= (16u << 20);
}

template <int BM, int BN, int WM, int WN, bool IS_F16, int BT, int S, bool PP = false>
static hipError_t launch_fast_cfg(FastArgs a, uint32_t splits, int reduce_xcd, hipStream_t s) {
  a.tiles_m = (a.m + BM - 1) / BM;
  a.tiles_n = (a.n + BN - 1) / BN;
  uint32_t tiles = a.tiles_m * a.tiles_n;
  if (a.grp) {  // the second GEMM's tiles follow the first's
    a.g.tiles_m = (a.g.m + BM - 1) / BM;
    a.grp_first = tiles;
    tiles += a.g.tiles_m * a.tiles_n;
  }
  const dim3 grid(tiles, splits), block(WM * WN * 64);
  if (a.rsplits > 1) {
    // slices store raw f32 sums (the output type does not matter to them), then one reduce pass
    hipLaunchKernelGGL((gemm_lds_kernel<BM, BN, WM, WN, IS_F16, BT, S, F32, PP>), grid, block, 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the slices' placement: the GEMM's tile id comes from xcd_remap_f, so with T tiles, T a multiple of 8, XCD x
    // ran tiles [x T / 8, (x + 1) T / 8) of every slice (slice z adds z T, a multiple of 8, to the linear id). The
    // reduce pass then reads each tile on its XCD, so every L2 holds only its own tiles' partial sums (the
    // row-major pass pulled all of them into every L2, evicting the GEMM's own inputs). Each output is the same
    // sum in slice order either way. Measured on MI355X (graph replays): 64 x 3072 x 3072 fp8 10.9 -> 9.2 us per
    // call, 12.2 -> 11.2 us with the weights streamed from HBM, 16 x 3072 x 3072 8.5 -> 8.1 us; but 64 x 3072 x
    // 12288 (37.7 MB of weights) 19.5 -> 20.2 us, so only up to 16 MB of weights (2 MB per XCD).
    // reduce_xcd 0: the row-major mapping (measurements)
    static_assert((BM * BN / 4) % 256 == 0, "whole reduce workgroups per tile");
    if (reduce_in_l2(tiles, a.w_bytes, reduce_xcd)) {
      const dim3 rg(tiles * (BM * BN / 4 / 256));
      switch (a.y_dtype) {
        case F32: hipLaunchKernelGGL((splitk_reduce_kernel<F32, BM, BN>), rg, dim3(256), 0, s, a); break;
        case F16: hipLaunchKernelGGL((splitk_reduce_kernel<F16, BM, BN>), rg, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL((splitk_reduce_kernel<BF16, BM, BN>), rg, dim3(256), 0, s, a); break;
      }
      return hipGetLastError();
    }
    const size_t threads = (size_t)a.m * ((a.n + 3) / 4);
    const dim3 rg((unsigned)((threads + 255) / 256));
    switch (a.y_dtype) {
      case F32: hipLaunchKernelGGL(splitk_reduce_kernel<F32>, rg, dim3(256), 0, s, a); break;
      case F16: hipLaunchKernelGGL(splitk_reduce_kernel<F16>, rg, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL(splitk_reduce_kernel<BF16>, rg, dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
  }
  switch (a.y_dtype) {
    case F32: hipLaunchKernelGGL((gemm_lds_kernel<BM, BN, WM, WN, IS_F16, BT, S, F32, PP>), grid, block, 0, s, a); break;
    case F16: hipLaunchKernelGGL((gemm_lds_kernel<BM, BN, WM, WN, IS_F16, BT, S, F16, PP>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_lds_kernel<BM, BN, WM, WN, IS_F16, BT, S, BF16, PP>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

template <bool IS_F16, int BT>
static hipError_t launch_fast_types(const FastArgs& a, uint32_t splits, int cfg, int rx, hipStream_t s) {
  constexpr bool B8 = BT == FP8;
  switch (cfg) {
    // ping-pong schedule, 2 x 4 waves (128 x 64 each): measured on MI355X the fastest layout for fp8
    // and 16-bit weights
    case GEMM_CFG_256x256: return launch_fast_cfg<256, 256, 2, 4, IS_F16, BT, B8 ? 3 : 2, true>(a, splits, rx, s);
    case GEMM_CFG_256x128: return launch_fast_cfg<256, 128, 4, 2, IS_F16, BT, 3>(a, splits, rx, s);
    // 256 x 192 (4 x 2 waves of 64 x 96, ping-pong): 4096 x 3072 outputs are exactly 256 tiles
    case GEMM_CFG_256x192: return launch_fast_cfg<256, 192, 4, 2, IS_F16, BT, B8 ? 3 : 2, true>(a, splits, rx, s);
    case GEMM_CFG_128x128: return launch_fast_cfg<128, 128, 2, 2, IS_F16, BT, 3>(a, splits, rx, s);
    case GEMM_CFG_64x64: return launch_fast_cfg<64, 64, 2, 2, IS_F16, BT, 3>(a, splits, rx, s);
    default: return launch_fast_cfg<32, 64, 1, 2, IS_F16, BT, 3>(a, splits, rx, s);
  }
}

namespace {

// Do the operands qualify for the fast path? (16-bit activations, fp8 or matching 16-bit weights, 16-byte
// aligned rows, K a multiple of 16, operand extents under the 32-bit buffer offsets.)
bool fast_supported(const GemmLaunch& L, uint32_t kc) {
  if (L.conv_width) return false;  // the 3x3 convolution input gathers x in the general kernel
  const bool f16 = L.x_dtype == F16;
  if (!(L.x_dtype == BF16 || L.x_dtype == F16)) return false;
  if (!(L.w_dtype == FP8 || (f16 ? L.w_dtype == F16 : L.w_dtype == BF16))) return false;
  const int wb = L.w_dtype == FP8 ? 1 : 2;
  if (L.k % 16 || kc % 16) return false;
  if (((uintptr_t)L.x + (uint64_t)L.x_offset * 2) % 16 || ((uintptr_t)L.w + (uint64_t)L.w_offset * wb) % 16 ||
      (L.x_stride * 2) % 16 || (L.w_stride * wb) % 16)
    return false;
  if (L.k_wrap && (L.k_wrap % BK || L.k % L.k_wrap || L.k / L.k_wrap > 3)) return false;
  const uint64_t xb = L.k ? ((uint64_t)(L.m - 1) * L.x_stride + L.k) * 2 : 0;
  const uint64_t wbytes = L.k ? ((uint64_t)(L.n - 1) * L.w_stride + (L.k_wrap ? L.k_wrap : L.k)) * wb : 0;
  return xb < kInvalid && wbytes < kInvalid;
}

constexpr uint32_t kCUs = 256;

// readable weight bytes of a GEMM (FastArgs::w_bytes)
uint64_t weight_extent(const GemmLaunch& L) {
  const int wb = L.w_dtype == FP8 ? 1 : 2;
  return L.k ? ((uint64_t)(L.n - 1) * L.w_stride + (L.k_wrap ? L.k_wrap : L.k)) * wb : 0;
}

// Tile shape by predicted speed: score = base x (tiles / slots) / (time in rounds). base is the tile shape's own
// speed relative to 256 x 256 (one per CU, the fastest per FLOP) at full occupancy; a full round of tiles costs 1,
// the last, partly filled round 0.6 + 0.3 f (f = the fraction of slots it fills). The chip runs at its power
// limit, so tiles run faster when fewer CUs are busy, and a partial round costs far more than its share but less
// than a full one. Fitted to the tile sweep (bench.py --sweep: bf16 activations and output, fp8 weights unless
// named, M = 4096 and 8740). With fp8 weights 256 x 192 runs at 0.90 of 256 x 256's speed, 128 x 128 (two per CU)
// at 0.81, 256 x 128 at 0.77. The tail term decides two shapes: 4096 x 3072 x 12288 (256 x 256: one round at
// f = 0.75) stays with 256 x 256 (1288 against 1254 TFLOP/s for 256 x 192), while 4096 x 9216 x 3072 (256 x 256:
// two full rounds and one at f = 0.25) goes to 256 x 192 (three full rounds; 7% faster). With 16-bit weights
// 128 x 128 tiles fit one per CU only and lose to the ping-pong tiles (4096 x 9216 x 3072 bf16: 801 against 1085
// TFLOP/s), so only the two 256-row shapes compete there, 256 x 192 at 0.95.
int pick_fast_cfg(uint32_t m, uint32_t n, uint32_t splits, bool w8) {
  if (m <= 32) return GEMM_CFG_32x64;
  if (m <= 64) return GEMM_CFG_64x64;
  struct Cand {
    int cfg;
    uint32_t bm, bn, per_cu;
    double base;
  };
  const Cand cands[] = {{GEMM_CFG_256x256, 256, 256, 1, 1.00}, {GEMM_CFG_256x192, 256, 192, 1, w8 ? 0.90 : 0.95},
                        {GEMM_CFG_128x128, 128, 128, 2, 0.81}, {GEMM_CFG_256x128, 256, 128, 1, 0.77}};
  int best = GEMM_CFG_128x128;
  double best_score = -1.0;
  for (const Cand& c : cands) {
    if (c.bm == 256 && m < 256) continue;
    if (!w8 && c.cfg != GEMM_CFG_256x256 && c.cfg != GEMM_CFG_256x192) continue;
    const uint64_t tiles = (uint64_t)((m + c.bm - 1) / c.bm) * ((n + c.bn - 1) / c.bn) * splits;
    const uint64_t slots = (uint64_t)kCUs * c.per_cu;
    const uint64_t full = tiles / slots, rest = tiles % slots;
    const double rounds = (double)full + (rest ? 0.6 + 0.3 * (double)rest / (double)slots : 0.0);
    const double score = c.base * ((double)tiles / (double)slots) / rounds;
    if (score > best_score + 1e-9) {
      best_score = score;
      best = c.cfg;
    }
  }
  return best;
}

uint32_t cfg_bm(int cfg) {
  return cfg == GEMM_CFG_32x64 ? 32 : cfg == GEMM_CFG_64x64 ? 64 : cfg == GEMM_CFG_128x128 ? 128 : 256;
}
uint32_t cfg_bn(int cfg) {
  return cfg == GEMM_CFG_256x256   ? 256
         : cfg == GEMM_CFG_256x192 ? 192
         : cfg == GEMM_CFG_256x128 || cfg == GEMM_CFG_128x128 ? 128
                                                               : 64;
}

}  // namespace

GemmReducePlan gemm_reduce_plan(const GemmLaunch& L, uint32_t force_splits) {
  GemmReducePlan p{1, L.k, 0, -1};
  if (L.generic || (L.splits > 1) || (L.flags & WE_EPI_SPLIT_K_BIT) || L.m == 0 || L.n == 0) return p;
  if (L.k < 512 || !fast_supported(L, L.k)) return p;
  const int cfg = L.cfg >= 0 ? L.cfg : pick_fast_cfg(L.m, L.n, 1, L.w_dtype == FP8);
  const uint64_t tiles = (uint64_t)((L.m + cfg_bm(cfg) - 1) / cfg_bm(cfg)) * ((L.n + cfg_bn(cfg) - 1) / cfg_bn(cfg));
  uint32_t rs;
  if (L.m <= 64) {
    if (tiles >= kCUs / 2) return p;
    // about one workgroup per CU; where the reduce pass reads the partial sums from L2 (reduce_in_l2), up to two
    // (at most 8 slices where one per CU needs fewer). Measured, 8 slices against one workgroup per CU, weights
    // cached / streamed from HBM: 64 x 3072 x 3072 9.24 / 10.22 -> 8.99 / 9.98 us, 16 x 3072 x 3072 8.07 / 9.05 ->
    // 7.61 / 8.67 us, 64 x 4096 x 4096 10.92 / 12.47 -> 10.23 / 11.78 us (12 slices of 64 x 3072 x 3072: 10.5 us);
    // without the L2 reduce more slices only add partial-sum traffic (64 x 6144 x 3072: 14.1 -> 15.9 us)
    const uint64_t one = (kCUs + tiles - 1) / tiles, two = (2 * kCUs + tiles - 1) / tiles;
    rs = reduce_in_l2(tiles, weight_extent(L), L.reduce_xcd) ? (uint32_t)std::max<uint64_t>(one, std::min<uint64_t>(8, two))
                                               : (uint32_t)one;
  } else {
    // larger M: split when the tiles fill less than half of the workgroup slots (M = 512, N = 3072:
    // 96 tiles of 128 x 128 for 512 slots), to about one workgroup per slot
    const uint64_t slots = (uint64_t)kCUs * (cfg == GEMM_CFG_128x128 ? 2 : 1);
    if (tiles * 2 > slots) return p;
    rs = (uint32_t)((slots + tiles - 1) / tiles);
    // with fp8 weights, M >= 256 and slices of at least 1024 k the slices run in 256 x 192 ping-pong tiles, about
    // one per CU: 512 x 3072 x 12288 58.2 -> 54.9 us against the 128 x 128 plan (6 slices, which the launch ran as
    // 192 workgroups of 256 x 192), same process, alternating order. At 512 x 3072 x 3072 (slices of 384 k) the
    // 128 x 128 plan stays: 30.3 against 31.4 us.
    if (L.cfg < 0 && L.m >= 256 && L.w_dtype == FP8) {
      const uint64_t t = (uint64_t)((L.m + 255) / 256) * ((L.n + 191) / 192);
      const uint32_t rs2 = (uint32_t)((kCUs + t - 1) / t);
      if (L.k / rs2 >= 1024) {
        p.rcfg = GEMM_CFG_256x192;
        rs = rs2;
      }
    }
  }
  rs = rs < L.k / 256 ? rs : L.k / 256;  // every slice keeps at least 256 of K
  if (force_splits) rs = force_splits < L.k / BK ? force_splits : L.k / BK;
  if (rs < 2) return p;
  const uint32_t kc = (L.k + rs * BK - 1) / (rs * BK) * BK;
  const uint32_t n_slices = (L.k + kc - 1) / kc;
  if (n_slices < 2) return p;
  p.rsplits = n_slices;
  p.rkc = kc;
  p.scratch_bytes = (size_t)n_slices * L.m * L.n * 4;
  return p;
}

bool gemm_qk_fusable(const GemmLaunch& L) {
  if (L.generic || L.splits > 1 || L.flags & ~WE_EPI_BIAS_BIT || L.mul || L.gate || L.res) return false;
  if (L.y_dtype == F32 || !fast_supported(L, L.k)) return false;
  if (gemm_reduce_plan(L, 0).rsplits > 1) return false;
  const int cfg = L.cfg >= 0 ? L.cfg : pick_fast_cfg(L.m, L.n, 1, L.w_dtype == FP8);
  // head-aligned tiles with 64-column waves outside the ping-pong kernels: 256 x 128 (4 x 2), 128 x 128 (2 x 2)
  if (cfg != GEMM_CFG_256x128 && cfg != GEMM_CFG_128x128) return false;
  const uint32_t bn = cfg_bn(cfg);
  return L.qk_cols % bn == 0 && L.q_cols % bn == 0 && L.qk_cols <= L.n && (L.y_stride % 4) == 0 &&
         (L.y_offset % 4) == 0 && ((uintptr_t)L.y % 16) == 0 && ((uintptr_t)L.qk_norm_q % 16) == 0 &&
         ((uintptr_t)L.qk_norm_k % 16) == 0 && ((uintptr_t)L.qk_cos % 8) == 0 && ((uintptr_t)L.qk_sin % 8) == 0 &&
         (!L.bias || ((uintptr_t)L.bias % 4) == 0);
}

namespace {

// The kernel arguments of one GEMM (no split-K slices, no tile pick yet).
FastArgs fast_args(const GemmLaunch& L, uint32_t kc) {
  const int wb = L.w_dtype == FP8 ? 1 : 2;
  const int yb = L.y_dtype == F32 ? 4 : 2;
  FastArgs a{};
  a.x = (const char*)L.x + (uint64_t)L.x_offset * 2;
  a.w = (const char*)L.w + (uint64_t)L.w_offset * wb;
  a.y = L.y;
  a.bias = L.bias;
  a.gate = L.gate;
  a.res = L.res;
  a.mul = (uint32_t)L.mul;
  a.qk_cols = L.qk_cols;
  a.q_cols = L.q_cols;
  a.qk_rope_from = L.qk_rope_from;
  a.qk_eps = L.qk_eps;
  a.qk_offset = L.qk_offset;
  a.qk_norm_q = L.qk_norm_q;
  a.qk_norm_k = L.qk_norm_k;
  a.qk_cos = L.qk_cos;
  a.qk_sin = L.qk_sin;
  a.x_bytes = L.k ? (uint32_t)(((uint64_t)(L.m - 1) * L.x_stride + L.k) * 2) : 0;
  a.w_bytes = (uint32_t)weight_extent(L);
  a.m = L.m;
  a.n = L.n;
  a.k = L.k;
  a.kwrap = L.k_wrap ? L.k_wrap : 0xffffffffu;
  a.kwrap2 = L.k_wrap ? 2 * L.k_wrap : 0xffffffffu;
  a.scale = L.scale;
  a.x_stride = L.x_stride;
  a.w_stride = L.w_stride;
  a.y_stride = L.y_stride;
  a.y_offset = L.y_offset;
  a.kc = kc;
  a.flags = L.flags;
  a.y_dtype = (uint32_t)L.y_dtype;
  a.vec_store = ((uintptr_t)L.y % (4 * yb) == 0 && (uintptr_t)L.res % (4 * yb) == 0 &&
                 (uintptr_t)L.gate % 16 == 0 && ((uint64_t)L.y_offset * yb) % (4 * yb) == 0 &&
                 ((uint64_t)L.y_stride * yb) % (4 * yb) == 0)
                    ? 1u
                    : 0u;
  a.store16 = ((uintptr_t)L.y % 16 == 0 && ((uint64_t)L.y_offset * yb) % 16 == 0 && ((uint64_t)L.y_stride * yb) % 16 == 0)
                  ? 1u
                  : 0u;
  return a;
}

}  // namespace

// Returns hipErrorNotSupported when the shape / dtypes / alignment are not for this path.
hipError_t gemm_fast_launch(const GemmLaunch& L, hipStream_t stream) {
  const bool reduce = L.rsplits > 1;
  const uint32_t splits = reduce ? L.rsplits : (L.splits < 1 ? 1 : L.splits);
  const uint32_t kc = reduce ? L.rkc : (splits > 1 ? L.kc : L.k);
  if (!fast_supported(L, kc)) return hipErrorNotSupported;
  const bool f16 = L.x_dtype == F16;
  FastArgs a = fast_args(L, kc);
  if (reduce) {
    if (!L.scratch) return hipErrorInvalidValue;
    a.part = (float*)L.scratch;
    a.rsplits = splits;
  }
  const int cfg = L.cfg >= 0                ? L.cfg
                  : reduce && L.rcfg >= 0 ? L.rcfg
                                          : pick_fast_cfg(L.m, L.n, splits, L.w_dtype == FP8);
  const int rx = L.reduce_xcd;
  if (f16) {
    if (L.w_dtype == FP8) return launch_fast_types<true, FP8>(a, splits, cfg, rx, stream);
    return launch_fast_types<true, F16>(a, splits, cfg, rx, stream);
  }
  if (L.w_dtype == FP8) return launch_fast_types<false, FP8>(a, splits, cfg, rx, stream);
  return launch_fast_types<false, BF16>(a, splits, cfg, rx, stream);
}

bool gemm_fast_supported(const GemmLaunch& L) {
  return L.splits <= 1 && !(L.flags & WE_EPI_SPLIT_K_BIT) && fast_supported(L, L.k);
}

bool gemm_pair_ok(const GemmLaunch& A, const GemmLaunch& B) {
  for (const GemmLaunch* L : {&A, &B})
    if (L->generic || L->conv_width || L->splits > 1 || L->qk_cols || L->k_wrap || (L->flags & WE_EPI_SPLIT_K_BIT) ||
        !fast_supported(*L, L->k))
      return false;
  return A.n == B.n && A.k == B.k && A.x_dtype == B.x_dtype && A.w_dtype == B.w_dtype && A.y_dtype == B.y_dtype &&
         A.flags == B.flags && A.mul == B.mul && A.cfg == B.cfg;
}

// Two GEMMs (gemm_pair_ok) as one launch: the tiles of both share the round(s) of workgroups, so a small GEMM
// beside a large one costs no launch and no partly empty round of its own. Full K per tile (no split-K), the
// tile shape picked for the two row counts together; each GEMM's tiles compute exactly as in a launch of its own
// with the same tile shape.
hipError_t gemm_fast_launch_pair(const GemmLaunch& A, const GemmLaunch& B, hipStream_t stream) {
  if (!gemm_pair_ok(A, B)) return hipErrorNotSupported;
  FastArgs a = fast_args(A, A.k);
  const FastArgs b = fast_args(B, B.k);
  a.g = FastArgs::Second{b.x,        b.w,        b.y,        b.bias,     b.gate,      b.res,
                         b.x_bytes,  b.w_bytes,  b.m,        b.x_stride, b.w_stride,  b.y_stride,
                         b.y_offset, 0u,         b.vec_store, b.store16, b.scale};
  a.grp = 1;
  const int cfg = A.cfg >= 0 ? A.cfg : pick_fast_cfg(A.m + B.m, A.n, 1, A.w_dtype == FP8);
  if (A.x_dtype == F16) {
    if (A.w_dtype == FP8) return launch_fast_types<true, FP8>(a, 1, cfg, 0, stream);
    return launch_fast_types<true, F16>(a, 1, cfg, 0, stream);
  }
  if (A.w_dtype == FP8) return launch_fast_types<false, FP8>(a, 1, cfg, 0, stream);
  return launch_fast_types<false, BF16>(a, 1, cfg, 0, stream);
}

}  // namespace we
