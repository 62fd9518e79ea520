// int4-weight GEMV / skinny GEMM on gfx950 (decode shapes):
//   y[m, n] = scale * sum_g s[n, g] * sum_{k in g} x[m, k] * q[n, k]
// W: u32 [N, K/8], eight two's-complement nibbles per word along K (low nibble = lowest k);
// s: f16 [N, K/group]. The per-group scale multiplies the f32 partial sum of that group, so the
// dequantized value q * s is never rounded to 16 bits.
//
// All three kernels are bound by the HBM stream of W (0.5 B per weight). The general and decode kernels
// share this structure (the shared-x kernel for 2 <= M <= 16 at the end differs in the work split):
//  * A workgroup of 4 waves owns 16 output columns n and one block of 16 rows m; wave w takes a quarter
//    of the 64-k blocks (a wavefront-level split-K); the four f32 partial tiles are summed through LDS.
//    At K = 3584, N = 18944 that is 1184 workgroups / 4736 waves.
//  * W reaches LDS through direct-to-LDS buffer loads that read whole 128-byte runs of 8 rows per
//    instruction (loads of the MFMA fragments straight from HBM read 32-byte pieces per row and doubled
//    the L1 -> L2 requests).
//  * MFMA 16x16x32 with x as the A operand (rows m) and W as the B operand (columns n): lane l holds
//    column n0 + l % 16 and, for each 64-k block, the two words [8b + 2g, 8b + 2g + 2) (g = l / 16),
//    read from LDS. MFMA e of the block consumes word e, so its k-slot g maps to k = 64b + 16g + 8e,
//    all inside one scale group; x is read from the same k. The 8 nibbles of a word become 8 exact
//    f16 or bf16 values in registers.
//  * The output column of a lane is fixed, so one f16 scale per lane and block multiplies the four
//    accumulator entries of that block's partial.
// The general kernel (any M, f32 / f16 / bf16 x) stages all of a wave's weights at once and reads x
// fragments from global memory two blocks ahead; the decode kernel further down (x fits in LDS) is the
// one the M = 1 decode shape runs; the shared-x kernel runs 2 <= M <= 16 with 16-bit x.
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "internal.h"

namespace we {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct Int4Args {
  const void* x;
  const uint32_t* w;
  const uint16_t* s;
  void* y;
  const float* bias;
  const float* gate;  // gated residual: y = res + gate[col] * v (res may be y; NULL: none)
  const void* res;
  uint32_t m, n, k, group;
  float scale;
  uint32_t x_stride, y_stride, x_offset, y_offset;
  uint32_t flags, y_dtype;
  uint32_t x_bytes, w_bytes, s_bytes;  // readable extents
  uint32_t gshift;                     // group = 64 << gshift (decode kernel)
};

namespace {
constexpr uint32_t kInvalid = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kCpolNt = 2;  // buffer-load cache policy: nt (non-temporal)
}  // namespace

// v_and_or_b32 with the mask in a VGPR and the constant in an SGPR (one instruction; the compiler
// otherwise splits it into an and and an or with literals)
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "s"(c));
  return r;
}

// eight nibbles (one word) -> eight f16 in k order, exact (13 VALU ops)
__device__ __forceinline__ u32x4 int4x8_to_f16(uint32_t w, uint32_t mask) {
  const uint32_t u = w ^ 0x88888888u;  // q + 8 in [0, 15] per nibble
  const f16x2 mul = {(_Float16)1.0f, (_Float16)0.0625f};
  const f16x2 add = {(_Float16)-1032.0f, (_Float16)-72.0f};
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    // byte p of u into bytes 0 and 2: lo half gets nibble 2p at bits 0-3, hi half nibble 2p+1 at bits 4-7
    const uint32_t sel = (uint32_t)p | (0x0cu << 8) | ((uint32_t)p << 16) | (0x0cu << 24);
    const uint32_t t = __builtin_amdgcn_perm(u, u, sel);
    const uint32_t v = and_or(t, mask, 0x64006400u);  // mask 0x00f0000f -> lo: 1024 + u0, hi: 1024 + 16 u1
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

template <bool IS_F16>
__device__ __forceinline__ f32x4_t mfma16(u32x4 a, u32x4 b, f32x4_t c) {
  if constexpr (IS_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// x fragments of one 64-k block for lane (m, g): k = 64b + 16g + 8e + (0..7), e = 0, 1. 16-bit x: one
// 16-B load per e. f32 x: two 16-B loads per e, split into three bf16 planes hi + mid + lo whose sum is the f32
// value exactly (8 + 8 + 8 significant bits), so every product with an int4 code keeps all 24 bits.
template <int XT>
struct XFrag {
  static constexpr int NA = XT == F32 ? 3 : 1;
  u32x4 v[2][NA];
};

template <int XT>
__device__ __forceinline__ void load_x(const __amdgpu_buffer_rsrc_t& rx, uint32_t off, XFrag<XT>& f) {
  if constexpr (XT == F32) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const u32x4 v0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, e * 32, 0));
      const u32x4 v1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, e * 32 + 16, 0));
      float fl[8] = {__uint_as_float(v0.x), __uint_as_float(v0.y), __uint_as_float(v0.z), __uint_as_float(v0.w),
                     __uint_as_float(v1.x), __uint_as_float(v1.y), __uint_as_float(v1.z), __uint_as_float(v1.w)};
      uint32_t hi[8], mid[8], lo[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        hi[i] = f32_to_bf16(fl[i]);
        const float r1 = fl[i] - bf16_to_f32((uint16_t)hi[i]);  // exact: at most 16 significant bits
        mid[i] = f32_to_bf16(r1);
        lo[i] = f32_to_bf16(r1 - bf16_to_f32((uint16_t)mid[i]));  // exact: at most 8 significant bits
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        f.v[e][0][i] = hi[2 * i] | (hi[2 * i + 1] << 16);
        f.v[e][1][i] = mid[2 * i] | (mid[2 * i + 1] << 16);
        f.v[e][2][i] = lo[2 * i] | (lo[2 * i + 1] << 16);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 2; e++)
      f.v[e][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, e * 16, 0));
  }
}

// the epilogue of one output: scale, bias, GELU, gate, then y = v, y += v or y = res + v
__device__ __forceinline__ void int4_store(const Int4Args& a, uint32_t row, uint32_t col, float sum) {
  float val = sum * a.scale;
  if (a.flags & WE_EPI_BIAS_BIT) val += a.bias[col];
  if (a.flags & WE_EPI_GELU_BIT) val = gelu_tanh(val);
  if (a.gate) val *= a.gate[col];
  const size_t o = (size_t)a.y_offset + (size_t)row * a.y_stride + col;
  const void* add = a.res ? a.res : ((a.flags & WE_EPI_ACCUMULATE_BIT) ? a.y : nullptr);
  if (a.y_dtype == F32) {
    ((float*)a.y)[o] = add ? ((const float*)add)[o] + val : val;
  } else if (a.y_dtype == BF16) {
    ((uint16_t*)a.y)[o] = f32_to_bf16(add ? bf16_to_f32(((const uint16_t*)add)[o]) + val : val);
  } else {
    ((uint16_t*)a.y)[o] = f32_to_f16(add ? f16_to_f32(((const uint16_t*)add)[o]) + val : val);
  }
}

constexpr int INT4_CH = 14;  // 64-k blocks whose weights a wave stages at once (7 KB of LDS per wave)
constexpr int INT4_XPF = 2;  // blocks of x fragments in flight ahead of the MFMAs

template <int XT>
__global__ void __launch_bounds__(256) int4_gemv_kernel(Int4Args a) {
  constexpr bool IS_F16 = XT == F16;
  constexpr int NA = XFrag<XT>::NA;
  constexpr int XB = XT == F32 ? 4 : 2;
  constexpr int WAVE_LDS = 16 * INT4_CH * 32;  // 16 rows x CH blocks x 32 B
  static_assert(WAVE_LDS % 1024 == 0 && 4 * WAVE_LDS >= 4 * 64 * 16, "LDS staging layout");
  __shared__ __attribute__((aligned(1024))) char lds[4 * WAVE_LDS];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const uint32_t n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const uint32_t m = m0 + l16;
  const uint32_t nblk = a.k / 64;
  const uint32_t per = (nblk + 3) / 4;
  const uint32_t b0 = min(nblk, wave * per), b1 = min(nblk, b0 + per);
  const uint32_t gpb = a.group / 64;  // blocks per scale group
  const uint32_t row_bytes = a.k / 2;
  char* wl = lds + wave * WAVE_LDS;  // this wave's staging area (no other wave touches it)

  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)a.w_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.s, (short)0, (int)a.s_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kRsrcWord3);
  const uint32_t s_off = n0 + l16 < a.n ? (n0 + l16) * (a.k / a.group) * 2 : kInvalid;        // + 2 per group
  const uint32_t x_off = m < a.m ? (a.x_offset + m * a.x_stride + g * 16) * XB : kInvalid;  // + 64 XB per block

  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t c = b0; c < b1; c += INT4_CH) {
    const int nb = (int)min((uint32_t)INT4_CH, b1 - c);  // wave-uniform
    // Stage W[n0 .. n0 + 16, blocks c .. c + nb) into LDS row-major (row r at r * nb * 32): 16-byte piece
    // p of the area is loaded by lane p % 64 of load p / 64, so every load reads whole runs of each row.
    const int pieces_row = 2 * nb;
#pragma unroll
    for (int j = 0; j < INT4_CH / 2; j++) {
      if (2 * j < nb) {
        const int p = j * 64 + lane;
        const int r = p / pieces_row, q = p - r * pieces_row;
        const uint32_t row = n0 + r;
        const uint32_t o = (r < 16 && row < a.n) ? row * row_bytes + c * 32 + q * 16 : kInvalid;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t*)(wl + j * 1024), 16, o, 0, 0, 0);
      }
    }
    uint16_t sc[INT4_CH];
#pragma unroll
    for (int i = 0; i < INT4_CH; i++)
      if (i < nb) sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, s_off + ((c + i) / gpb) * 2, 0, 0);
    XFrag<XT> xf[INT4_XPF + 1];
#pragma unroll
    for (int i = 0; i < INT4_XPF; i++)
      if (i < nb) load_x<XT>(rx, x_off + (c + i) * 64 * XB, xf[i]);
    // the staged weights (and the first scales / x fragments) must have landed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < INT4_CH; i++) {
      if (i < nb) {
        if (i + INT4_XPF < nb) load_x<XT>(rx, x_off + (c + i + INT4_XPF) * 64 * XB, xf[(i + INT4_XPF) % (INT4_XPF + 1)]);
        const XFrag<XT>& cur = xf[i % (INT4_XPF + 1)];
        // lane (n, g): words [2g, 2g + 2) of block i of row n, i.e. k = 64 (c + i) + 16 g + 8 e
        const u32x2 wq = *(const u32x2*)(wl + l16 * (nb * 32) + i * 32 + g * 8);
        f32x4_t part = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const u32x4 wf = IS_F16 ? int4x8_to_f16(wq[e], 0x00f0000fu) : int4x8_to_bf16(wq[e]);
#pragma unroll
          for (int p = 0; p < NA; p++) part = mfma16<IS_F16>(cur.v[e][p], wf, part);
        }
        acc += part * f16_to_f32(sc[i]);
      }
    }
    // every lane has read its fragments before the next chunk's loads overwrite the area
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // lane l holds column n0 + l % 16 and rows m0 + 4 (l / 16) + (0..3); the staging areas are reused
  f32x4_t* red = (f32x4_t*)lds;  // [4 waves][64 lanes]
  __syncthreads();
  red[wave * 64 + lane] = acc;
  __syncthreads();
  const int ln = threadIdx.x & 63, r = threadIdx.x >> 6;
  const float sum = red[ln][r] + red[64 + ln][r] + red[128 + ln][r] + red[192 + ln][r];
  const uint32_t row = m0 + 4 * (ln >> 4) + r, col = n0 + (ln & 15);
  if (row < a.m && col < a.n) int4_store(a, row, col, sum);
}

// ------------------------------------------------------------------------------------------------------
// Decode kernel (M * K * 2 bytes of x fit in LDS, 16-bit x): the same work split and MFMA layout as
// above, with the weight stream software-pipelined. Each wave walks its blocks in chunks of 4 (2 KB of W)
// through a 2-slot LDS ring: both slots are requested up front and chunk i + 2 as soon as chunk i has been
// unpacked and multiplied. Two slots (not more) keep the workgroup at 25.5 KB of LDS, so 6 workgroups fit
// per CU and all 1184 workgroups of the decode shape are resident at once; measured on MI355X that beats
// deeper rings with fewer resident workgroups. Each chunk issues exactly 2 direct-to-LDS loads
// (out-of-range ones read zeros) and nothing else, so the vmcnt waits are constants.
// The workgroup's scale tile (16 rows x K / group halves, contiguous) is staged in LDS once.
// x is staged once per workgroup in LDS with each 8-value chunk stored in the order
// (x0, x4, x1, x5, x2, x6, x3, x7): that is the order in which a word's nibbles come out of the cheap
// unpack below (no byte permute per pair), so both MFMA operands agree on the k of every slot.
// Lanes whose row m >= M read row 0 of x: rows of the 16x16 tile past M are never stored.

constexpr int PIPE_CB = 4;                     // 64-k blocks per chunk
constexpr int PIPE_NBUF = 2;                   // chunk slots per wave (6 workgroups per CU fit)
constexpr int PIPE_CHUNK = 16 * PIPE_CB * 32;  // 2 KB: 16 rows x 4 blocks x 32 B
constexpr int PIPE_XMAX = 7680;                // bytes of staged x (25.5 KB of LDS per workgroup in all)
constexpr int PIPE_LOADS = 2;                  // loads per chunk (direct-to-LDS)
constexpr int PIPE_MAXB = 16;                  // 64-k blocks per wave at most (K <= 4096)
constexpr int PIPE_XPT = (PIPE_XMAX / 16 + 255) / 256;  // 16-byte x chunks staged per thread
constexpr int PIPE_SMAX = 16 * PIPE_MAXB * 4 * 2;       // scale tile: 16 rows x (K / 64) groups x 2 B

// eight nibbles -> eight exact f16, slots ordered (k0, k4), (k1, k5), (k2, k6), (k3, k7): 10 VALU ops
__device__ __forceinline__ u32x4 int4x8_to_f16_il(uint32_t w, uint32_t m_lo, uint32_t m_hi) {
  const uint32_t u = w ^ 0x88888888u;  // q + 8 per nibble
  const uint32_t u8 = u >> 8;
  const f16x2 sub = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const f16x2 mul = {(_Float16)0.0625f, (_Float16)0.0625f};
  const f16x2 add = {(_Float16)-72.0f, (_Float16)-72.0f};
  const uint32_t t0 = and_or(u, m_lo, 0x64006400u);   // 1024 + u0, 1024 + u4
  const uint32_t t1 = and_or(u, m_hi, 0x64006400u);   // 1024 + 16 u1, 1024 + 16 u5
  const uint32_t t2 = and_or(u8, m_lo, 0x64006400u);  // 1024 + u2, 1024 + u6
  const uint32_t t3 = and_or(u8, m_hi, 0x64006400u);  // 1024 + 16 u3, 1024 + 16 u7
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, t0) + sub);
  r[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, t1), mul, add));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, t2) + sub);
  r[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, t3), mul, add));
  return r;
}

// (x0..x7) -> (x0, x4, x1, x5, x2, x6, x3, x7)
__device__ __forceinline__ u32x4 interleave8(u32x4 v) {
  return u32x4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
               __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}


// dma16 with the non-temporal cache policy, for weights read once per call (the shared-x kernel's weight pieces:
// M = 8 12.85-13.44 -> 12.47-12.77 us, M = 16 13.69-13.96 -> 13.42-13.54 us, alternating processes, same box; x and
// the scales, which every workgroup reads, keep the default policy)
__device__ __forceinline__ void dma16_nt(const __amdgpu_buffer_rsrc_t& r, void* dst, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"((uint32_t)(uintptr_t)(lds_ptr_t*)dst), "v"(voff), "s"(r)
               : "memory");
}

template <int XT>
__global__ void __launch_bounds__(256) int4_gemv_pipe_kernel(Int4Args a) {
  constexpr bool IS_F16 = XT == F16;
  __shared__ __attribute__((aligned(1024))) char wst[4 * PIPE_NBUF * PIPE_CHUNK];
  __shared__ __attribute__((aligned(16))) char xs[PIPE_XMAX];
  __shared__ __attribute__((aligned(16))) char ss[PIPE_SMAX];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const uint32_t n0 = blockIdx.x * 16;
  const uint32_t nblk = a.k / 64;
  const uint32_t per = (nblk + 3) / 4;
  const uint32_t b0 = min(nblk, wave * per), b1 = min(nblk, b0 + per);
  const int nch = (int)((b1 - b0 + PIPE_CB - 1) / PIPE_CB);
  const uint32_t gshift = a.gshift;  // group = 64 << gshift
  const uint32_t row_bytes = a.k / 2;
  char* ws = wst + wave * (PIPE_NBUF * PIPE_CHUNK);

  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)a.w_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.s, (short)0, (int)a.s_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kRsrcWord3);

  // chunk image in LDS: row r (of 16) at r * 128, 16-byte piece q at position q ^ (r & 7); piece q of a
  // row holds block q / 2, words 4 (q % 2) .. + 4. Lane l of load j fills position (64 j + l) % 8 of row
  // (64 j + l) / 8.
  uint32_t dma_off[2];
  int dma_blk[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int p = j * 64 + lane, r = p >> 3, q = (p & 7) ^ (r & 7);
    const uint32_t row = n0 + r;
    dma_off[j] = row < a.n ? row * row_bytes + q * 16 : kInvalid;
    dma_blk[j] = q >> 1;
  }
  auto issue = [&](int ci, auto SLOT) {
    constexpr int s = decltype(SLOT)::value;
    const uint32_t c = b0 + (uint32_t)ci * PIPE_CB;
    char* slot = ws + s * PIPE_CHUNK;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t o = c + dma_blk[j] < b1 ? dma_off[j] + c * 32 : kInvalid;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t*)(slot + j * 1024), 16, o, 0, 0, 0);
    }
  };

  // x rows m < M -> LDS, interleaved per 8-value chunk; the first two weight chunks load meanwhile
  const uint32_t xchunks = a.m * (a.k / 8), cpr = a.k / 8;
  u32x4 xv[PIPE_XPT];
#pragma unroll
  for (int j = 0; j < PIPE_XPT; j++) {
    const uint32_t idx = tid + 256 * j;
    const uint32_t m = idx / cpr, t = idx - m * cpr;
    const uint32_t o = idx < xchunks ? (a.x_offset + m * a.x_stride + t * 8) * 2 : kInvalid;
    xv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
  }
  // the workgroup's scale tile s[n0 .. n0 + 16, :] is contiguous (16 G halves): 16-byte loads by the
  // first threads, staged in LDS with x; loaded before the weights, so waiting for them never waits
  // for the weight stream, and only direct-to-LDS loads are in flight in the main loop
  const uint32_t ng = a.k / a.group;
  const uint32_t s_pieces = ng * 2;  // 16 rows x ng halves = 2 ng pieces of 16 bytes
  // a 16-byte load that straddles the end of the buffer reads nothing, so the last column tile (rows past
  // N) loads its scales as halves
  const bool s_whole = n0 + 16 <= a.n;
  constexpr int SH = PIPE_SMAX / 2 / 256;  // halves per thread on the tail path
  u32x4 sv = {0u, 0u, 0u, 0u};
  uint16_t sh[SH] = {};
  if (s_whole) {
    sv = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)tid < s_pieces ? n0 * ng * 2 + tid * 16 : kInvalid, 0, 0));
  } else {
#pragma unroll
    for (int j = 0; j < SH; j++) {
      const uint32_t i = tid + 256 * j;
      sh[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, i < 16 * ng ? (n0 * ng + i) * 2 : kInvalid, 0, 0);
    }
  }
  static_for<0, PIPE_NBUF>([&](auto CI) {
    if (decltype(CI)::value < nch) issue(decltype(CI)::value, CI);
  });
#pragma unroll
  for (int j = 0; j < PIPE_XPT; j++) {
    const uint32_t idx = tid + 256 * j;
    if (idx < xchunks) *(u32x4*)(xs + idx * 16) = IS_F16 ? interleave8(xv[j]) : xv[j];
  }
  if (s_whole) {
    if ((uint32_t)tid < s_pieces) *(u32x4*)(ss + tid * 16) = sv;
  } else {
#pragma unroll
    for (int j = 0; j < SH; j++) {
      const uint32_t i = tid + 256 * j;
      if (i < 16 * ng) *(uint16_t*)(ss + i * 2) = sh[j];
    }
  }
  // x and scales visible to every wave; unlike __syncthreads this does not wait for the weight loads
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const uint32_t m_lo = 0x000f000fu, m_hi = 0x00f000f0u;
  const uint32_t xrow = (l16 < (int)a.m ? (uint32_t)l16 : 0u) * a.k * 2;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto step = [&](auto CI) {
    constexpr int ci = decltype(CI)::value, s = ci % PIPE_NBUF;
    // chunks ci + 1 .. min(ci + NBUF - 1, nch - 1) may still be in flight
    static_assert(PIPE_NBUF >= 2 && PIPE_NBUF <= 4, "wait ladder below");
    if (PIPE_NBUF >= 4 && ci + 3 < nch) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * PIPE_LOADS) : "memory");
    else if (PIPE_NBUF >= 3 && ci + 2 < nch) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PIPE_LOADS) : "memory");
    else if (ci + 1 < nch) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PIPE_LOADS) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint32_t c = b0 + (uint32_t)ci * PIPE_CB;
    const char* slot = ws + s * PIPE_CHUNK;
#pragma unroll
    for (int i = 0; i < PIPE_CB; i++) {
      if (c + i < b1) {
        // lane (n, g): words [2g, 2g + 2) of block i of row n = piece 2i + g / 2, half g % 2
        const u32x2 wq = *(const u32x2*)(slot + l16 * 128 + (((2 * i + (g >> 1)) ^ (l16 & 7)) * 16) + (g & 1) * 8);
        const uint32_t xo = xrow + ((c + i) * 8 + 2 * g) * 16;  // chunk t = 8 b + 2 g + e
        f32x4_t part = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const u32x4 xa = *(const u32x4*)(xs + xo + e * 16);
          const u32x4 wf = IS_F16 ? int4x8_to_f16_il(wq[e], m_lo, m_hi) : int4x8_to_bf16(wq[e]);
          part = mfma16<IS_F16>(xa, wf, part);
        }
        acc += part * f16_to_f32(*(const uint16_t*)(ss + (l16 * ng + ((c + i) >> gshift)) * 2));
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot s is free: load chunk ci + NBUF into it
    if (ci + PIPE_NBUF < nch) issue(ci + PIPE_NBUF, std::integral_constant<int, s>{});
  };
  static_for<0, PIPE_MAXB / PIPE_CB>([&](auto CI) {
    if (decltype(CI)::value < nch) step(CI);
  });

  // lane l holds column n0 + l % 16 and rows 4 (l / 16) + (0..3); sum the four waves' K-quarters
  f32x4_t* red = (f32x4_t*)wst;
  __syncthreads();
  red[wave * 64 + lane] = acc;
  __syncthreads();
  const int ln = tid & 63, r = tid >> 6;
  const float sum = red[ln][r] + red[64 + ln][r] + red[128 + ln][r] + red[192 + ln][r];
  const uint32_t row = 4 * (ln >> 4) + r, col = n0 + (ln & 15);
  if (row < a.m && col < a.n) int4_store(a, row, col, sum);
}

// ------------------------------------------------------------------------------------------------------
// Shared-x kernel (2 <= M <= 16, 16-bit x, K / group <= 64): a workgroup of TILES x WPT waves owns 16 TILES
// columns over ALL of K. The waves walk K in lock step through an NBUF-slot LDS ring; a slot holds one chunk
// of 4 blocks (256 k): XR x rows (XR x 512 B, rows >= M read as zeros; XR = 8 when M <= 8) and the TILES column
// tiles' 16 x 4 weight blocks (2 KB images of the decode kernel's layout). x thus crosses L2 -> LDS once per
// 16 TILES columns.
// Wave w multiplies column tile w % TILES with the blocks i = w / TILES (mod WPT) of every chunk; the WPT
// partial tiles of a column tile are summed through LDS at the end, in the same order for every TILES.
// Several waves per tile keep several waves on each SIMD: with one wave per SIMD the dependent LDS read ->
// unpack -> MFMA chain of every block was exposed.
// Per chunk every lane issues LPC 16-byte direct-to-LDS loads (out-of-range ones read zeros); where the slot
// has fewer pieces than LPC x threads, the spare loads of whole waves read nothing into a pad, so the waits
// stay constants. No load in the loop targets a register (the compiler would add its own, stricter waits for
// those). The scale tile (16 TILES rows x K / group halves) is staged once.
// Step ci: wait for chunk ci (own loads), barrier (everyone's loads landed, everyone is done with the slot
// of chunk ci - 1), issue chunk ci + NBUF - 1 into that slot, then unpack and multiply chunk ci.
// x rows in a slot: row m at m * 512, 16-byte piece p at position p ^ (m & 15) (conflict-free b128 reads).
// Workgroup size: at N = 18944, 64 columns make 296 workgroups, so 40 CUs run two while the others run one
// and set the time (M = 8: 14.0 us, against 10.4 us for the 256 workgroups of N = 16384). For M <= 8, 32
// columns and 8 x rows make 592 smaller workgroups (28 KB of LDS, 8 waves), two or three on every CU: 12.5 us.
constexpr int SK_WB = 16 * PIPE_CB * 32;  // one column tile's weights per chunk: 2 KB
constexpr int SK_NBUF = 3;                // ring slots (4 measured no faster for either shape)

// WPT: waves per column tile (each takes PIPE_CB / WPT blocks of every chunk)
template <int XT, int TILES, int XR, int WPT>
__global__ void __launch_bounds__(64 * TILES * WPT) int4_gemv_shared_kernel(Int4Args a) {
  constexpr bool IS_F16 = XT == F16;
  constexpr int NW = TILES * WPT, NT = 64 * NW;  // waves, threads
  constexpr int XB = XR * 512;                    // x rows of one chunk
  constexpr int SLOT = XB + TILES * SK_WB;
  constexpr int XP = XB / 16, PIECES = SLOT / 16;  // 16-byte pieces: x, then weights
  constexpr int LPC = (PIECES + NT - 1) / NT;      // loads per lane per chunk
  constexpr bool PAD = LPC * NT > PIECES;          // spare loads (whole waves) land in a pad
  constexpr int BPW = PIPE_CB / WPT;               // blocks per wave per chunk
  constexpr int SROWS = 16 * TILES, SMAX = SROWS * 64 * 2;  // scale tile: rows x at most 64 groups
  static_assert(XP % 64 == 0 && PIECES % 64 == 0, "x / weight loads are whole waves");
  __shared__ __attribute__((aligned(1024))) char ring[SK_NBUF * SLOT + (PAD ? 1024 : 0)];
  __shared__ __attribute__((aligned(16))) char ss[SMAX];
  static_assert(SK_NBUF * SLOT >= NW * 64 * 16, "reduction area");

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int tile = wave % TILES, phase = wave / TILES;
  const uint32_t n0 = blockIdx.x * SROWS, nw = n0 + 16 * tile;
  const uint32_t nblk = a.k / 64;
  const int nch = (int)((nblk + PIPE_CB - 1) / PIPE_CB);
  const uint32_t gshift = a.gshift;
  const uint32_t row_bytes = a.k / 2;

  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)a.w_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.s, (short)0, (int)a.s_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kRsrcWord3);

  // piece P = j NT + tid of a slot: P < XP are x rows (row P / 32, position P % 32), then the TILES weight
  // images (tile (P - XP) / 128, rows nw .. nw + 16), then spares; which kind a load is, is wave-uniform
  uint32_t src[LPC];
  int blk[LPC];
#pragma unroll
  for (int j = 0; j < LPC; j++) {
    const int P = j * NT + tid;
    if (P < XP) {
      const int m = P >> 5, p = (P & 31) ^ (m & 15);
      src[j] = (uint32_t)m < a.m ? (a.x_offset + m * a.x_stride) * 2 + p * 16 : kInvalid;
      blk[j] = p >> 3;
    } else if (P < PIECES) {
      const int T = (P - XP) >> 7, p = (P - XP) & 127, r = p >> 3, q = (p & 7) ^ (r & 7);
      const uint32_t row = n0 + 16 * T + r;
      src[j] = row < a.n ? row * row_bytes + q * 16 : kInvalid;
      blk[j] = q >> 1;
    } else {
      src[j] = kInvalid;
      blk[j] = 0;
    }
  }

  auto issue = [&](int ci, auto S) {  // chunk ci (possibly past the end) into slot S
    constexpr int s = decltype(S)::value;
    const uint32_t c = (uint32_t)ci * PIPE_CB;
    char* slot = ring + s * SLOT;
#pragma unroll
    for (int j = 0; j < LPC; j++) {
      const int first = j * NT + wave * 64;
      if (first < XP) dma16(rx, slot + first * 16, c + blk[j] < nblk ? src[j] + c * 128 : kInvalid);
      else if (first < PIECES) dma16_nt(rw, slot + first * 16, c + blk[j] < nblk ? src[j] + c * 32 : kInvalid);
      else dma16(rw, ring + SK_NBUF * SLOT, kInvalid);  // a spare: zeros into the pad, counted like the others
    }
  };

  // scale tile s[n0 .. n0 + SROWS, :] (contiguous): 16-byte pieces straight to LDS, or halves through
  // registers on the last column tile (a 16-byte load that straddles the end of the buffer reads nothing)
  const uint32_t ng = a.k / a.group;
  const bool s_whole = n0 + SROWS <= a.n;
  constexpr int SH = SMAX / 2 / NT;
  uint16_t sh[SH];
  if (s_whole) {
    if (wave < SMAX / 1024)
      dma16(rs, ss + wave * 1024, (uint32_t)tid < (uint32_t)(SROWS / 8) * ng ? n0 * ng * 2 + tid * 16 : kInvalid);
  } else {
#pragma unroll
    for (int j = 0; j < SH; j++) {
      const uint32_t i = tid + NT * j;
      sh[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, i < SROWS * ng ? (n0 * ng + i) * 2 : kInvalid, 0, 0);
    }
  }
  static_for<0, SK_NBUF - 1>([&](auto CI) { issue(decltype(CI)::value, CI); });
  if (!s_whole) {
#pragma unroll
    for (int j = 0; j < SH; j++) {
      const uint32_t i = tid + NT * j;
      if (i < SROWS * ng) *(uint16_t*)(ss + i * 2) = sh[j];
    }
  }
  const char* srow = ss + (16 * tile + l16) * ng * 2;  // visible after the first step's barrier

  const uint32_t x_rd = l16 * 512, x_sw = l16;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto step = [&](int ci, auto S) {
    constexpr int s = decltype(S)::value;
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((SK_NBUF - 2) * LPC) : "memory");
    issue(ci + SK_NBUF - 1, std::integral_constant<int, (s + SK_NBUF - 1) % SK_NBUF>{});
    const uint32_t c = (uint32_t)ci * PIPE_CB;
    const char* slot = ring + s * SLOT;
    const char* wsl = slot + XB + tile * SK_WB;
#pragma unroll
    for (int ii = 0; ii < BPW; ii++) {
      const int i = WPT * ii + phase;
      if (c + i < nblk) {
        const u32x2 wq2 = *(const u32x2*)(wsl + l16 * 128 + (((2 * i + (g >> 1)) ^ (l16 & 7)) * 16) + (g & 1) * 8);
        f32x4_t part = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 2; e++) {
          // with 8 staged rows, lanes of rows 8-15 feed zeros (those rows are past M)
          u32x4 xa = *(const u32x4*)(slot + x_rd + (((8 * i + 2 * g + e) ^ x_sw) * 16));
          if constexpr (XR < 16) xa = l16 < XR ? xa : u32x4{0, 0, 0, 0};
          const u32x4 wf = IS_F16 ? int4x8_to_f16(wq2[e], 0x00f0000fu) : int4x8_to_bf16(wq2[e]);
          part = mfma16<IS_F16>(xa, wf, part);
        }
        acc += part * f16_to_f32(*(const uint16_t*)(srow + ((c + i) >> gshift) * 2));
      }
    }
  };
  for (int ci = 0; ci < nch; ci += SK_NBUF) {
    static_for<0, SK_NBUF>([&](auto S) {
      if (ci + decltype(S)::value < nch) step(ci + decltype(S)::value, S);
    });
  }
  // the ring's last loads (chunks past the end, zeros) land before the ring is reused for the sums
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // lane l of wave (tile, phase) holds column nw + l % 16, rows 4 (l / 16) + (0..3), summed over the
  // blocks of its phase; it stores rows 4 (l / 16) + (4 / WPT) phase + .. of the sum over all phases
  f32x4_t* red = (f32x4_t*)ring;  // [NW waves][64 lanes]
  red[wave * 64 + lane] = acc;
  __syncthreads();
  const uint32_t col = nw + l16;
#pragma unroll
  for (int rr = 0; rr < 4 / WPT; rr++) {
    const int r = (4 / WPT) * phase + rr;
    const uint32_t row = 4 * g + r;
    float sum = 0.0f;
#pragma unroll
    for (int p = 0; p < WPT; p++) sum += red[(tile + TILES * p) * 64 + lane][r];
    if (row < a.m && col < a.n) int4_store(a, row, col, sum);
  }
}

// ------------------------------------------------------------------------------------------------------
// Decode kernel for M = 1 with f16 x (the decode shape). Every weight byte a wave needs is requested at its
// start, straight into registers (K / 32 16-byte pieces per row, 16 lanes per row, up to 8 pieces per lane),
// so the whole matrix is in flight at once, as in a streaming read: no LDS ring whose refills wait on the
// arithmetic. x (interleaved per 8 values like the pipe kernel's) and the workgroup's scale tile go through
// LDS; they are requested before the weights, so waiting for them never waits for the weight stream.
//  * A workgroup of 4 waves owns 16 rows n (4 per wave, 16 lanes each): N / 16 workgroups, about 4.6 per CU at
//    N = 18944, all resident at once (about 90 VGPRs and 10 KB of LDS each).
//  * Lane (row, l) holds pieces P = l + 16 j: k = 32 P .. 32 P + 31, inside one scale group (group >= 64).
//    Each word of a piece is 8 nibbles, unpacked exactly to f16 pairs ordered (k0, k4), (k1, k5), ... and
//    multiplied with x by v_dot2_f32_f16 (products exact, f32 sums); the piece's f32 sum times its group's
//    f16 scale adds to the lane's total.
//  * The 16 lanes of a row are summed by a butterfly of cross-lane adds (fixed order), then one lane
//    runs the epilogue.
// a.x * b.x + a.y * b.y + c for two packed f16 pairs (v_dot2_f32_f16). The words come in by value: a
// __builtin_bit_cast of a vector component expression (v.y) reads component 0 with this compiler.
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

constexpr int DIRECT_NP = 8;                                     // pieces per lane at most: K <= 4096
constexpr int DIRECT_XMAX = DIRECT_NP * 16 * 32 * 2;             // staged x: K f16 values
constexpr int DIRECT_SMAX = 16 * (DIRECT_NP * 16 * 32 / 64) * 2;  // scale tile: 16 rows x K / 64 groups

template <int NP>  // pieces per lane: ceil(K / 512)
__global__ void __launch_bounds__(256) int4_gemv_direct_kernel(Int4Args a) {
  __shared__ __attribute__((aligned(16))) char xs[DIRECT_XMAX];
  __shared__ __attribute__((aligned(16))) char ss[DIRECT_SMAX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, rl = wave * 4 + (lane >> 4);  // the lane's row among the workgroup's 16
  const uint32_t n0 = blockIdx.x * 16, row = n0 + rl;
  const uint32_t npc = a.k / 32;  // 16-byte pieces per row, at most 16 NP
  const uint32_t gshift = a.gshift, ng = a.k / a.group;

  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)a.w_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.s, (short)0, (int)a.s_bytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kRsrcWord3);

  // x: K / 8 chunks of 16 bytes, at most two per thread
  const uint32_t xchunks = a.k / 8;
  u32x4 xv[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const uint32_t idx = tid + 256 * j;
    xv[j] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, idx < xchunks ? (a.x_offset + idx * 8) * 2 : kInvalid, 0, 0));
  }
  // the scale tile s[n0 .. n0 + 16, :] is contiguous: 16-byte pieces, or halves for the last column tile
  const uint32_t s_pieces = ng * 2;
  const bool s_whole = n0 + 16 <= a.n;
  constexpr int SH = DIRECT_SMAX / 2 / 256;
  u32x4 sv = {0u, 0u, 0u, 0u};
  uint16_t sh[SH] = {};
  if (s_whole) {
    sv = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)tid < s_pieces ? n0 * ng * 2 + tid * 16 : kInvalid, 0, 0));
  } else {
#pragma unroll
    for (int j = 0; j < SH; j++) {
      const uint32_t i = tid + 256 * j;
      sh[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, i < 16 * ng ? (n0 * ng + i) * 2 : kInvalid, 0, 0);
    }
  }
  // the weights: all of the lane's pieces at once (pieces past the row read as zeros and are skipped below).
  // Non-temporal (cache policy nt): every weight byte is read once per call (M = 1 decode shape: 9.54-10.0 ->
  // 9.20-9.30 us, alternating processes, same box)
  u32x4 wv[NP];
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const uint32_t pc = (uint32_t)(l16 + 16 * j);
    const uint32_t o = row < a.n && pc < npc ? row * (a.k / 2) + pc * 16 : kInvalid;
    wv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, kCpolNt));
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const uint32_t idx = tid + 256 * j;
    if (idx < xchunks) *(u32x4*)(xs + idx * 16) = interleave8(xv[j]);
  }
  if (s_whole) {
    if ((uint32_t)tid < s_pieces) *(u32x4*)(ss + tid * 16) = sv;
  } else {
#pragma unroll
    for (int j = 0; j < SH; j++) {
      const uint32_t i = tid + 256 * j;
      if (i < 16 * ng) *(uint16_t*)(ss + i * 2) = sh[j];
    }
  }
  // x and scales visible to every wave; unlike __syncthreads this does not wait for the weight loads
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const uint32_t m_lo = 0x000f000fu, m_hi = 0x00f000f0u;
  const uint16_t* srow = (const uint16_t*)ss + rl * ng;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    {  // pieces past the row's end (K % 512 != 0) are dropped by a select
      const uint32_t pc = (uint32_t)(l16 + 16 * j);
      const char* xp = xs + pc * 64;  // the piece's 4 chunks of 8 x values (inside xs for every pc)
      float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const u32x4 q = int4x8_to_f16_il(wv[j][e], m_lo, m_hi);
        const u32x4 xx = *(const u32x4*)(xp + e * 16);
        c0 = dot2_f16(xx.x, q.x, c0);
        c1 = dot2_f16(xx.y, q.y, c1);
        c0 = dot2_f16(xx.z, q.z, c0);
        c1 = dot2_f16(xx.w, q.w, c1);
      }
      const float part = __builtin_fmaf(c0 + c1, f16_to_f32(srow[(pc >> (1 + gshift)) & 63u]), acc);
      acc = pc < npc ? part : acc;
    }
  }
  // the row's 16 lanes: butterfly over lane bits 3, 2, 1, 0 (every lane ends with the same sum)
#pragma unroll
  for (int d = 8; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, 16);
  if (l16 == 0 && row < a.n) int4_store(a, 0, row, acc);
}

hipError_t int4_launch(const Int4Launch& L, hipStream_t stream) {
  const int xb = L.x_dtype == F32 ? 4 : 2;
  const uint64_t x_need = L.k ? ((uint64_t)L.x_offset + (uint64_t)(L.m - 1) * L.x_stride + L.k) * xb : 0;
  const uint64_t w_need = (uint64_t)L.n * L.k / 2, s_need = (uint64_t)L.n * (L.k / L.group) * 2;
  if (x_need >= kInvalid || w_need >= kInvalid || s_need >= kInvalid) return hipErrorNotSupported;
  Int4Args a{};
  a.x = L.x;
  a.w = L.w;
  a.s = L.scales;
  a.y = L.y;
  a.bias = L.bias;
  a.gate = L.gate;
  a.res = L.res;
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
  a.x_bytes = (uint32_t)x_need;
  a.w_bytes = (uint32_t)w_need;
  a.s_bytes = (uint32_t)s_need;
  dim3 grid((L.n + 15) / 16, (L.m + 15) / 16);
  uint32_t gshift = 0;
  while ((64u << gshift) < L.group) gshift++;
  a.gshift = gshift;
  // L.path (Tuning::int4_path) 1 / 2 / 3 forces the general / shared-x / LDS-ring kernel (tests, measurements)
  const int path = L.path;
  const bool generic = path == 1;
  const bool ring = L.x_dtype != F32 && L.m <= 16 && (64u << gshift) == L.group && !generic;
  const bool pipe = ring && !path && (uint64_t)L.m * L.k * 2 <= (uint64_t)PIPE_XMAX && L.k / 64 <= 4 * (uint32_t)PIPE_MAXB;
  // M = 1, f16 x, K <= 4096: every weight in flight at once (WE_INT4_PATH=pipe selects the ring kernel)
  const bool direct = L.m == 1 && L.x_dtype == F16 && (64u << gshift) == L.group && L.k % 64 == 0 &&
                      L.k <= (uint32_t)(DIRECT_NP * 16 * 32) && !path;
  if (direct) {
    const dim3 gd((L.n + 15) / 16), bd(256);
    switch ((L.k / 32 + 15) / 16) {
      case 1: hipLaunchKernelGGL(int4_gemv_direct_kernel<1>, gd, bd, 0, stream, a); break;
      case 2: hipLaunchKernelGGL(int4_gemv_direct_kernel<2>, gd, bd, 0, stream, a); break;
      case 3: hipLaunchKernelGGL(int4_gemv_direct_kernel<3>, gd, bd, 0, stream, a); break;
      case 4: hipLaunchKernelGGL(int4_gemv_direct_kernel<4>, gd, bd, 0, stream, a); break;
      case 5: hipLaunchKernelGGL(int4_gemv_direct_kernel<5>, gd, bd, 0, stream, a); break;
      case 6: hipLaunchKernelGGL(int4_gemv_direct_kernel<6>, gd, bd, 0, stream, a); break;
      case 7: hipLaunchKernelGGL(int4_gemv_direct_kernel<7>, gd, bd, 0, stream, a); break;
      default: hipLaunchKernelGGL(int4_gemv_direct_kernel<8>, gd, bd, 0, stream, a); break;
    }
    return hipGetLastError();
  }
  const bool force_pipe = path == 3;
  if (ring && !pipe && !force_pipe && L.k / L.group <= 64) {
    // M <= 8: 32 columns and 8 staged x rows per workgroup; larger M: 64 columns, 16 rows (32 columns there
    // double the x traffic and leave a third of each chunk's loads spare: slower)
    const bool x8 = L.m <= 8;
    const bool f16 = L.x_dtype == F16;
    void (*kern)(Int4Args);
    // (measured: 80-column workgroups of 5 tiles x 2 waves, one round of 237 on 256 CUs, gave M = 16 no faster and
    // M = 8 14.7 against 13.0 us: fewer waves in flight per CU cost more than the second round saves)
    const int tiles = x8 ? 2 : 4, wpt = 4;
    if (x8) kern = f16 ? int4_gemv_shared_kernel<F16, 2, 8, 4> : int4_gemv_shared_kernel<BF16, 2, 8, 4>;
    else kern = f16 ? int4_gemv_shared_kernel<F16, 4, 16, 4> : int4_gemv_shared_kernel<BF16, 4, 16, 4>;
    const dim3 gs((L.n + 16 * tiles - 1) / (16 * tiles)), bs(64 * tiles * wpt);
    hipLaunchKernelGGL(kern, gs, bs, 0, stream, a);
    return hipGetLastError();
  }
  if (pipe || (force_pipe && ring && (uint64_t)L.m * L.k * 2 <= (uint64_t)PIPE_XMAX && L.k / 64 <= 4 * (uint32_t)PIPE_MAXB)) {
    if (L.x_dtype == F16) hipLaunchKernelGGL(int4_gemv_pipe_kernel<F16>, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(int4_gemv_pipe_kernel<BF16>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  switch (L.x_dtype) {
    case F16: hipLaunchKernelGGL(int4_gemv_kernel<F16>, grid, dim3(256), 0, stream, a); break;
    case BF16: hipLaunchKernelGGL(int4_gemv_kernel<BF16>, grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(int4_gemv_kernel<F32>, grid, dim3(256), 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace we
