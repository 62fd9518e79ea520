// Scaled dot-product attention for gfx950, one pass over the keys with an online softmax.
//
// Semantics of src/kernels/attention.ts:20-51: q [tokens, heads, dim], k and v [tokens, kvHeads, dim];
// query head h reads kv head h / (heads / kvHeads); out [tokens, heads, dim] = softmax(q k^T / sqrt(dim)) v,
// over all keys or (causal) keys j <= i. Each token's heads may start `stride` elements after the previous
// token's, so q, k and v can be column slices of one fused QKV projection output.
//
// Work split: a wave owns 32 queries of one head and walks the keys in tiles of 64 shared through LDS with
// the other waves of its workgroup. Four kernels:
//   * attn16_kernel / attn32_kernel: any head dim up to 128; 4 waves (128 queries), tiles staged through
//     registers.
//   * attn_pp_kernel (head dim 128, 16-bit, the default there): 8 waves (256 queries); K and V tiles
//     reach a 4-stage LDS ring by direct-to-LDS loads; the two waves sharing a SIMD alternate MFMA and
//     softmax phases between workgroup barriers (ping-pong); 32x32x16 MFMAs.
//   * attn_pp16_kernel (WE_ATTN_PATH=mfma16): the same ping-pong on 16x16x32 MFMAs. Faster while the chip has
//     power to spare (a single call after idle), slower at the power limit a run of blocks holds it at.
//   * attn_dma_kernel (WE_ATTN_PATH=ring): the ring with a 3-stage depth and one phase per tile.
// For 16-bit operands at head dim 128 the 32x32x16 kernels run the same per-tile arithmetic in the same order,
// so their outputs agree bit for bit; the 16x16x32 kernel sums the same products in another order inside each
// MFMA.
//
// 16-bit kernel (bf16 or f16 operands, fp32 accumulation, 32x32x16 MFMA):
//   * S^T = K Q^T: the MFMA's A operand is a K tile row (a key), B is the wave's Q held in registers. In the
//     32x32 result a lane owns ONE query (column lane % 32) and 16 keys, so the running max, the rescale of
//     the output and the row sum are per-lane scalars; the two half-waves (the other 16 keys of each 32)
//     meet through one permlane32 swap.
//   * O^T = V^T P^T: P never leaves registers. The 8 values a lane feeds the next MFMA are the keys it
//     owns in the S^T result ({0-3, 8-11} or {4-7, 12-15} of each 16); V^T is written to LDS with bits 2 and
//     3 of the key index swapped, which puts exactly those 8 keys side by side for one 16-byte read.
//   * K rows and V^T rows are XOR-swizzled by 16-byte chunk so the MFMA operand reads are bank-conflict free.
//   * LDS is double-buffered: the next tile's loads are in flight during this tile's MFMAs, then stored to
//     the other buffer; one barrier per tile.
// f32 kernel (reference f32 API, 32x32x2 f32 MFMA, exact f32 products): same work split, a single LDS
// buffer, P kept in f32.
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "internal.h"

namespace we {
namespace {

constexpr int ATT_BM = 128;  // queries per workgroup
constexpr int ATT_BN = 64;   // keys per tile
constexpr int ATT_NT = 256;  // threads per workgroup

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  uint32_t tokens, heads, group, dim;  // group = heads / kvHeads
  uint32_t qs, ks, vs, os;             // elements between consecutive tokens
  uint32_t nqb;                        // query blocks per head
  float scale_log2;                    // log2(e) / sqrt(dim)
  int causal;
};

__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// (query block, head) of this workgroup. When the grid splits evenly over the 8 XCDs, each XCD takes a
// contiguous run of (head-major) blocks, so the workgroups reading one head's K and V share an L2.
__device__ __forceinline__ void block_coords(const AttnArgs& a, uint32_t& qb, uint32_t& h) {
  uint32_t b = blockIdx.x;
  const uint32_t nb = gridDim.x;
  if ((nb & 7u) == 0u) b = (b & 7u) * (nb >> 3) + (b >> 3);
  qb = b % a.nqb;
  h = b / a.nqb;
}

// One 64-key tile for QB blocks of 32 queries of one wave, in three steps (attn_tile16 runs them in order; the
// ping-pong kernel runs the scores of tile t with the P V^T of tile t - 1 in one phase and the softmax in
// the next): S^T = K Q^T, online softmax, O^T += V^T P^T. Every K and V^T fragment read from LDS feeds QB
// MFMAs. ks: the K tile (64 rows of DP values, 16-byte chunks XOR-swizzled by (row >> KSH)); vt: the V^T
// tile (DP rows of 64 keys, keys in bit-2/3-swapped order, chunks swizzled by (row >> 1) & 7). qw[qb]: first
// query of block qb; qi[qb]: this lane's query in it.
template <int DP, bool IS_F16, int QB>
__device__ __forceinline__ void attn_scores16(const char* ks, const u32x4 (&qf)[QB][DP / 16], f32x16 (&sacc)[QB][2],
                                              int c, int hf) {
  constexpr int NCH = DP / 8;
  constexpr int KSH = NCH == 16 ? 0 : NCH == 8 ? 1 : 2;
  static_for<0, QB>([&](auto Q) { sacc[Q][0] = f32x16{}; sacc[Q][1] = f32x16{}; });
  // the two key halves alternate, so consecutive MFMAs never wait on each other's accumulator
  static_for<0, DP / 16>([&](auto S) {
    constexpr int s = S;
    static_for<0, 2>([&](auto B) {
      constexpr int b = B;
      const int r = 32 * b + c;
      const u32x4 af = *(const u32x4*)(ks + r * DP * 2 + (((2 * s + hf) ^ ((r >> KSH) & (NCH - 1))) << 4));
      static_for<0, QB>([&](auto Q) { sacc[Q][b] = mfma_32x32x16<IS_F16>(af, qf[Q][s], sacc[Q][b]); });
    });
  });
}

// FAST (QB = 1): the caller's running max must not move; if it would, the call returns false and changes
// nothing (the caller redoes the tile with the general version). O is then never multiplied.
template <int DP, bool IS_F16, int QB, bool FAST = false>
__device__ __forceinline__ bool attn_softmax16(const f32x16 (&sacc)[QB][2], u32x4 (&pf)[QB][4],
                                               f32x16 (&o)[QB][DP / 32], float (&m)[QB], float (&l)[QB], uint32_t k0,
                                               const uint32_t (&qw)[QB], const uint32_t (&qi)[QB], int hf,
                                               const AttnArgs& a) {
  static_assert(!FAST || QB == 1, "the fast softmax handles one query block");
  bool ok = true;
  static_for<0, QB>([&](auto Q) {
    constexpr int qb = Q;
    // raw scores; keys past the end (or after the query, causal) get -inf
    float x[32];
    const bool mask = (k0 + ATT_BN > a.tokens) || (a.causal && k0 + ATT_BN - 1 > qw[qb]);
    static_for<0, 32>([&](auto I) {
      constexpr int i = I, b = i / 16, v = i % 16;
      x[i] = sacc[qb][b][v];
      if (mask) {
        const uint32_t key = k0 + 32 * b + 8 * (v / 4) + 4 * hf + (v % 4);
        if (key >= a.tokens || (a.causal && key > qi[qb])) x[i] = -__builtin_inff();
      }
    });
    float tmax = x[0];
    static_for<1, 32>([&](auto I) { tmax = fmaxf(tmax, x[I]); });
    // the row max in log2 units: rounding is monotone, so max(x) * scale is exactly max(x * scale)
    tmax = halves_max(tmax) * a.scale_log2;
    const float mn = fmaxf(m[qb], tmax);
    // Lazy rescale: the running max only moves (and O, l are rescaled) when some query of the wave sees its
    // max rise by more than 8 (log2 units); otherwise the stale max stays the shift, so p <= 2^8. Softmax is
    // invariant to the shift, and the wave skips 64 multiplies of O on most tiles.
    const bool rescale = __any(mn > m[qb] + 8.0f);
    if constexpr (FAST) {
      if (rescale) {
        ok = false;
        return;
      }
    }
    const float mref = rescale ? mn : m[qb];
    const float ms = mref == -__builtin_inff() ? 0.0f : mref;
    float ps = 0.0f;
    static_for<0, 4>([&](auto S) {
      constexpr int s = S;
      float p[8];
      static_for<0, 8>([&](auto I) {
        p[I] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[16 * (s / 2) + 8 * (s % 2) + I], a.scale_log2, -ms));
        ps += p[I];
      });
      static_for<0, 4>([&](auto J) {
        constexpr int j = J;
        pf[qb][s][j] = pack2(p[2 * j], p[2 * j + 1], std::integral_constant<bool, IS_F16>{});
      });
    });
    if constexpr (FAST) {
      l[qb] = __builtin_fmaf(l[qb], 1.0f, ps);
    } else {
      // alpha = 1 unless the max moved; multiplying O by it on every tile keeps O in one set of registers
      // (a branch around the multiply makes the compiler copy all of O on the path that skips it)
      const float alpha = rescale ? __builtin_amdgcn_exp2f(m[qb] - ms) : 1.0f;
      l[qb] = __builtin_fmaf(l[qb], alpha, ps);
      if (rescale) m[qb] = mn;
      static_for<0, DP / 32>([&](auto D) { o[qb][D] *= alpha; });
    }
  });
  return ok;
}

template <int DP, bool IS_F16, int QB>
__device__ __forceinline__ void attn_pv16(const char* vt, const u32x4 (&pf)[QB][4], f32x16 (&o)[QB][DP / 32], int c,
                                          int hf) {
  static_for<0, 4>([&](auto S) {
    constexpr int s = S;
    static_for<0, DP / 32>([&](auto D) {
      constexpr int db = D;
      const int r = 32 * db + c;
      const u32x4 vf = *(const u32x4*)(vt + r * ATT_BN * 2 + (((2 * s + hf) ^ ((r >> 1) & 7)) << 4));
      static_for<0, QB>([&](auto Q) { o[Q][db] = mfma_32x32x16<IS_F16>(vf, pf[Q][s], o[Q][db]); });
    });
  });
}

template <int DP, bool IS_F16, int QB>
__device__ __forceinline__ void attn_tile16(const char* ks, const char* vt, const u32x4 (&qf)[QB][DP / 16],
                                            f32x16 (&o)[QB][DP / 32], float (&m)[QB], float (&l)[QB], uint32_t k0,
                                            const uint32_t (&qw)[QB], const uint32_t (&qi)[QB], int c, int hf,
                                            const AttnArgs& a) {
  f32x16 sacc[QB][2];
  u32x4 pf[QB][4];
  attn_scores16<DP, IS_F16, QB>(ks, qf, sacc, c, hf);
  attn_softmax16<DP, IS_F16, QB>(sacc, pf, o, m, l, k0, qw, qi, hf, a);
  attn_pv16<DP, IS_F16, QB>(vt, pf, o, c, hf);
}

// O = O^T / l for this lane's query, as 16-bit values, 4 consecutive dims per store.
template <int DP, bool IS_F16>
__device__ __forceinline__ void attn_store16(const f32x16 (&o)[DP / 32], float l, uint32_t qi, uint32_t h, int hf,
                                             const AttnArgs& a) {
  const float inv = 1.0f / halves_sum(l);
  if (qi >= a.tokens) return;
  uint16_t* O = (uint16_t*)a.o + (size_t)qi * a.os + (size_t)h * a.dim;
  static_for<0, DP / 32>([&](auto D) {
    constexpr int db = D;
    static_for<0, 4>([&](auto G) {
      constexpr int g4 = G;
      const uint32_t d = 32 * db + 8 * g4 + 4 * hf;
      if (d < a.dim) {
        const auto tag = std::integral_constant<bool, IS_F16>{};
        const u32x2 w{pack2(o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv, tag),
                      pack2(o[db][4 * g4 + 2] * inv, o[db][4 * g4 + 3] * inv, tag)};
        *(u32x2*)(O + d) = w;
      }
    });
  });
}

// ------------------------------------------------------------------------------------ 16-bit kernel
// DP = head dim padded to 32, 64 or 128 (dims below DP read as zeros and are not stored).
template <int DP, bool IS_F16>
__global__ void __launch_bounds__(ATT_NT, 2) attn16_kernel(AttnArgs a) {
  constexpr int NCH = DP / 8;                       // 16-byte chunks per K row
  constexpr int KSH = NCH == 16 ? 0 : NCH == 8 ? 1 : 2;
  constexpr int KS_BYTES = ATT_BN * DP * 2;
  constexpr int STAGE = 2 * KS_BYTES;               // K tile + V^T tile
  constexpr int KL = ATT_BN * NCH / ATT_NT;         // K chunks each thread loads
  constexpr int VU = (ATT_BN / 4) * NCH;            // V units: 4 keys x 8 dims
  static_assert(KL >= 1 && VU <= ATT_NT, "tile split");
  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

  uint32_t qb, h;
  block_coords(a, qb, h);
  const uint32_t g = h / a.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hf = lane >> 5;
  const uint32_t q0 = qb * ATT_BM;
  const uint32_t qw = q0 + 32 * wave;  // first query of this wave
  const uint32_t qi = qw + c;          // this lane's query
  const uint16_t* Q = (const uint16_t*)a.q;
  const uint16_t* K = (const uint16_t*)a.k + (size_t)g * a.dim;
  const uint16_t* V = (const uint16_t*)a.v + (size_t)g * a.dim;

  // Q as the B operand of S^T = K Q^T: query qi, dims 16 s + 8 hf .. + 7
  u32x4 qf[DP / 16];
  static_for<0, DP / 16>([&](auto S) {
    constexpr int s = S;
    const uint32_t d = 16 * s + 8 * hf;
    qf[s] = u32x4{0, 0, 0, 0};
    if (qi < a.tokens && d < a.dim) qf[s] = *(const u32x4*)(Q + (size_t)qi * a.qs + (size_t)h * a.dim + d);
  });

  const uint32_t kv_end = a.causal ? min(a.tokens, q0 + ATT_BM) : a.tokens;
  const int nt = (int)((kv_end + ATT_BN - 1) / ATT_BN);

  u32x4 kr[KL], vr[4];
  auto load_tile = [&](int t) {
    const uint32_t k0 = (uint32_t)t * ATT_BN;
#pragma unroll
    for (int i = 0; i < KL; i++) {
      const int idx = tid + ATT_NT * i, r = idx / NCH, ch = idx % NCH;
      const uint32_t key = k0 + r, d = 8 * ch;
      kr[i] = u32x4{0, 0, 0, 0};
      if (key < a.tokens && d < a.dim) kr[i] = *(const u32x4*)(K + (size_t)key * a.ks + d);
    }
    if (tid < VU) {
      const int kg = tid & 15, ch = tid >> 4;
      const uint32_t d = 8 * ch;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t key = k0 + 4 * kg + j;
        vr[j] = u32x4{0, 0, 0, 0};
        if (key < a.tokens && d < a.dim) vr[j] = *(const u32x4*)(V + (size_t)key * a.vs + d);
      }
    }
  };
  auto store_tile = [&](int stage) {
    char* ks = lds + stage * STAGE;
    char* vt = ks + KS_BYTES;
#pragma unroll
    for (int i = 0; i < KL; i++) {
      const int idx = tid + ATT_NT * i, r = idx / NCH, ch = idx % NCH;
      *(u32x4*)(ks + r * DP * 2 + ((ch ^ ((r >> KSH) & (NCH - 1))) << 4)) = kr[i];
    }
    if (tid < VU) {
      const int kg = tid & 15, ch = tid >> 4;
      // keys 4 kg .. 4 kg + 3 sit at position 4 kg with bits 2 and 3 swapped
      const int pos = 16 * (kg >> 2) + 4 * (((kg & 1) << 1) | ((kg >> 1) & 1));
      const int pch = pos >> 3, off = (pos & 7) * 2;
#pragma unroll
      for (int dd = 0; dd < 8; dd++) {
        const int d = 8 * ch + dd, w = dd >> 1, sh = (dd & 1) * 16;
        const uint32_t e0 = (vr[0][w] >> sh) & 0xffffu, e1 = (vr[1][w] >> sh) & 0xffffu;
        const uint32_t e2 = (vr[2][w] >> sh) & 0xffffu, e3 = (vr[3][w] >> sh) & 0xffffu;
        *(u32x2*)(vt + d * ATT_BN * 2 + ((pch ^ ((d >> 1) & 7)) << 4) + off) = u32x2{e0 | (e1 << 16), e2 | (e3 << 16)};
      }
    }
  };

  f32x16 o1[1][DP / 32];
  static_for<0, DP / 32>([&](auto D) { o1[0][D] = f32x16{}; });
  float m1[1] = {-__builtin_inff()}, l1[1] = {0.0f};
  const uint32_t qw1[1] = {qw}, qi1[1] = {qi};
  u32x4 qf1[1][DP / 16];
  static_for<0, DP / 16>([&](auto S) { qf1[0][S] = qf[S]; });

  if (nt > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();
  for (int t = 0; t < nt; t++) {
    if (t + 1 < nt) load_tile(t + 1);
    const uint32_t k0 = (uint32_t)t * ATT_BN;
    // a wave whose queries all precede the tile has nothing to add (causal)
    if (!(a.causal && k0 > qw + 31)) {
      const char* ks = lds + (t & 1) * STAGE;
      attn_tile16<DP, IS_F16, 1>(ks, ks + KS_BYTES, qf1, o1, m1, l1, k0, qw1, qi1, c, hf, a);
    }
    if (t + 1 < nt) store_tile((t + 1) & 1);
    __syncthreads();
  }
  attn_store16<DP, IS_F16>(o1[0], l1[0], qi, h, hf, a);
}

// ------------------------------------------------------------------------------------ V^T for the DMA path
// VT[g][d][p] = V[key(p)][g][d], key(p) = p with bits 2 and 3 swapped inside its group of 16 (the order the
// tile update reads V^T in), zero past the last token; p < tp (tokens rounded up to 64). One workgroup
// moves 64 positions x 128 dims of one kv head through LDS.
__global__ void __launch_bounds__(256) attn_vt_kernel(const uint16_t* v, uint32_t vs, uint32_t tokens, uint32_t tp,
                                                      uint16_t* vt) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][136];
  const int tid = threadIdx.x;
  const uint32_t p0 = blockIdx.x * 64, g = blockIdx.y;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int idx = tid + 256 * i, r = idx >> 4, ch = idx & 15;
    const uint32_t p = p0 + r;
    const uint32_t key = (p & ~15u) | (p & 3u) | ((p & 4u) << 1) | ((p & 8u) >> 1);
    u32x4 val = u32x4{0u, 0u, 0u, 0u};
    if (key < tokens) val = *(const u32x4*)(v + (size_t)key * vs + (size_t)g * 128 + ch * 8);
    *(u32x4*)&tile[r][ch * 8] = val;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int idx = tid + 256 * i, d = idx >> 3, ch = idx & 7;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) w[e] = (uint32_t)tile[ch * 8 + 2 * e][d] | ((uint32_t)tile[ch * 8 + 2 * e + 1][d] << 16);
    *(u32x4*)(vt + ((size_t)g * 128 + d) * tp + p0 + ch * 8) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// ------------------------------------------------------------------------------------ 16-bit, DMA ring
// Head dim 128. A workgroup owns 256 queries: 8 waves of 32 (QB = 1, two waves per SIMD). QB = 2 (4 waves of
// 64, each K and V^T fragment feeding two MFMAs) needs more than 256 VGPRs and spills; measured 2.5x slower,
// it is not launched. K tiles and V^T tiles (from attn_vt_kernel) reach LDS
// through direct-to-LDS loads into a 3-stage ring: the tile two ahead is issued right after the barrier that
// opens each tile, so its latency is hidden behind two tiles of MFMAs, with no staging registers.
constexpr int DMA_BM = 256;
constexpr int DMA_NS = 3;
constexpr uint32_t kAttInvalid = 0x80000000u;

template <bool IS_F16, int QB>
__global__ void __launch_bounds__(512 / QB, 1) attn_dma_kernel(AttnArgs a, const uint16_t* vtg, uint32_t tp,
                                                               uint32_t kv_heads) {
  constexpr int DP = 128;
  constexpr int NW = 8 / QB;                 // waves
  constexpr int IPW = 16 / NW;               // load instructions per wave per tile, each of K and V^T
  constexpr int KS_BYTES = ATT_BN * DP * 2;  // 16 KB
  constexpr int STAGE = 2 * KS_BYTES;        // K + V^T
  __shared__ __attribute__((aligned(1024))) char lds[DMA_NS * STAGE];

  uint32_t qblk, h;
  block_coords(a, qblk, h);
  const uint32_t g = h / a.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hf = lane >> 5;
  const uint32_t q0 = qblk * DMA_BM;
  uint32_t qw[QB], qi[QB];
  static_for<0, QB>([&](auto Q) {
    qw[Q] = q0 + 32 * QB * wave + 32 * Q;
    qi[Q] = qw[Q] + c;
  });
  const uint16_t* Qp = (const uint16_t*)a.q;

  u32x4 qf[QB][DP / 16];
  static_for<0, QB>([&](auto Q) {
    static_for<0, DP / 16>([&](auto S) {
      constexpr int s = S;
      const uint32_t d = 16 * s + 8 * hf;
      qf[Q][s] = u32x4{0, 0, 0, 0};
      if (qi[Q] < a.tokens) qf[Q][s] = *(const u32x4*)(Qp + (size_t)qi[Q] * a.qs + (size_t)h * DP + d);
    });
  });

  const uint32_t kv_end = a.causal ? min(a.tokens, q0 + DMA_BM) : a.tokens;
  const int nt = (int)((kv_end + ATT_BN - 1) / ATT_BN);
  const uint32_t k_bytes = ((a.tokens - 1) * a.ks + kv_heads * DP) * 2;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)a.k, (short)0, (int)k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)vtg, (short)0, (int)(kv_heads * DP * tp * 2), 0x00020000);
  // instruction j (0 .. 15) fills K rows 4j .. 4j + 3, or V^T rows 8j .. 8j + 7; wave w issues j = w + NW u
  auto issue = [&](int t, int stage) {
    const uint32_t k0 = (uint32_t)t * ATT_BN;
    char* base = lds + stage * STAGE;
#pragma unroll
    for (int u = 0; u < IPW; u++) {
      const int j = wave + NW * u;
      const int row = 4 * j + (lane >> 4), phys = lane & 15, logical = phys ^ (row & 15);
      const uint32_t key = k0 + row;
      const uint32_t off = key < a.tokens ? (key * a.ks + g * DP + logical * 8) * 2 : kAttInvalid;
      dma16(rk, base + j * 1024, off);
    }
#pragma unroll
    for (int u = 0; u < IPW; u++) {
      const int j = wave + NW * u;
      const int row = 8 * j + (lane >> 3), phys = lane & 7, logical = phys ^ ((row >> 1) & 7);
      const uint32_t off = ((g * DP + row) * tp + k0 + logical * 8) * 2;
      dma16(rv, base + KS_BYTES + j * 1024, off);
    }
  };

  f32x16 o[QB][DP / 32];
  float m[QB], l[QB];
  static_for<0, QB>([&](auto Q) {
    static_for<0, DP / 32>([&](auto D) { o[Q][D] = f32x16{}; });
    m[Q] = -__builtin_inff();
    l[Q] = 0.0f;
  });
  if (nt > 0) issue(0, 0);
  if (nt > 1) issue(1, 1);
  // Q is consumed here, so the compiler waits for its loads once, before the loop, instead of at the first
  // MFMA of every tile (it cannot tell the first iteration from the others)
#pragma unroll
  for (int qq = 0; qq < QB; qq++)
#pragma unroll
    for (int ss = 0; ss < DP / 16; ss++) asm volatile("" ::"v"(qf[qq][ss]));
  int st = 0;
  for (int t = 0; t < nt; t++) {
    // own loads of tile t done (tile t + 1's 2 IPW may still be in flight), then everyone's
    if (t + 1 < nt) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * IPW) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // tile t + 2 goes to the stage tile t - 1 used; every wave has finished reading it
    if (t + 2 < nt) issue(t + 2, st == 0 ? 2 : st - 1);
    const uint32_t k0 = (uint32_t)t * ATT_BN;
    if (!(a.causal && k0 > qw[QB - 1] + 31)) {
      const char* ks = lds + st * STAGE;
      attn_tile16<DP, IS_F16, QB>(ks, ks + KS_BYTES, qf, o, m, l, k0, qw, qi, c, hf, a);
    }
    st = st == DMA_NS - 1 ? 0 : st + 1;
  }
  static_for<0, QB>([&](auto Q) { attn_store16<DP, IS_F16>(o[Q], l[Q], qi[Q], h, hf, a); });
}

// ------------------------------------------------------------------------------------ 16-bit, ping-pong
// Same work split, LDS layout and per-tile arithmetic as attn_dma_kernel (QB = 1, 8 waves of 32 queries), with
// the MFMA and the softmax work of the two waves that share a SIMD (waves w and w + 4: a workgroup's waves go
// round-robin over the 4 SIMDs) kept out of step. Each wave alternates
//   M(t): O^T += V^T P^T of tile t - 1, then S^T = K Q^T of tile t   (32 MFMAs, LDS reads)
//   V(t): the online softmax of tile t                                (VALU: scale, max, exp2, sum, pack)
// and group 1 (waves 4-7) runs one phase behind group 0, so between two workgroup barriers one wave of every
// SIMD issues MFMAs while the other one runs its softmax. The order of the operations on O is the one of
// attn_tile16 (rescale by tile t's softmax, then add tile t's P V^T), so the result is the same bit for bit.
// Interval j (between barriers): group 0 runs phase j (even: M(j / 2), odd: V((j - 1) / 2)), group 1 phase
// j - 1; M(nt) is the last P V^T alone. K of tile t is read in intervals 2t and 2t + 1, its V^T in 2t + 2 and
// 2t + 3, so tile t + PP_NS goes into its stage at the start of interval 2t + 4. Tile t is first read in
// interval 2t: every wave waits for its own loads of it before the barrier that ends interval 2t - 1.
constexpr int PP_NS = 4;

// M phase of the ping-pong kernel (head dim 128, 32 queries): O^T += V^T P^T of the previous tile (PV), then
// S^T = K Q^T of this tile (SC), as one pipeline of 16-byte LDS fragment reads running PP_LA reads ahead of
// the MFMAs. A scheduling barrier after every step keeps that order: left to itself the compiler issues all
// 32 reads first, runs out of registers and moves O between register ranges on every tile. Each
// accumulator sees its MFMAs in the order of attn_pv16 / attn_scores16, so the results are the same.
constexpr int PP_LA = 5;
typedef short attn_v4s __attribute__((ext_vector_type(4)));

// Per-lane constants of the transposing V read (VTR): the V tile sits in LDS key-major like the K tile (rows of
// 128 dims, 16-byte chunk c of row r at chunk c ^ (r & 15)). ds_read_b64_tr_b16 hands lane 4a + b of each
// 16-lane group element b of the 4-value rows that lanes a, a + 4, a + 8, a + 12 address (measured on gfx950).
// Lane 4q + a' of a group therefore addresses key kq + q of dims d0 + 4a' .. + 3, and lane 4a + b receives
// keys kq .. kq + 3 of dim d0 + 4a + b: the 16 lanes get 16 consecutive dims. With the group's dims
// 32 db + (lane & 16) + (0..15) and kq = 4 hf (then 8 + 4 hf), a lane gathers the 8 keys {4hf .. 4hf + 3,
// 8 + 4hf .. 8 + 4hf + 3} of its dim 32 db + c: the k order of its P fragment.
struct VtrLane {
  uint32_t base1, base2;  // byte offsets of (key kq + q, sub-chunk) for the two reads, before the chunk term
  uint32_t k1, k2;        // kq + q of the two reads (the XOR swizzle key)
  uint32_t cc;            // the lane's chunk inside its 32-dim block: (lane & 16) / 8 + a' / 2
};

__device__ __forceinline__ VtrLane vtr_lane(int lane) {
  const int hf = lane >> 5, q = (lane & 15) >> 2, ap = lane & 3;
  VtrLane v;
  v.k1 = (uint32_t)(4 * hf + q);
  v.k2 = v.k1 + 8u;
  v.cc = (uint32_t)(((lane & 16) >> 3) + (ap >> 1));
  const uint32_t sub = (uint32_t)(ap & 1) * 8u;
  v.base1 = v.k1 * 256u + sub;
  v.base2 = v.k2 * 256u + sub;
  return v;
}

template <bool IS_F16, bool PV, bool SC, bool VTR = false>
__device__ __forceinline__ void attn_mphase16(const char* vt, const char* ks, const u32x4 (&qf)[1][8],
                                              const u32x4 (&pf)[1][4], f32x16 (&o)[1][4], f32x16 (&sacc)[1][2],
                                              int c, int hf, const VtrLane& vl = VtrLane{}) {
  constexpr int N = (PV ? 16 : 0) + (SC ? 16 : 0);
  // step i is P V^T step i / 2 (even i) or scores step i / 2 (odd i) when both run, so the MFMAs of one
  // accumulator are 4 (P V^T) or 8 (scores) apart and none waits on the previous one's result
  constexpr auto is_pv = [](int i) { return PV && (!SC || i % 2 == 0); };
  constexpr auto idx = [](int i) { return PV && SC ? i / 2 : i; };
  auto frag = [&](auto I) -> u32x4 {
    constexpr int i = I;
    if constexpr (is_pv(i) && VTR) {
      constexpr int s = idx(i) / 4, db = idx(i) % 4;  // dims 32 db + c, keys 16 s .. 16 s + 15 of the V tile
      const char* t = vt + s * 16 * 256;
      const uint32_t o1 = vl.base1 + ((((uint32_t)(4 * db) + vl.cc) ^ vl.k1) << 4);
      const uint32_t o2 = vl.base2 + ((((uint32_t)(4 * db) + vl.cc) ^ vl.k2) << 4);
      const attn_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) attn_v4s*)(t + o1));
      const attn_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) attn_v4s*)(t + o2));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      return u32x4{l2.x, l2.y, h2.x, h2.y};
    } else if constexpr (is_pv(i)) {
      constexpr int s = idx(i) / 4, db = idx(i) % 4;  // V^T rows 32 db + c, keys 16 s .. 16 s + 15
      const int r = 32 * db + c;
      return *(const u32x4*)(vt + r * ATT_BN * 2 + (((2 * s + hf) ^ ((r >> 1) & 7)) << 4));
    } else {
      constexpr int s = idx(i) / 2, b = idx(i) % 2;  // K row 32 b + c, dims 16 s .. 16 s + 15
      const int r = 32 * b + c;
      return *(const u32x4*)(ks + r * 256 + (((2 * s + hf) ^ (r & 15)) << 4));
    }
  };
  if constexpr (SC) {
    sacc[0][0] = f32x16{};
    sacc[0][1] = f32x16{};
  }
  u32x4 f[PP_LA + 1];
  static_for<0, PP_LA>([&](auto I) {
    if constexpr (I < N) f[I] = frag(I);
  });
  static_for<0, N>([&](auto I) {
    constexpr int i = I;
    if constexpr (i + PP_LA < N) f[(i + PP_LA) % (PP_LA + 1)] = frag(std::integral_constant<int, i + PP_LA>{});
    if constexpr (is_pv(i)) {
      constexpr int s = idx(i) / 4, db = idx(i) % 4;
      o[0][db] = mfma_32x32x16<IS_F16>(f[i % (PP_LA + 1)], pf[0][s], o[0][db]);
    } else {
      constexpr int s = idx(i) / 2, b = idx(i) % 2;
      sacc[0][b] = mfma_32x32x16<IS_F16>(f[i % (PP_LA + 1)], qf[0][s], sacc[0][b]);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

// V tiles reach LDS key-major through the same direct-to-LDS loads as K (no V^T pre-pass); the P V^T
// fragments are gathered from them by ds_read_b64_tr_b16 (VtrLane).
template <bool IS_F16, bool CAUSAL>
__global__ void __launch_bounds__(512, 1) attn_pp_kernel(AttnArgs a, uint32_t kv_heads) {
  constexpr int DP = 128, NW = 8, IPW = 2;
  constexpr int KS_BYTES = ATT_BN * DP * 2;  // 16 KB
  constexpr int STAGE = 2 * KS_BYTES;        // K + V
  __shared__ __attribute__((aligned(1024))) char lds[PP_NS * STAGE];

  uint32_t qblk, h;
  block_coords(a, qblk, h);
  const uint32_t g = h / a.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int c = lane & 31, hf = lane >> 5;
  const uint32_t q0 = qblk * DMA_BM;
  const uint32_t qw[1] = {q0 + 32 * wave};
  const uint32_t qi[1] = {qw[0] + c};
  const uint16_t* Qp = (const uint16_t*)a.q;

  u32x4 qf[1][DP / 16];
  static_for<0, DP / 16>([&](auto S) {
    constexpr int s = S;
    qf[0][s] = u32x4{0, 0, 0, 0};
    if (qi[0] < a.tokens) qf[0][s] = *(const u32x4*)(Qp + (size_t)qi[0] * a.qs + (size_t)h * DP + 16 * s + 8 * hf);
  });

  const uint32_t kv_end = CAUSAL ? min(a.tokens, q0 + DMA_BM) : a.tokens;
  const int nt = (int)((kv_end + ATT_BN - 1) / ATT_BN);
  const uint32_t k_bytes = ((a.tokens - 1) * a.ks + kv_heads * DP) * 2;
  const uint32_t v_bytes = ((a.tokens - 1) * a.vs + kv_heads * DP) * 2;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)a.k, (short)0, (int)k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)a.v, (short)0, (int)v_bytes, 0x00020000);
  // instruction j (0 .. 15) fills K rows 4j .. 4j + 3, or V rows 4j .. 4j + 3 (keys past the last token load
  // zeros); wave w issues j = w + 8u
  auto issue = [&](int t) {
    const uint32_t k0 = (uint32_t)t * ATT_BN;
    char* base = lds + (t % PP_NS) * STAGE;
#pragma unroll
    for (int u = 0; u < IPW; u++) {
      const int j = wave + NW * u;
      const int row = 4 * j + (lane >> 4), phys = lane & 15, logical = phys ^ (row & 15);
      const uint32_t key = k0 + row;
      dma16(rk, base + j * 1024, key < a.tokens ? (key * a.ks + g * DP + logical * 8) * 2 : kAttInvalid);
    }
#pragma unroll
    for (int u = 0; u < IPW; u++) {
      const int j = wave + NW * u;
      const int row = 4 * j + (lane >> 4), phys = lane & 15, logical = phys ^ (row & 15);
      const uint32_t key = k0 + row;
      dma16(rv, base + KS_BYTES + j * 1024, key < a.tokens ? (key * a.vs + g * DP + logical * 8) * 2 : kAttInvalid);
    }
  };
  const VtrLane vl = vtr_lane(lane);
  // own loads of tile t complete; the tiles issued after it (at most PP_NS - 1) may still be in flight
  auto wait_tile = [&](int t) {
    const int ahead = min(nt - 1, max(PP_NS - 1, t + 1)) - t;
    if (ahead >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * IPW) : "memory");
    else if (ahead == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * IPW) : "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * IPW) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // tile t contributes to this wave's queries (causal: not entirely after them)
  auto active = [&](int t) { return !CAUSAL || (uint32_t)t * ATT_BN <= qw[0] + 31; };
  const char* kst = lds;             // K of tile t: kst + (t % PP_NS) * STAGE
  const char* vst = lds + KS_BYTES;  // V of tile t (key-major)

  f32x16 o[1][DP / 32];
  static_for<0, DP / 32>([&](auto D) { o[0][D] = f32x16{}; });
  float m[1] = {-__builtin_inff()}, l[1] = {0.0f};
  f32x16 sacc[1][2];
  u32x4 pf[1][4];
  for (int t = 0; t < PP_NS; t++)
    if (t < nt) issue(t);
  // Q is consumed here, so the compiler waits for its loads once, before the loop
#pragma unroll
  for (int ss = 0; ss < DP / 16; ss++) asm volatile("" ::"v"(qf[0][ss]));
  wait_tile(0);
  barrier();
  if (grp == 1) barrier();  // group 1 runs one phase behind group 0
  // tile 0: M(0) is the scores alone
  if (active(0)) attn_mphase16<IS_F16, false, true>(nullptr, kst, qf, pf, o, sacc, c, hf);
  if (grp == 1 && nt > 1) wait_tile(1);
  barrier();
  if (active(0)) attn_softmax16<DP, IS_F16, 1>(sacc, pf, o, m, l, 0u, qw, qi, hf, a);
  if (grp == 0 && nt > 1) wait_tile(1);
  barrier();
  auto m_half = [&](int t) {
    if (grp == 0 && t >= 2 && t + 2 < nt) issue(t + 2);
    const int cs = (t % PP_NS) * STAGE, ps = ((t - 1) % PP_NS) * STAGE;
    // causal: the scores of a tile no query of this wave sees are computed and left unused
    // the wave in its MFMA phase wins issue arbitration over its SIMD's softmax wave (causal 4608 x 24 x 128:
    // 215 -> 212 us; non-causal unchanged)
    __builtin_amdgcn_s_setprio(3);
    if (active(t - 1)) attn_mphase16<IS_F16, true, true, true>(vst + ps, kst + cs, qf, pf, o, sacc, c, hf, vl);
    __builtin_amdgcn_s_setprio(0);
    if (grp == 1 && t + 1 < nt) wait_tile(t + 1);
    barrier();
    if (grp == 1 && t + 3 < nt) issue(t + 3);
  };
  auto v_end = [&](int t) {
    if (grp == 0 && t + 1 < nt) wait_tile(t + 1);
    barrier();
  };
  // While no query's max moves (most tiles once the first has set it), the softmax never touches O. The
  // first tile that would move it, and every tile after, takes the general step (O multiplied by alpha).
  int t = 1;
  for (; t < nt; t++) {
    m_half(t);
    if (active(t) && !attn_softmax16<DP, IS_F16, 1, true>(sacc, pf, o, m, l, (uint32_t)t * ATT_BN, qw, qi, hf, a))
      break;
    v_end(t);
  }
  if (t < nt) {
    attn_softmax16<DP, IS_F16, 1>(sacc, pf, o, m, l, (uint32_t)t * ATT_BN, qw, qi, hf, a);
    v_end(t);
    for (t++; t < nt; t++) {
      m_half(t);
      if (active(t)) attn_softmax16<DP, IS_F16, 1>(sacc, pf, o, m, l, (uint32_t)t * ATT_BN, qw, qi, hf, a);
      v_end(t);
    }
  }
  // M(nt): the last P V^T
  if (active(nt - 1))
    attn_mphase16<IS_F16, true, false, true>(vst + ((nt - 1) % PP_NS) * STAGE, nullptr, qf, pf, o, sacc, c, hf, vl);
  if (grp == 0) barrier();  // both groups pass the same number of barriers
  attn_store16<DP, IS_F16>(o[0], l[0], qi[0], h, hf, a);
}

// ------------------------------------------------------------------------------------ 16-bit, ping-pong, 16x16x32
// The ping-pong kernel's work split, LDS ring, loads and schedule with the products on 16x16x32 MFMAs. Measured at
// the block shape (4608 tokens, 24 heads): alone after settling 250 us against 267 us for attn_pp_kernel, but after
// 20 block forwards (the power limit a run of blocks holds the chip at) 303-311 against 283-288 us, so it is not the
// default. A wave's 32 queries are two blocks of 16; lane (c16, g): c16 = lane & 15, g = lane >> 4.
//   S^T block (kb, qb) = K rows 16 kb .. 16 kb + 15 of the tile times Q^T of query block qb (A = K, the lane's key
//   row 16 kb + c16 and dims 8 g .. of each 32-dim step; B = Q, query 16 qb + c16): the lane holds the scores of
//   keys 16 kb + 4 g + e (e = 0..3) for query 16 qb + c16.
//   P V^T step ks covers keys 32 ks .. 32 ks + 31 with k slot group g <-> keys 32 ks + 4 g + e and 32 ks + 16 + 4 g
//   + e: exactly the scores the lane holds for kb = 2 ks and 2 ks + 1, so P stays in the lane. The V^T fragments
//   are gathered from the key-major V tile by ds_read_b64_tr_b16 in that key order (two reads per fragment).
//   O^T block (db, qb): the lane holds dims 16 db + 4 g + e of query 16 qb + c16.
// The running max and sum are per query; a query's four lane groups share them (the max is reduced across the
// groups every tile, the sum only at the end).

struct Vtr16 {
  uint32_t base;  // byte offset of the lane's first row and 8-byte half, before the chunk term
  uint32_t xk;    // the XOR swizzle key of the lane's rows (vswz16)
  uint32_t cc;    // the lane's 16-byte chunk inside a 16-dim block
};

// This kernel's V tile puts 16-byte chunk c of key row r at c ^ vswz16(r). A transposing read of a 16-lane group
// touches rows 4 g + q (q = 0..3) at chunks 2 db and 2 db + 1: with the K tile's swizzle (r & 15) rows 4 g and
// 4 g + 1 put one of those chunks on the same banks; 2 (r & 7) sends the 4 rows (and the other group of the
// 32-lane half, rows + 4) to 16 distinct chunk positions.
__device__ __forceinline__ int vswz16(int r) { return 2 * (r & 7); }

// ds_read_b64_tr_b16: in each group of 16 lanes, lane 4 q + a' addresses key kq + q of dims d0 + 4 a' .. + 3, and
// lane 4 a + b receives keys kq .. kq + 3 of dim d0 + 4 a + b (measured on gfx950). With kq = 4 g (then 16 + 4 g)
// and d0 = 16 db, lane (c16, g) gathers dim 16 db + c16 of the keys of its P fragment.
__device__ __forceinline__ Vtr16 vtr16_lane(int lane) {
  const int g = lane >> 4, q = (lane & 15) >> 2, ap = lane & 3;
  Vtr16 v;
  const int kr = 4 * g + q;  // the row inside 16 (rows + 16 and + 32 ks have the same swizzle)
  v.xk = (uint32_t)vswz16(kr);
  v.base = (uint32_t)kr * 256u + (uint32_t)(ap & 1) * 8u;
  v.cc = (uint32_t)(ap >> 1);
  return v;
}

template <int DB, int KS>
__device__ __forceinline__ u32x4 vtr16_frag(const char* vt, const Vtr16& v) {
  const char* t = vt + KS * 32 * 256 + v.base + ((((uint32_t)(2 * DB) + v.cc) ^ v.xk) << 4);
  const attn_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) attn_v4s*)t);
  const attn_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) attn_v4s*)(t + 16 * 256));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{l2.x, l2.y, h2.x, h2.y};
}

// max / sum over the four lane groups of a query (lanes c16, c16 + 16, c16 + 32, c16 + 48)
__device__ __forceinline__ float quads_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float quads_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// M phase: O^T += V^T P^T of the previous tile (PV), then S^T = K Q^T of this tile (SC): 32 fragment reads, each
// feeding the two query blocks' MFMAs, pipelined PP_LA reads ahead. PV fragment p: ks = p / 8, db = p % 8 (an O
// block is hit every 8 fragments); SC fragment q: step q / 4, kb = q % 4 (an S block every 4).
template <bool IS_F16, bool PV, bool SC>
__device__ __forceinline__ void attn_mphase_q16(const char* vt, const char* ks, const u32x4 (&qf)[2][4],
                                                const u32x4 (&pf)[2][2], f32x4 (&o)[8][2], f32x4 (&sacc)[4][2],
                                                int c16, int g, const Vtr16& vl) {
  constexpr int N = (PV ? 16 : 0) + (SC ? 16 : 0);
  constexpr auto is_pv = [](int i) { return PV && (!SC || i % 2 == 0); };
  constexpr auto idx = [](int i) { return PV && SC ? i / 2 : i; };
  auto frag = [&](auto I) -> u32x4 {
    constexpr int i = I;
    if constexpr (is_pv(i)) {
      constexpr int pi = idx(i);
      return vtr16_frag<pi % 8, pi / 8>(vt, vl);
    } else {
      constexpr int qi = idx(i), st = qi / 4, kb = qi % 4;
      return *(const u32x4*)(ks + (16 * kb + c16) * 256 + (((4 * st + g) ^ c16) << 4));
    }
  };
  if constexpr (SC) {
    static_for<0, 4>([&](auto KB) {
      sacc[KB][0] = f32x4{};
      sacc[KB][1] = f32x4{};
    });
  }
  u32x4 f[PP_LA + 1];
  static_for<0, PP_LA>([&](auto I) {
    if constexpr (I < N) f[I] = frag(I);
  });
  static_for<0, N>([&](auto I) {
    constexpr int i = I;
    if constexpr (i + PP_LA < N) f[(i + PP_LA) % (PP_LA + 1)] = frag(std::integral_constant<int, i + PP_LA>{});
    if constexpr (is_pv(i)) {
      constexpr int pi = idx(i), ksi = pi / 8, db = pi % 8;
      o[db][0] = mfma_16x16x32<IS_F16>(f[i % (PP_LA + 1)], pf[ksi][0], o[db][0]);
      o[db][1] = mfma_16x16x32<IS_F16>(f[i % (PP_LA + 1)], pf[ksi][1], o[db][1]);
    } else {
      constexpr int qi = idx(i), st = qi / 4, kb = qi % 4;
      sacc[kb][0] = mfma_16x16x32<IS_F16>(f[i % (PP_LA + 1)], qf[0][st], sacc[kb][0]);
      sacc[kb][1] = mfma_16x16x32<IS_F16>(f[i % (PP_LA + 1)], qf[1][st], sacc[kb][1]);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

// The online softmax of one tile for the wave's two query blocks (the lazy rescale of attn_softmax16: the running
// max moves, and O and the sums are rescaled, only when some query's max would rise by more than 8 in log2 units).
// FAST (the common step): p = exp2(s * scale - m) against the running max as it is, and the call returns false,
// changing nothing, when some lane's sum of p over its 16 scores of a query exceeds 2^8. Every accepted p is then at
// most 2^8, which is all the lazy rescale asks for; a rejected tile takes the full step, whose p equal FAST's
// where its max does not move. Full step: whether some query's max rises by more than 8 is whether some lane's own
// 16 scores do (a query's max is the max of its four lanes'), so it votes on the lanes' maxima and reduces a
// query's max across its lane groups only when it moves.
template <bool IS_F16, bool FAST = false>
__device__ __forceinline__ bool attn_softmax_q16(f32x4 (&sacc)[4][2], u32x4 (&pf)[2][2], f32x4 (&o)[8][2],
                                                 float (&m)[2], float (&l)[2], uint32_t k0, uint32_t qw, int c16,
                                                 int g, const AttnArgs& a) {
  // the mask, in place and behind one wave-uniform branch: only the last tile and (causal) the tiles that cross
  // the wave's queries hold keys to drop; masking twice (a FAST call that returns false, then the full call) is
  // the same as once
  if (__builtin_expect((k0 + ATT_BN > a.tokens) || (a.causal && k0 + ATT_BN - 1 > qw), 0)) {
    static_for<0, 2>([&](auto QB) {
      // key k0 + 4 g + c stays when c < lim: below the sequence end and (causal) at most the query
      const uint32_t query = qw + 16 * QB + (uint32_t)c16;
      const uint32_t end = a.causal ? min(a.tokens, query + 1) : a.tokens;
      const int lim = (int)end - (int)(k0 + 4 * (uint32_t)g);
      static_for<0, 4>([&](auto KB) {
        static_for<0, 4>([&](auto E) {
          constexpr int kb = KB, qb = QB, e = E;
          sacc[kb][qb][e] = 16 * kb + e < lim ? sacc[kb][qb][e] : -__builtin_inff();
        });
      });
    });
  }
  const auto tag = std::integral_constant<bool, IS_F16>{};
  // p of query block qb against the reference max ms, packed to the operand type; returns the lane's sum
  auto exps = [&](auto QB, float ms) -> float {
    constexpr int qb = QB;
    float ps = 0.0f;
    float p[16];
    static_for<0, 16>([&](auto I) {
      p[I] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[I / 4][qb][I % 4], a.scale_log2, -ms));
      ps += p[I];
    });
    static_for<0, 2>([&](auto KS) {
      constexpr int k2 = KS;  // scores of kb = 2 k2 (k slots 0-3) and 2 k2 + 1 (slots 4-7)
      pf[k2][qb] = u32x4{pack2(p[8 * k2], p[8 * k2 + 1], tag), pack2(p[8 * k2 + 2], p[8 * k2 + 3], tag),
                         pack2(p[8 * k2 + 4], p[8 * k2 + 5], tag), pack2(p[8 * k2 + 6], p[8 * k2 + 7], tag)};
    });
    return ps;
  };
  if constexpr (FAST) {
    // m is finite here: the first tile takes the full step and holds a key of every query
    const float ps0 = exps(std::integral_constant<int, 0>{}, m[0]);
    const float ps1 = exps(std::integral_constant<int, 1>{}, m[1]);
    // also rejects inf and NaN sums (a score far above the max)
    if (__any(!(ps0 <= 256.0f) | !(ps1 <= 256.0f))) return false;
    l[0] += ps0;
    l[1] += ps1;
    return true;
  } else {
    float lmax[2];
    bool grow = false;
    static_for<0, 2>([&](auto QB) {
      constexpr int qb = QB;
      float t = fmaxf(fmaxf(sacc[0][qb][0], sacc[0][qb][1]), sacc[0][qb][2]);
      static_for<3, 16>([&](auto I) { t = fmaxf(t, sacc[I / 4][qb][I % 4]); });
      // in log2 units: rounding is monotone, so max(x) * scale is exactly max(x * scale)
      lmax[qb] = t * a.scale_log2;
      grow |= lmax[qb] > m[qb] + 8.0f;
    });
    const bool rescale = __any(grow);
    float mref[2] = {m[0], m[1]};
    if (rescale) {  // wave-uniform: every lane takes part in the cross-lane reduction
      static_for<0, 2>([&](auto QB) { mref[QB] = fmaxf(m[QB], quads_max(lmax[QB])); });
    }
    static_for<0, 2>([&](auto QB) {
      constexpr int qb = QB;
      const float ms = mref[qb] == -__builtin_inff() ? 0.0f : mref[qb];
      const float ps = exps(QB, ms);
      // alpha = 1 unless the max moved; O is multiplied on every full step (a branch around it copies all of O)
      const float alpha = rescale ? __builtin_amdgcn_exp2f(m[qb] - ms) : 1.0f;
      l[qb] = __builtin_fmaf(l[qb], alpha, ps);
      m[qb] = mref[qb];
      static_for<0, 8>([&](auto D) { o[D][qb] *= alpha; });
    });
    return true;
  }
}

template <bool IS_F16, bool CAUSAL>
__global__ void __launch_bounds__(512, 1) attn_pp16_kernel(AttnArgs a, uint32_t kv_heads) {
  constexpr int DP = 128, NW = 8, IPW = 2;
  constexpr int KS_BYTES = ATT_BN * DP * 2;  // 16 KB
  constexpr int STAGE = 2 * KS_BYTES;        // K + V
  __shared__ __attribute__((aligned(1024))) char lds[PP_NS * STAGE];

  uint32_t qblk, h;
  block_coords(a, qblk, h);
  const uint32_t g = h / a.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int c16 = lane & 15, lg = lane >> 4;
  const uint32_t q0 = qblk * DMA_BM;
  const uint32_t qw = q0 + 32 * wave;
  const uint16_t* Qp = (const uint16_t*)a.q;

  // B operand of S^T: query block qb, step st holds dims 32 st + 8 g .. + 7 of query qw + 16 qb + c16
  u32x4 qf[2][4];
  static_for<0, 2>([&](auto QB) {
    const uint32_t qi = qw + 16 * QB + (uint32_t)c16;
    static_for<0, 4>([&](auto ST) {
      qf[QB][ST] = u32x4{0, 0, 0, 0};
      if (qi < a.tokens) qf[QB][ST] = *(const u32x4*)(Qp + (size_t)qi * a.qs + (size_t)h * DP + 32 * ST + 8 * lg);
    });
  });

  const uint32_t kv_end = CAUSAL ? min(a.tokens, q0 + DMA_BM) : a.tokens;
  const int nt = (int)((kv_end + ATT_BN - 1) / ATT_BN);
  const uint32_t k_bytes = ((a.tokens - 1) * a.ks + kv_heads * DP) * 2;
  const uint32_t v_bytes = ((a.tokens - 1) * a.vs + kv_heads * DP) * 2;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)a.k, (short)0, (int)k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)a.v, (short)0, (int)v_bytes, 0x00020000);
  // the tiles' loads: as attn_pp_kernel (instruction j fills K or V rows 4 j .. 4 j + 3; wave w issues j = w + 8 u),
  // the V rows with this kernel's swizzle
  auto issue = [&](int t) {
    const uint32_t k0 = (uint32_t)t * ATT_BN;
    char* base = lds + (t % PP_NS) * STAGE;
#pragma unroll
    for (int u = 0; u < IPW; u++) {
      const int j = wave + NW * u;
      const int row = 4 * j + (lane >> 4), phys = lane & 15, logical = phys ^ (row & 15);
      const uint32_t key = k0 + row;
      dma16(rk, base + j * 1024, key < a.tokens ? (key * a.ks + g * DP + logical * 8) * 2 : kAttInvalid);
    }
#pragma unroll
    for (int u = 0; u < IPW; u++) {
      const int j = wave + NW * u;
      const int row = 4 * j + (lane >> 4), phys = lane & 15, logical = phys ^ vswz16(row);
      const uint32_t key = k0 + row;
      dma16(rv, base + KS_BYTES + j * 1024, key < a.tokens ? (key * a.vs + g * DP + logical * 8) * 2 : kAttInvalid);
    }
  };
  const Vtr16 vl = vtr16_lane(lane);
  auto wait_tile = [&](int t) {
    const int ahead = min(nt - 1, max(PP_NS - 1, t + 1)) - t;
    if (ahead >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * IPW) : "memory");
    else if (ahead == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * IPW) : "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * IPW) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto active = [&](int t) { return !CAUSAL || (uint32_t)t * ATT_BN <= qw + 31; };
  const char* kst = lds;
  const char* vst = lds + KS_BYTES;

  f32x4 o[8][2];
  static_for<0, 8>([&](auto D) {
    o[D][0] = f32x4{};
    o[D][1] = f32x4{};
  });
  float m[2] = {-__builtin_inff(), -__builtin_inff()}, l[2] = {0.0f, 0.0f};
  f32x4 sacc[4][2];
  u32x4 pf[2][2];
  for (int t = 0; t < PP_NS; t++)
    if (t < nt) issue(t);
#pragma unroll
  for (int qq = 0; qq < 2; qq++)
#pragma unroll
    for (int ss = 0; ss < 4; ss++) asm volatile("" ::"v"(qf[qq][ss]));
  wait_tile(0);
  barrier();
  if (grp == 1) barrier();  // group 1 runs one phase behind group 0
  if (active(0)) attn_mphase_q16<IS_F16, false, true>(nullptr, kst, qf, pf, o, sacc, c16, lg, vl);
  if (grp == 1 && nt > 1) wait_tile(1);
  barrier();
  if (active(0)) attn_softmax_q16<IS_F16>(sacc, pf, o, m, l, 0u, qw, c16, lg, a);
  if (grp == 0 && nt > 1) wait_tile(1);
  barrier();
  auto m_half = [&](int t) {
    if (grp == 0 && t >= 2 && t + 2 < nt) issue(t + 2);
    const int cs = (t % PP_NS) * STAGE, ps = ((t - 1) % PP_NS) * STAGE;
    // the wave in its MFMA phase wins issue arbitration over its SIMD's softmax wave
    __builtin_amdgcn_s_setprio(3);
    if (active(t - 1)) attn_mphase_q16<IS_F16, true, true>(vst + ps, kst + cs, qf, pf, o, sacc, c16, lg, vl);
    __builtin_amdgcn_s_setprio(0);
    if (grp == 1 && t + 1 < nt) wait_tile(t + 1);
    barrier();
    if (grp == 1 && t + 3 < nt) issue(t + 3);
  };
  auto v_end = [&](int t) {
    if (grp == 0 && t + 1 < nt) wait_tile(t + 1);
    barrier();
  };
  for (int t = 1; t < nt; t++) {
    m_half(t);
    // the common step leaves O alone; a tile that moves a max takes the full step
    if (active(t) && !attn_softmax_q16<IS_F16, true>(sacc, pf, o, m, l, (uint32_t)t * ATT_BN, qw, c16, lg, a))
      attn_softmax_q16<IS_F16>(sacc, pf, o, m, l, (uint32_t)t * ATT_BN, qw, c16, lg, a);
    v_end(t);
  }
  if (active(nt - 1))
    attn_mphase_q16<IS_F16, true, false>(vst + ((nt - 1) % PP_NS) * STAGE, nullptr, qf, pf, o, sacc, c16, lg, vl);
  if (grp == 0) barrier();  // both groups pass the same number of barriers
  // O = O^T / l: lane (c16, g) stores dims 16 db + 4 g .. + 3 of its two queries
  static_for<0, 2>([&](auto QB) {
    const float inv = 1.0f / quads_sum(l[QB]);
    const uint32_t qi = qw + 16 * QB + (uint32_t)c16;
    if (qi < a.tokens) {
      uint16_t* O = (uint16_t*)a.o + (size_t)qi * a.os + (size_t)h * DP;
      const auto tag = std::integral_constant<bool, IS_F16>{};
      static_for<0, 8>([&](auto D) {
        const f32x4 v = o[D][QB];
        *(u32x2*)(O + 16 * D + 4 * lg) = u32x2{pack2(v[0] * inv, v[1] * inv, tag), pack2(v[2] * inv, v[3] * inv, tag)};
      });
    }
  });
}

// ------------------------------------------------------------------------------------ f32 kernel
template <int DP>
__global__ void __launch_bounds__(ATT_NT, 1) attn32_kernel(AttnArgs a) {
  constexpr int KROW = DP + 4;                       // floats per K row (padding breaks bank aliasing)
  constexpr int F4 = ATT_BN * DP / 4 / ATT_NT;       // float4 per thread per tile, each of K and V
  __shared__ __attribute__((aligned(16))) float ks[ATT_BN * KROW];
  __shared__ __attribute__((aligned(16))) float vs[ATT_BN * DP];

  uint32_t qb, h;
  block_coords(a, qb, h);
  const uint32_t g = h / a.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hf = lane >> 5;
  const uint32_t q0 = qb * ATT_BM;
  const uint32_t qw = q0 + 32 * wave;
  const uint32_t qi = qw + c;
  const float* Q = (const float*)a.q;
  const float* K = (const float*)a.k + (size_t)g * a.dim;
  const float* V = (const float*)a.v + (size_t)g * a.dim;

  // B operand of S^T: step (j, i) contracts dim 8 j + 4 hf + i
  f32x4 qf[DP / 8];
  static_for<0, DP / 8>([&](auto J) {
    const uint32_t d = 8 * J + 4 * hf;
    qf[J] = f32x4{0, 0, 0, 0};
    if (qi < a.tokens && d < a.dim) qf[J] = *(const f32x4*)(Q + (size_t)qi * a.qs + (size_t)h * a.dim + d);
  });

  const uint32_t kv_end = a.causal ? min(a.tokens, q0 + ATT_BM) : a.tokens;
  const int nt = (int)((kv_end + ATT_BN - 1) / ATT_BN);
  f32x16 o[DP / 32];
  static_for<0, DP / 32>([&](auto D) { o[D] = f32x16{}; });
  float m = -__builtin_inff(), l = 0.0f;

  for (int t = 0; t < nt; t++) {
    const uint32_t k0 = (uint32_t)t * ATT_BN;
    f32x4 kr[F4], vr[F4];
#pragma unroll
    for (int i = 0; i < F4; i++) {
      const int idx = tid + ATT_NT * i, r = idx / (DP / 4), d = 4 * (idx % (DP / 4));
      const uint32_t key = k0 + r;
      kr[i] = vr[i] = f32x4{0, 0, 0, 0};
      if (key < a.tokens && (uint32_t)d < a.dim) {
        kr[i] = *(const f32x4*)(K + (size_t)key * a.ks + d);
        vr[i] = *(const f32x4*)(V + (size_t)key * a.vs + d);
      }
    }
    __syncthreads();  // the previous tile is no longer read
#pragma unroll
    for (int i = 0; i < F4; i++) {
      const int idx = tid + ATT_NT * i, r = idx / (DP / 4), d = 4 * (idx % (DP / 4));
      *(f32x4*)(ks + r * KROW + d) = kr[i];
      *(f32x4*)(vs + r * DP + d) = vr[i];
    }
    __syncthreads();
    if (a.causal && k0 > qw + 31) continue;

    f32x16 sacc[2];
    static_for<0, 2>([&](auto B) {
      constexpr int b = B;
      sacc[b] = f32x16{};
      static_for<0, DP / 8>([&](auto J) {
        constexpr int j = J;
        const f32x4 kf = *(const f32x4*)(ks + (32 * b + c) * KROW + 8 * j + 4 * hf);
        static_for<0, 4>([&](auto I) {
          constexpr int i = I;
          sacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i], qf[j][i], sacc[b], 0, 0, 0);
        });
      });
    });
    float x[32];
    const bool mask = (k0 + ATT_BN > a.tokens) || (a.causal && k0 + ATT_BN - 1 > qw);
    static_for<0, 32>([&](auto I) {
      constexpr int i = I, b = i / 16, v = i % 16;
      x[i] = sacc[b][v] * a.scale_log2;
      if (mask) {
        const uint32_t key = k0 + 32 * b + 8 * (v / 4) + 4 * hf + (v % 4);
        if (key >= a.tokens || (a.causal && key > qi)) x[i] = -__builtin_inff();
      }
    });
    float tmax = x[0];
    static_for<1, 32>([&](auto I) { tmax = fmaxf(tmax, x[I]); });
    tmax = halves_max(tmax);
    const float mn = fmaxf(m, tmax);
    const float ms = mn == -__builtin_inff() ? 0.0f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - ms);
    float ps = 0.0f;
    static_for<0, 32>([&](auto I) {
      x[I] = __builtin_amdgcn_exp2f(x[I] - ms);
      ps += x[I];
    });
    l = l * alpha + ps;
    m = mn;
    static_for<0, DP / 32>([&](auto D) { o[D] *= alpha; });
    // O^T += V^T P^T: step v of key block b contracts key 32 b + 8 (v / 4) + 4 hf + v % 4
    static_for<0, DP / 32>([&](auto D) {
      constexpr int db = D;
      static_for<0, 32>([&](auto I) {
        constexpr int i = I, b = i / 16, v = i % 16;
        const float vv = vs[(32 * b + 8 * (v / 4) + 4 * hf + (v % 4)) * DP + 32 * db + c];
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, x[i], o[db], 0, 0, 0);
      });
    });
  }

  const float inv = 1.0f / halves_sum(l);
  if (qi < a.tokens) {
    float* O = (float*)a.o + (size_t)qi * a.os + (size_t)h * a.dim;
    static_for<0, DP / 32>([&](auto D) {
      constexpr int db = D;
      static_for<0, 4>([&](auto G) {
        constexpr int g4 = G;
        const uint32_t d = 32 * db + 8 * g4 + 4 * hf;
        if (d < a.dim)
          *(f32x4*)(O + d) = f32x4{o[db][4 * g4] * inv, o[db][4 * g4 + 1] * inv, o[db][4 * g4 + 2] * inv,
                                   o[db][4 * g4 + 3] * inv};
      });
    });
  }
}

template <class Kern>
hipError_t launch_attn(Kern kern, const AttnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(kern, dim3(a.nqb * a.heads), dim3(ATT_NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace

namespace {
// head dim 128, 16-bit, operand extents within the 32-bit buffer offsets: the DMA kernels
bool attn_dma_ok(const AttnLaunch& L) {
  if (L.dtype == F32 || L.dim != 128 || L.tokens == 0 || L.heads == 0) return false;
  if (L.path == 1) return false;  // Tuning::attn_path: the register-staged kernel
  const uint64_t kb = ((uint64_t)(L.tokens - 1) * L.k_stride + (uint64_t)L.kv_heads * 128) * 2;
  const uint64_t vb = ((uint64_t)(L.tokens - 1) * L.v_stride + (uint64_t)L.kv_heads * 128) * 2;
  return kb < kAttInvalid && vb < kAttInvalid;
}
bool attn_ring_path(const AttnLaunch& L) { return L.path == 2; }
}  // namespace

// Only the ring kernel (WE_ATTN_PATH=ring) stages V^T through scratch; the default kernel reads V as it is.
size_t attention_scratch_bytes(const AttnLaunch& L) {
  if (!attn_dma_ok(L) || !attn_ring_path(L)) return 0;
  const size_t tp = (L.tokens + ATT_BN - 1) / ATT_BN * ATT_BN;
  return (size_t)L.kv_heads * 128 * tp * 2;
}

hipError_t attention_launch(const AttnLaunch& L, hipStream_t s) {
  if (L.tokens == 0 || L.heads == 0) return hipSuccess;
  AttnArgs a;
  a.q = L.q;
  a.k = L.k;
  a.v = L.v;
  a.o = L.out;
  a.tokens = L.tokens;
  a.heads = L.heads;
  a.group = L.heads / L.kv_heads;
  a.dim = L.dim;
  a.qs = L.q_stride;
  a.ks = L.k_stride;
  a.vs = L.v_stride;
  a.os = L.out_stride;
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)L.dim);
  a.causal = L.causal;
  if (attn_dma_ok(L)) {
    a.nqb = (L.tokens + DMA_BM - 1) / DMA_BM;
    const dim3 grid(a.nqb * L.heads);
    if (attn_ring_path(L)) {
      // the ring kernel: V^T pre-pass into scratch, then the one-phase DMA ring
      if (!L.scratch) return hipErrorInvalidValue;
      const uint32_t tp = (L.tokens + ATT_BN - 1) / ATT_BN * ATT_BN;
      uint16_t* vt = (uint16_t*)L.scratch;
      hipLaunchKernelGGL(attn_vt_kernel, dim3(tp / 64, L.kv_heads), dim3(256), 0, s, (const uint16_t*)L.v, L.v_stride,
                         L.tokens, tp, vt);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      if (L.dtype == F16) hipLaunchKernelGGL((attn_dma_kernel<true, 1>), grid, dim3(512), 0, s, a, (const uint16_t*)vt, tp, L.kv_heads);
      else hipLaunchKernelGGL((attn_dma_kernel<false, 1>), grid, dim3(512), 0, s, a, (const uint16_t*)vt, tp, L.kv_heads);
    } else if (L.path == 3) {  // the ping-pong kernel on 16x16x32 MFMAs
      const auto kern = L.dtype == F16 ? (L.causal ? attn_pp16_kernel<true, true> : attn_pp16_kernel<true, false>)
                                       : (L.causal ? attn_pp16_kernel<false, true> : attn_pp16_kernel<false, false>);
      hipLaunchKernelGGL(kern, grid, dim3(512), 0, s, a, L.kv_heads);
    } else {
      const auto kern = L.dtype == F16 ? (L.causal ? attn_pp_kernel<true, true> : attn_pp_kernel<true, false>)
                                       : (L.causal ? attn_pp_kernel<false, true> : attn_pp_kernel<false, false>);
      hipLaunchKernelGGL(kern, grid, dim3(512), 0, s, a, L.kv_heads);
    }
    return hipGetLastError();
  }
  a.nqb = (L.tokens + ATT_BM - 1) / ATT_BM;
  const int dp = L.dim <= 32 ? 32 : L.dim <= 64 ? 64 : 128;
  switch (L.dtype) {
    case BF16:
      return dp == 32 ? launch_attn(attn16_kernel<32, false>, a, s)
                      : dp == 64 ? launch_attn(attn16_kernel<64, false>, a, s) : launch_attn(attn16_kernel<128, false>, a, s);
    case F16:
      return dp == 32 ? launch_attn(attn16_kernel<32, true>, a, s)
                      : dp == 64 ? launch_attn(attn16_kernel<64, true>, a, s) : launch_attn(attn16_kernel<128, true>, a, s);
    default:
      return dp == 32 ? launch_attn(attn32_kernel<32>, a, s)
                      : dp == 64 ? launch_attn(attn32_kernel<64>, a, s) : launch_attn(attn32_kernel<128>, a, s);
  }
}

}  // namespace we
