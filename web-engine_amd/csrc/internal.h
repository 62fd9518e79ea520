// Internal interface between the C-ABI runtime (runtime.cpp) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define WE_EPI_ACCUMULATE_BIT 1u
#define WE_EPI_SPLIT_K_BIT 2u
#define WE_EPI_BIAS_BIT 4u
#define WE_EPI_GELU_BIT 8u

namespace we {

enum GemmCfgId {
  GEMM_CFG_256x256 = 0,
  GEMM_CFG_256x128 = 1,
  GEMM_CFG_128x128 = 2,
  GEMM_CFG_64x64 = 3,
  GEMM_CFG_32x64 = 4,
  GEMM_CFG_256x192 = 5
};

// Kernel-choice switches of a context (we_set_tuning): the context reads the WE_* environment variables once, when
// it is created, and every launch takes the values from here. Keys and meanings as WE_TUNE_* of we.h.
struct Tuning {
  int gemm_cfg = -1;        // GemmCfgId, -1: pick by shape
  int gemm_generic = 0;     // 1: the general GEMM kernel only
  int gemm_splitk = -1;     // -1: split-K plan by shape, 0: off, n > 0: n slices
  int gemm_reduce_xcd = 1;  // 1: the split-K reduce reads each tile on its XCD where that pays, 0: never
  int attn_path = 0;        // 0: default kernel, 1: register-staged kernel, 2: DMA ring with the V^T pre-pass,
                            // 3: ping-pong kernel on 16x16x32 MFMAs
  int int4_path = 0;        // 0: by shape, 1: general kernel, 2: shared-x kernel, 3: LDS-ring decode kernel
};
Tuning tuning_from_env();

struct GemmLaunch {
  const void* x;
  const void* w;
  void* y;
  const float* bias;
  // gated residual (gatedAdd fused): y = res + gate[col] * v, v the value after scale / bias / GELU; res has
  // y's type and layout (it may be y itself). gate NULL: off. res NULL with a gate: y = gate * v (or y +=
  // gate * v under ACCUMULATE).
  const float* gate;
  const void* res;
  // product with a second operand of y's type and layout (res names it; gate NULL, no accumulate):
  // 0 none, 1: y = silu(res) * v (swiglu with this GEMM as `up`), 2: y = res * sigmoid(v) (sigmoidGate with this
  // GEMM as `gate`); v the value after scale and bias
  int mul;
  // fused q/k path of attention (GemmLaunch::qk_cols > 0): columns [0, qk_cols) are heads of 128 values, q heads
  // below q_cols (norm weight qk_norm_q) and k heads above (qk_norm_k); each head is RMS-normalized (qk_eps,
  // qk_offset) and, on rows >= qk_rope_from (when qk_cos is set), rotated with interleaved pairs, cos / sin row
  // = row - qk_rope_from ([., 64] f32)
  uint32_t qk_cols, q_cols, qk_rope_from;
  float qk_eps, qk_offset;
  const float* qk_norm_q;
  const float* qk_norm_k;
  const float* qk_cos;
  const float* qk_sin;
  // 3x3 convolution input (conv_width > 0, the general kernel only): x is a channel-last image
  // [m / conv_width, conv_width, conv_cin] and k runs over (tap, channel), K = 9 * conv_cin
  uint32_t conv_width, conv_cin;
  int x_dtype, w_dtype, y_dtype;
  uint32_t m, n, k;
  float scale;
  uint32_t x_stride, w_stride, y_stride, x_offset, w_offset, y_offset;
  uint32_t splits, kc;
  uint32_t flags;
  int cfg;         // -1: pick by shape
  int generic;     // 1: skip the fast path (tests of the general kernel)
  int reduce_xcd;  // Tuning::gemm_reduce_xcd
  // 0, or the weights' K when x holds k / k_wrap planes of k_wrap values per row (f32 activations split into bf16
  // planes): k runs over all planes and the weights are read at k mod k_wrap. Fast path only (k_wrap % 64 == 0).
  uint32_t k_wrap;
  // split-K for small M: K in rsplits slices of rkc, partial sums in scratch (rsplits * m * n f32), then a
  // reduce pass that runs the epilogue; rcfg: the tile configuration the slices were sized for (-1: by shape)
  uint32_t rsplits, rkc;
  int rcfg;
  void* scratch;
};
hipError_t gemm_launch(const GemmLaunch& L, hipStream_t stream);
// Two GEMMs of one N, K, types and epilogue as one launch of the fast kernels (both through the fast path, full K);
// gemm_pair_ok says whether a pair qualifies, gemm_fast_launch_pair refuses others with hipErrorNotSupported.
bool gemm_pair_ok(const GemmLaunch& A, const GemmLaunch& B);
hipError_t gemm_fast_launch_pair(const GemmLaunch& A, const GemmLaunch& B, hipStream_t stream);

// The split-K plan of a launch on the fast path: rsplits > 1 when the output tiles alone would leave most
// CUs idle (small M); the scratch it needs, in bytes.
struct GemmReducePlan {
  uint32_t rsplits, rkc;
  size_t scratch_bytes;
  int rcfg;  // the tile configuration the slices are sized for, -1: the launch picks by shape
};
GemmReducePlan gemm_reduce_plan(const GemmLaunch& L, uint32_t force_splits = 0);  // force_splits: sweeps
// The straight-line fast path; hipErrorNotSupported when the operands do not qualify.
hipError_t gemm_fast_launch(const GemmLaunch& L, hipStream_t stream);
// Would gemm_fast_launch take this launch (types, alignment, extents)? (Not for split-K partial modes.)
bool gemm_fast_supported(const GemmLaunch& L);
int pick_gemm_cfg(uint32_t m, uint32_t n, uint32_t splits);

struct Int4Launch {
  const void* x;
  const uint32_t* w;
  const uint16_t* scales;
  void* y;
  const float* bias;
  const float* gate;  // as GemmLaunch
  const void* res;
  int x_dtype, y_dtype;
  uint32_t m, n, k, group;
  float scale;
  uint32_t x_stride, y_stride, x_offset, y_offset;
  uint32_t flags;
  int path;  // Tuning::int4_path
};
hipError_t int4_launch(const Int4Launch& L, hipStream_t stream);

// peak probes (peak.hip): kinds as WE_PEAK_* of we.h
enum PeakKind { PEAK_F32 = 0, PEAK_F16 = 1, PEAK_I8 = 2, PEAK_MFMA_BF16 = 3, PEAK_MFMA_BF16_DATA = 4 };
constexpr int READ_PEAK_U = 8;  // 16-byte chunks per thread of the streaming read: one u32 out per 32 KB / 4 waves
inline uint64_t read_peak_out_words(uint64_t bytes) { return 4 * ((bytes / 16 + 256 * READ_PEAK_U - 1) / (256 * READ_PEAK_U)); }
hipError_t peak_launch(int kind, uint32_t workgroups, uint32_t iters, uint32_t* out, hipStream_t stream);
hipError_t read_peak_launch(const void* buf, uint64_t bytes, uint32_t* out, hipStream_t stream);

struct AttnLaunch {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int dtype;  // F32, F16 or BF16 for q, k, v and out
  uint32_t tokens, heads, kv_heads, dim;
  uint32_t q_stride, k_stride, v_stride, out_stride;  // elements between consecutive tokens
  int causal;
  int path;       // Tuning::attn_path
  void* scratch;  // attention_scratch_bytes(L) bytes, or null (the register-staged kernel)
};
// Scratch the fast path needs (V^T of a head dim 128, 16-bit attention), 0 when it does not apply.
size_t attention_scratch_bytes(const AttnLaunch& L);
hipError_t attention_launch(const AttnLaunch& L, hipStream_t stream);

// Scratch of the allocation-free entry point (noalloc.hip): a file-scope device array of this many bytes per GPU.
// It holds the split-K partial sums of we_matmul_noalloc (at most about 10 MB for any M <= 64).
constexpr size_t kNoallocScratchBytes = 16u << 20;
// Looks up the array's address on `device`, which must be current; once per device (later calls return at once).
hipError_t noalloc_scratch_init(int device);
// The address noalloc_scratch_init found on `device`, or null before it succeeded.
void* noalloc_scratch(int device);
// The array of `device` belongs to one context at a time: claim returns true when it was free (it is then
// `owner`'s) or already `owner`'s; release frees it if `owner` holds it (context destruction).
bool noalloc_claim(int device, const void* owner);
void noalloc_release(int device, const void* owner);

// Can gemm_fast_launch run this GEMM with the fused q/k epilogue (fast path, a head-aligned tile chosen, no
// split-K plan)? qk_cols / q_cols must be set in L.
bool gemm_qk_fusable(const GemmLaunch& L);

hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);
hipError_t launch_fill(void* p, size_t bytes, uint8_t byte, hipStream_t s);
hipError_t launch_unpack_fp8(const void* packed, size_t n, const float* scale, float* out, hipStream_t s);
// f32 rows [m, k] (x_stride floats apart, 16-byte aligned, k % 8 == 0) -> bf16 [m, 3k]: planes hi | mid | lo along k,
// whose sum is each value exactly
hipError_t launch_split_f32_planes(const float* x, uint32_t m, uint32_t k, uint32_t x_stride, uint16_t* out,
                                   hipStream_t s);
hipError_t launch_dequant_int4(const uint32_t* w, const uint16_t* sc, uint32_t rows, uint32_t k, uint32_t group,
                               float* out, hipStream_t s);
hipError_t launch_elementwise(int op, size_t n, size_t d, int dtype, const void* a, const void* b, const void* c,
                              void* out, hipStream_t s);
hipError_t launch_layer_sum(uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w, float* out,
                            hipStream_t s);
hipError_t launch_rmsnorm(uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                          const float* weight, const float* scale, const float* shift, void* out, hipStream_t s);
hipError_t launch_rmsnorm_mod(uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                              const float* weight, const float* tvec, const float* table, uint32_t mod_n, float* mod,
                              void* out, hipStream_t s);
hipError_t launch_rope(uint32_t tokens, uint32_t heads, uint32_t pairs, int half, int dtype, const void* x,
                       const float* c, const float* sn, void* out, hipStream_t s);
hipError_t launch_qk_norm_rope(uint32_t tokens, uint32_t heads, uint32_t head_dim, float eps, float offset,
                               const float* weight, uint32_t rope_from, int half, const float* c, const float* sn,
                               int dtype, const void* x, uint32_t x_stride, void* out, uint32_t out_stride,
                               hipStream_t s);

}  // namespace we
