// Device-side helpers shared by the gfx950 kernels: vector types, 16-bit float conversions, the fp8 and
// int4 decoders, and MFMA wrappers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace we {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

enum DType { F32 = 0, F16 = 1, BF16 = 2, FP8 = 3, INT4 = 4 };

// 16-bit float storage types (raw bits in memory)
struct bf16_t { uint16_t v; };
struct f16_t { uint16_t v; };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// two f32 -> two 16-bit values in one word (lo in bits 0-15), round to nearest even; one
// v_cvt_pk_bf16_f32 for bf16
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float lo, float hi, std::true_type /*f16*/) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi, std::false_type /*bf16*/) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}

// Load / store one value of a storage type as f32.
template <int DT> __device__ __forceinline__ float load_as_f32(const void* p, size_t i);
template <> __device__ __forceinline__ float load_as_f32<F32>(const void* p, size_t i) { return ((const float*)p)[i]; }
template <> __device__ __forceinline__ float load_as_f32<F16>(const void* p, size_t i) {
  return f16_to_f32(((const uint16_t*)p)[i]);
}
template <> __device__ __forceinline__ float load_as_f32<BF16>(const void* p, size_t i) {
  return bf16_to_f32(((const uint16_t*)p)[i]);
}
template <int DT> __device__ __forceinline__ void store_from_f32(void* p, size_t i, float v);
template <> __device__ __forceinline__ void store_from_f32<F32>(void* p, size_t i, float v) { ((float*)p)[i] = v; }
template <> __device__ __forceinline__ void store_from_f32<F16>(void* p, size_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_f16(v);
}
template <> __device__ __forceinline__ void store_from_f32<BF16>(void* p, size_t i, float v) {
  ((uint16_t*)p)[i] = f32_to_bf16(v);
}

// e4m3fn -> f32 exactly as the reference shader does (src/kernels/fp8.ts:12-20): exponent rebias,
// subnormals as m * 2^-9, sign last, no NaN branch (0x7f -> 480).
__device__ __forceinline__ float e4m3_shader(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
  const float normal = __uint_as_float(((e + 120u) << 23) | (m << 20));
  const float sub = (float)m * 0.001953125f;
  const float v = e == 0u ? sub : normal;
  return (b & 0x80u) ? -v : v;
}

// Four fp8 bytes of one word -> four 16-bit values (two packed words). The hardware converter decodes
// OCP e4m3fn and turns the two NaN codes into NaN; the reference shader turns them into +-480, so words
// holding a NaN code take a slow path that writes +-480 (0x43f0 bf16 / 0x5f80 f16) for those bytes.
__device__ __forceinline__ bool has_nan_code(uint32_t w) {
  return (((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u) != 0u;
}
template <bool IS_F16>
__device__ __forceinline__ u32x2 fp8x4_to_16(uint32_t w) {
  u32x2 r;
  if constexpr (IS_F16) {
    f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
    f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true);
    r.x = __builtin_bit_cast(uint32_t, lo);
    r.y = __builtin_bit_cast(uint32_t, hi);
  } else {
    bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    r.x = __builtin_bit_cast(uint32_t, lo);
    r.y = __builtin_bit_cast(uint32_t, hi);
  }
  if (__builtin_expect(has_nan_code(w), 0)) {
    const uint32_t big = IS_F16 ? 0x5f80u : 0x43f0u;
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t b = (w >> (8 * i)) & 0xffu;
      const uint32_t cur = ((i < 2 ? r.x : r.y) >> (16 * (i & 1))) & 0xffffu;
      h[i] = ((b & 0x7fu) == 0x7fu) ? (big | ((b & 0x80u) << 8)) : cur;
    }
    r.x = h[0] | (h[1] << 16);
    r.y = h[2] | (h[3] << 16);
  }
  return r;
}

// MFMA 32x32x16 with bf16 or f16 operands (8 values per lane, as 4 dwords), fp32 accumulators.
template <bool IS_F16>
__device__ __forceinline__ f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (IS_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                   0);
}

// MFMA 16x16x32 with bf16 or f16 operands (8 values per lane, as 4 dwords), fp32 accumulators. The same work as
// two 32x32x16 steps of a quarter of the tile; measured on MI355X at the power limit, on random operands with the
// fp8-weight GEMM's bit statistics, it sustains 1.90-1.93 PFLOP/s against 1.73 for 32x32x16 (zero operands: 2.44
// both): it moves half the accumulator bits per multiply-add.
template <bool IS_F16>
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (IS_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                   0);
}

// Compile-time loop: f(std::integral_constant<int, I>{}) for I in [B, E). Unlike #pragma unroll it cannot
// be refused by the optimizer, so register arrays indexed inside stay in registers.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// PyTorch tanh GELU in the reference's form (src/kernels/elementwise.ts:25-29).
// GELU, tanh form (src/kernels/elementwise.ts:25-29): 0.5 v (1 + tanh u) with u = sqrt(2/pi) (v + 0.044715 v^3),
// evaluated as v / (1 + e^(-2u)) (the same function: (1 + tanh u) / 2 = 1 / (1 + e^(-2u))). The exponential is
// v_exp_f32 (2^x, log2 e folded into the constant) and the reciprocal v_rcp_f32, both within about 1 ulp:
// 5 VALU ops and 2 transcendentals, no division. It saturates without a clamp: e -> 0 gives v, e -> inf
// gives -0.
__device__ __forceinline__ float gelu_tanh(float v) {
  constexpr float c = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
  const float p = __builtin_fmaf(v * v, 0.044715f * c, c);                // c (1 + 0.044715 v^2)
  const float e = __builtin_amdgcn_exp2f(v * p);                         // e^(-2u)
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float sigmoid(float v) { return 1.0f / (1.0f + __expf(-v)); }

// The product epilogues (GemmLaunch::mul): 1 swiglu (src/kernels/elementwise.ts:38-43) with the GEMM value as
// `up` and aux as `gate`: (aux * sigmoid(aux)) * v; 2 sigmoidGate (:45-50) with the GEMM value as `gate`:
// aux * sigmoid(v).
__device__ __forceinline__ float mul_epilogue(uint32_t mul, float aux, float v) {
  return mul == 1u ? aux * sigmoid(aux) * v : aux * sigmoid(v);
}

typedef __attribute__((address_space(3))) void lds_ptr_t;

// 16-byte direct-to-LDS buffer load issued as inline asm: lane i writes dst + 16 i. The compiler does not
// see it, so it adds no waits of its own for the LDS it fills (it otherwise waits for every such load in
// flight before any LDS read it cannot tell apart); the kernels that use it wait with explicit vmcnt
// counts. The compiler's waits for its own register loads stay correct: it can only undercount the loads
// in flight after one, which makes a wait stricter. M0 is set here; nothing else in those kernels reads it.
__device__ __forceinline__ void dma16(const __amdgpu_buffer_rsrc_t& r, void* dst, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"((uint32_t)(uintptr_t)(lds_ptr_t*)dst), "v"(voff), "s"(r)
               : "memory");
}

}  // namespace we
