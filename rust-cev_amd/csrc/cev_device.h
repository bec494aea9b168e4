// Device-side helpers for the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Round-to-nearest-even f32 -> bf16 -> f32 (the value the model dtype holds):
// v_cvt_pk_bf16_f32 (RNE, denormals kept under the kernels' f32 denorm
// mode) and a shift back.
__device__ __forceinline__ float bf16_round(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ uint16_t bf16_bits(float x) {
  return (uint16_t)(__float_as_uint(bf16_round(x)) >> 16);
}

__device__ __forceinline__ float bf16_from_bits(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Exchange a value with the lane 32 away (the other half of a wave64).
__device__ __forceinline__ float swap_half(float x) { return __shfl_xor(x, 32, 64); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A value moved across lanes by a DPP control (row-local permutes such as
// quad_perm 0x4E = lane ^ 2); every lane of the row must be active.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kCtrl, 0xF, 0xF, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __uint_as_float(dpp_u<kCtrl>(__float_as_uint(v)));
}

// Orders this wave's LDS writes before its later LDS reads by other lanes of
// the same wave (no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The bf16 SiLU of a bf16 value, v / (1 + e^-v) with each op rounded to
// bf16, depends on its 16 bits only.  Kernels that apply it to many values
// tabulate it in LDS for |v| in [2^-16, 2^7) (23 binades of 128 mantissas
// per sign), evaluated by the same silu_bf16, so a table hit is
// bit-identical to evaluating it; values outside take silu_bf16 itself.
// (The translation units that use it are built without FMA contraction.)
constexpr uint32_t kSiluLo = (127 - 16) * 128;  // |bits| of 2^-16
constexpr uint32_t kSiluSpan = 23 * 128;        // entries per sign
constexpr int kSiluEntries = 2 * (int)kSiluSpan;

__device__ __forceinline__ float silu_bf16(float v) {
  const float ex = bf16_round(expf(-v));
  const float den = bf16_round(1.0f + ex);
  return bf16_round(v / den);
}

// table slot of a bf16-exact value: negative values after the positive ones;
// >= kSiluEntries when |v| is outside the table
__device__ __forceinline__ uint32_t silu_slot(float v) {
  const uint32_t b = __float_as_uint(v) >> 16;
  const uint32_t m = (b & 0x7fffu) - kSiluLo;
  return m < kSiluSpan ? m + (b >> 15) * kSiluSpan : (uint32_t)kSiluEntries;
}

// Every thread of a workgroup of `threads` fills its share of the table.
__device__ __forceinline__ void silu_fill(float* tab, int threads) {
  for (int i = threadIdx.x; i < kSiluEntries; i += threads) {
    const uint32_t neg = i >= (int)kSiluSpan;
    const uint32_t bits = (neg << 15) | (kSiluLo + (uint32_t)i - neg * kSiluSpan);
    tab[i] = silu_bf16(bf16_from_bits((uint16_t)bits));
  }
}

template <typename Fn, int... I>
__device__ __forceinline__ void static_for_impl(Fn&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, 0>), ..., f(integral_constant<int, N-1>).
template <int N, typename Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
