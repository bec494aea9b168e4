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

template <typename Fn, int... I>
__device__ __forceinline__ void static_for_impl(Fn&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, 0>), ..., f(integral_constant<int, N-1>).
template <int N, typename Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
