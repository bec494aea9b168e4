// Fused QK RMSNorm + RoPE with per-token positions for gfx950: the prologue
// of Attention::forward, crates/cev-model/src/qwen3.rs:193-196 (weight w,
// full rotary) and crates/cev-model/src/qwen35.rs:529-539 (weight 1 + w,
// partial rotary, q read out of the [q | gate] head layout).
//
// The op order is the reference's (candle_nn::ops::rms_norm then
// candle_nn::rotary_emb::rope), each op rounded to the model dtype:
//   sum2 = sum_e x_e^2  (f32, left to right)
//   m    = dtype(sqrt(sum2 / D + eps))
//   y_e  = dtype(dtype(x_e / m) * w_e)
//   rope: y_i = dtype(dtype(y_i c) - dtype(y_{i+h} s)), y_{i+h} = dtype(dtype(y_i s) + dtype(y_{i+h} c))
// This file is compiled with -ffp-contract=off so no product is fused into
// an add, as in the reference.  Plain `/` and sqrtf are the correctly
// rounded HIP forms (hipcc's default); __fsqrt_rn is not (it maps to the
// native approximate square root) and must not be used here.
//
// Work split: a wave normalises 8 vectors (token, head) at a time.  Lanes
// load the 8 x D elements coalesced, the squares go through LDS and lanes
// 0..7 each sum one vector in element order, so the sum matches the
// reference's sequential f32 sum bit for bit.
#include "cev_device.h"
#include "cev_internal.h"

namespace {

struct QkArgs {
  const void* q_in;
  const void* k_in;
  const void* w_q;
  const void* w_k;
  const int32_t* pos;
  const void* cos_t;
  const void* sin_t;
  void* q_out;
  void* k_out;
  int64_t qi_st, qi_sh, ki_st, ki_sh, qo_st, qo_sh, ko_st, ko_sh;
  int32_t t, hq, hkv, rot, n_pos, plus_one;
  float eps;
};

constexpr int VPW = 8;    // vectors per wave
constexpr int WAVES = 4;  // waves per workgroup

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_from_bits(p[i]);
}

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ __forceinline__ void st<uint16_t>(uint16_t* p, int64_t i, float v) {
  p[i] = bf16_bits(v);
}

template <typename T, int D>
__global__ __launch_bounds__(WAVES * 64) void qknorm_rope_kernel(QkArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int EPL = D / 64;  // elements per lane per vector
  __shared__ float buf[WAVES][VPW][D];
  __shared__ float msh[WAVES][VPW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nq = (int64_t)a.t * a.hq;
  const int64_t total = nq + (int64_t)a.t * a.hkv;
  const int64_t v0 = ((int64_t)blockIdx.x * WAVES + wave) * VPW;
  auto rnd = [](float x) { return BF ? bf16_round(x) : x; };

  float x[VPW][EPL];
  const T* src[VPW];
  T* dst[VPW];
  const T* wgt[VPW];
  int tok[VPW];
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const int64_t v = v0 + j;
    src[j] = nullptr;
    dst[j] = nullptr;
    wgt[j] = nullptr;
    tok[j] = 0;
    if (v < nq) {
      const int tk = (int)(v / a.hq), h = (int)(v % a.hq);
      src[j] = (const T*)a.q_in + tk * a.qi_st + h * a.qi_sh;
      dst[j] = (T*)a.q_out + tk * a.qo_st + h * a.qo_sh;
      wgt[j] = (const T*)a.w_q;
      tok[j] = tk;
    } else if (v < total) {
      const int64_t vk = v - nq;
      const int tk = (int)(vk / a.hkv), h = (int)(vk % a.hkv);
      src[j] = (const T*)a.k_in + tk * a.ki_st + h * a.ki_sh;
      dst[j] = (T*)a.k_out + tk * a.ko_st + h * a.ko_sh;
      wgt[j] = (const T*)a.w_k;
      tok[j] = tk;
    }
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int e = lane + 64 * k;
      x[j][k] = src[j] ? ld<T>(src[j], e) : 0.0f;
      buf[wave][j][e] = x[j][k] * x[j][k];
    }
  }
  __syncthreads();
  if (lane < VPW) {
    float s = 0.0f;
    for (int e = 0; e < D; ++e) s += buf[wave][lane][e];
    msh[wave][lane] = rnd(sqrtf(s / (float)D + a.eps));
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    const float m = msh[wave][j];
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int e = lane + 64 * k;
      float w = wgt[j] ? ld<T>(wgt[j], e) : 0.0f;
      if (a.plus_one) w = rnd(w + 1.0f);
      const float y = rnd(rnd(x[j][k] / m) * w);
      x[j][k] = y;
      buf[wave][j][e] = y;
    }
  }
  __syncthreads();
  const int half = a.rot / 2;
#pragma unroll
  for (int j = 0; j < VPW; ++j) {
    if (!dst[j]) continue;
    const int p = a.pos[tok[j]];
    const bool p_ok = p >= 0 && p < a.n_pos;
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int e = lane + 64 * k;
      float y = x[j][k];
      if (e < a.rot) {
        // A position outside the table yields NaN instead of a stray read.
        const int i = e < half ? e : e - half;
        const float c = p_ok ? ld<T>((const T*)a.cos_t, (int64_t)p * half + i) : __builtin_nanf("");
        const float s = p_ok ? ld<T>((const T*)a.sin_t, (int64_t)p * half + i) : __builtin_nanf("");
        if (e < half) {
          const float b = buf[wave][j][e + half];
          y = rnd(rnd(y * c) - rnd(b * s));
        } else {
          const float a1 = buf[wave][j][e - half];
          y = rnd(rnd(a1 * s) + rnd(y * c));
        }
      }
      st<T>(dst[j], e, y);
    }
  }
}

template <typename T>
int32_t launch_qk(const QkArgs& a, int d, hipStream_t s) {
  const int64_t vecs = (int64_t)a.t * (a.hq + a.hkv);
  const int64_t per_wg = (int64_t)WAVES * VPW;
  const int64_t grid = (vecs + per_wg - 1) / per_wg;
  if (grid == 0) return CEV_OK;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "qknorm grid too large");
  if (d == 128)
    hipLaunchKernelGGL((qknorm_rope_kernel<T, 128>), dim3((unsigned)grid), dim3(WAVES * 64), 0, s, a);
  else
    hipLaunchKernelGGL((qknorm_rope_kernel<T, 256>), dim3((unsigned)grid), dim3(WAVES * 64), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "qknorm_rope launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

}  // namespace

extern "C" int32_t cev_qknorm_rope(const cev_qknorm_desc* d, const void* q_in, const void* k_in, const void* w_q, const void* w_k,
                                   const int32_t* pos, const void* cos_t, const void* sin_t, void* q_out, void* k_out, cev_stream stream) {
  CEV_CHECK_ARG(d != nullptr, "cev_qknorm_rope: null descriptor");
  if (d->dtype != CEV_F32 && d->dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_qknorm_rope: dtype %d", d->dtype);
  if (d->head_dim != 128 && d->head_dim != 256) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_qknorm_rope: head_dim %d", d->head_dim);
  CEV_CHECK_ARG(d->t >= 0 && d->n_q_heads >= 0 && d->n_kv_heads >= 0, "cev_qknorm_rope: negative sizes");
  CEV_CHECK_ARG(d->rotary_dim >= 2 && d->rotary_dim % 2 == 0 && d->rotary_dim <= d->head_dim, "cev_qknorm_rope: rotary_dim %d",
                d->rotary_dim);
  CEV_CHECK_ARG(d->n_pos >= 1, "cev_qknorm_rope: empty cos/sin table");
  CEV_CHECK_ARG(d->eps >= 0.0f, "cev_qknorm_rope: negative eps");
  if (d->t == 0 || d->n_q_heads + d->n_kv_heads == 0) return CEV_OK;
  CEV_CHECK_ARG(pos && cos_t && sin_t, "cev_qknorm_rope: null pos or table");
  CEV_CHECK_ARG(d->n_q_heads == 0 || (q_in && q_out && w_q), "cev_qknorm_rope: null q buffers");
  CEV_CHECK_ARG(d->n_kv_heads == 0 || (k_in && k_out && w_k), "cev_qknorm_rope: null k buffers");
  QkArgs a;
  a.q_in = q_in;
  a.k_in = k_in;
  a.w_q = w_q;
  a.w_k = w_k;
  a.pos = pos;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.q_out = q_out;
  a.k_out = k_out;
  a.qi_st = d->qi_stride_t;
  a.qi_sh = d->qi_stride_h;
  a.ki_st = d->ki_stride_t;
  a.ki_sh = d->ki_stride_h;
  a.qo_st = d->qo_stride_t;
  a.qo_sh = d->qo_stride_h;
  a.ko_st = d->ko_stride_t;
  a.ko_sh = d->ko_stride_h;
  a.t = d->t;
  a.hq = d->n_q_heads;
  a.hkv = d->n_kv_heads;
  a.rot = d->rotary_dim;
  a.n_pos = d->n_pos;
  a.plus_one = d->weight_plus_one;
  a.eps = d->eps;
  hipStream_t s = (hipStream_t)stream;
  if (d->dtype == CEV_BF16) return launch_qk<uint16_t>(a, d->head_dim, s);
  return launch_qk<float>(a, d->head_dim, s);
}
