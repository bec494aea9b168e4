// The decoder-layer pieces around attention for gfx950: the rest of one
// Qwen3 layer (crates/cev-model/src/qwen3.rs:223-262) and of the packed
// forward (qwen3.rs:346-401), each in candle's op order with every op rounded
// to the model dtype:
//   rms_norm      y = dtype(dtype(x / dtype(sqrt(sum x^2 / H + eps))) * w)
//                 (candle_nn RmsNorm: input_layernorm, post_attention_layernorm,
//                 the final norm), the sum of squares in element order;
//   add_rms_norm  x' = dtype(x + h), y = rms_norm(x') (the residual adds of
//                 qwen3.rs:261, :358 and :397 fused with the norm that follows);
//   swiglu        a = dtype(silu(g) * u), silu(v) = v / (1 + exp(-v)) with each
//                 op in the model dtype (Mlp::forward, qwen3.rs:230-233).
// The projections around them are plain GEMMs (the library's).
//
// Norm work split: a workgroup takes kNormRows rows.  Lanes 0..kNormRows-1
// of wave 0 each sum one row's squares in element order (the reference's
// sequential f32 sum, bit for bit); then all 256 threads normalise the rows
// with coalesced 16-byte accesses.
#include "cev_device.h"
#include "cev_internal.h"

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormRows = 16;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct NormArgs {
  const void* x;
  const void* h;  // nullptr: plain norm
  void* x_out;    // x + h (may alias x)
  const void* w;
  void* y;
  int64_t rows, x_st, h_st, xo_st, y_st;
  int32_t hidden, plus_one;
  float eps;
};

template <typename T>
__device__ __forceinline__ float elem(const u32x4& c, int j) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w = c[j >> 1];
    return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(c[j]);
  }
}

// Packs VEC rounded values into one 16-byte chunk.
template <typename T>
__device__ __forceinline__ u32x4 pack(const float* v) {
  u32x4 c;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const __bf16 lo = (__bf16)v[2 * i], hi = (__bf16)v[2 * i + 1];
      c[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = __float_as_uint(v[i]);
  }
  return c;
}

template <typename T>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int VEC = 16 / (int)sizeof(T);
  auto rnd = [](float v) { return BF ? bf16_round(v) : v; };
  __shared__ float msh[kNormRows];
  const int64_t r0 = (int64_t)blockIdx.x * kNormRows;
  const int nrows = (int)min<int64_t>(kNormRows, a.rows - r0);
  const int nc = a.hidden / VEC;
  const int tid = threadIdx.x;

  if (tid < nrows) {
    const int64_t r = r0 + tid;
    const T* xr = (const T*)a.x + r * a.x_st;
    const T* hr = a.h ? (const T*)a.h + r * a.h_st : nullptr;
    float s = 0.0f;
#pragma unroll 4
    for (int k = 0; k < nc; ++k) {
      const u32x4 cx = *(const u32x4*)(xr + k * VEC);
      u32x4 ch = {};
      if (hr) ch = *(const u32x4*)(hr + k * VEC);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float v = hr ? rnd(elem<T>(cx, j) + elem<T>(ch, j)) : elem<T>(cx, j);
        s += v * v;
      }
    }
    msh[tid] = rnd(sqrtf(s / (float)a.hidden + a.eps));
  }
  __syncthreads();

  for (int i = tid; i < nrows * nc; i += kNormThreads) {
    const int rr = i / nc, k = i % nc;
    const int64_t r = r0 + rr;
    const float m = msh[rr];
    const u32x4 cx = *(const u32x4*)((const T*)a.x + r * a.x_st + k * VEC);
    const u32x4 cw = *(const u32x4*)((const T*)a.w + k * VEC);
    float xs[VEC], ys[VEC];
    if (a.h) {
      const u32x4 ch = *(const u32x4*)((const T*)a.h + r * a.h_st + k * VEC);
#pragma unroll
      for (int j = 0; j < VEC; ++j) xs[j] = rnd(elem<T>(cx, j) + elem<T>(ch, j));
      *(u32x4*)((T*)a.x_out + r * a.xo_st + k * VEC) = pack<T>(xs);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) xs[j] = elem<T>(cx, j);
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      float w = elem<T>(cw, j);
      if (a.plus_one) w = rnd(w + 1.0f);
      ys[j] = rnd(rnd(xs[j] / m) * w);
    }
    *(u32x4*)((T*)a.y + r * a.y_st + k * VEC) = pack<T>(ys);
  }
}

struct SwigluArgs {
  const void* g;
  const void* u;
  void* out;
  int64_t rows, in_st, out_st;
  int32_t inter;
};

template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(SwigluArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int VEC = 16 / (int)sizeof(T);
  auto rnd = [](float v) { return BF ? bf16_round(v) : v; };
  const int nc = a.inter / VEC;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.rows * nc) return;
  const int64_t r = i / nc;
  const int k = (int)(i % nc);
  const u32x4 cg = *(const u32x4*)((const T*)a.g + r * a.in_st + k * VEC);
  const u32x4 cu = *(const u32x4*)((const T*)a.u + r * a.in_st + k * VEC);
  float o[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const float v = elem<T>(cg, j);
    float s;
    if constexpr (BF) {
      const float e = rnd(expf(-v));
      const float den = rnd(1.0f + e);
      s = rnd(v / den);
    } else {
      s = v / (1.0f + expf(-v));
    }
    o[j] = rnd(s * elem<T>(cu, j));
  }
  *(u32x4*)((T*)a.out + r * a.out_st + k * VEC) = pack<T>(o);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int32_t cev_rms_norm(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h,
                                int64_t h_stride, void* x_out, int64_t x_out_stride, const void* w, float eps, int32_t weight_plus_one,
                                void* y, int64_t y_stride, cev_stream stream) {
  if (dtype != CEV_F32 && dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_rms_norm: dtype %d", dtype);
  const int vec = dtype == CEV_BF16 ? 8 : 4;
  CEV_CHECK_ARG(rows >= 0 && hidden > 0 && hidden % vec == 0, "cev_rms_norm: hidden %d must be a positive multiple of %d", hidden, vec);
  CEV_CHECK_ARG(eps >= 0.0f, "cev_rms_norm: negative eps");
  if (rows == 0) return CEV_OK;
  CEV_CHECK_ARG(x && w && y && (!h || x_out), "cev_rms_norm: null buffer");
  CEV_CHECK_ARG(aligned16(x) && aligned16(w) && aligned16(y) && (!h || (aligned16(h) && aligned16(x_out))),
                "cev_rms_norm: buffers must be 16-byte aligned");
  CEV_CHECK_ARG(x_stride >= hidden && y_stride >= hidden && x_stride % vec == 0 && y_stride % vec == 0 &&
                    (!h || (h_stride >= hidden && x_out_stride >= hidden && h_stride % vec == 0 && x_out_stride % vec == 0)),
                "cev_rms_norm: row strides must cover a row and keep rows 16-byte aligned");
  NormArgs a{x, h, x_out, w, y, rows, x_stride, h_stride, x_out_stride, y_stride, hidden, weight_plus_one, eps};
  const int64_t grid = (rows + kNormRows - 1) / kNormRows;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_rms_norm: too many rows");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CEV_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<uint16_t>, dim3((unsigned)grid), dim3(kNormThreads), 0, s, a);
  else
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)grid), dim3(kNormThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_rms_norm launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

extern "C" int32_t cev_swiglu(int32_t dtype, int64_t rows, int32_t inter, const void* gate, const void* up, int64_t in_stride, void* out,
                              int64_t out_stride, cev_stream stream) {
  if (dtype != CEV_F32 && dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_swiglu: dtype %d", dtype);
  const int vec = dtype == CEV_BF16 ? 8 : 4;
  CEV_CHECK_ARG(rows >= 0 && inter > 0 && inter % vec == 0, "cev_swiglu: inter %d must be a positive multiple of %d", inter, vec);
  if (rows == 0) return CEV_OK;
  CEV_CHECK_ARG(gate && up && out, "cev_swiglu: null buffer");
  CEV_CHECK_ARG(aligned16(gate) && aligned16(up) && aligned16(out), "cev_swiglu: buffers must be 16-byte aligned");
  CEV_CHECK_ARG(in_stride >= inter && out_stride >= inter && in_stride % vec == 0 && out_stride % vec == 0,
                "cev_swiglu: row strides must cover a row and keep rows 16-byte aligned");
  SwigluArgs a{gate, up, out, rows, in_stride, out_stride, inter};
  const int64_t n = rows * (inter / vec);
  const int64_t grid = (n + 255) / 256;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_swiglu: too many rows");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CEV_BF16)
    hipLaunchKernelGGL(swiglu_kernel<uint16_t>, dim3((unsigned)grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3((unsigned)grid), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_swiglu launch: %s", hipGetErrorString(e));
  return CEV_OK;
}
