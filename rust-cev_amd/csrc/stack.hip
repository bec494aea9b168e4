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
// Two norm kernels.  rms_norm_wave_kernel (cev_rms_norm): one wave per row,
// each lane keeping its 16-byte chunks in registers; the sum of squares is
// each lane's partial sum in chunk order, then an xor-butterfly over the
// wave (tree order: every lane ends with the same bits).  It differs from
// the reference's sequential f32 sum only in the last bits of the sum.
// rms_norm_kernel (cev_rms_norm_seq) keeps the reference's element order
// bit for bit.
//
// Sequential-sum work split: a workgroup takes up to kNormRows rows.  All 1024 threads
// load them with coalesced 16-byte accesses (x + h for the fused residual,
// written back as they go), keep their chunks in registers and put the
// squares, as f32, in LDS; lanes 0..rows-1 of wave 0 then each add one row's
// squares in element order (the reference's sequential f32 sum, bit for bit:
// one dependent add per element), and every thread normalises its own
// chunks.  Rows of squares sit 16 bytes apart beyond their length, so the
// summing lanes' 16-byte reads fall on different banks.
//
// x / m is correctly rounded for every element.  With y = RN(1/m),
// q0 = RN(x y) and the exact residual r = x - q0 m, RN(q0 + r y) is the
// correctly rounded quotient (Markstein) while r can neither underflow nor
// overflow: every nonzero |x| in [2^-96, 2^60] (the sum of squares <= 2^120
// bounds the top) and m in [2^-20, 2^20].  A row outside that range takes
// the IEEE division; copysign keeps the sign of -0 / m.
#include <algorithm>
#include <type_traits>

#include "cev_device.h"
#include "cev_internal.h"

namespace {

constexpr int kNormThreads = 1024;
constexpr int kNormRows = 16;                   // rows per workgroup at most
constexpr int kNormLdsBytes = 132 * 1024;       // LDS for the rows' squares
constexpr int kNormChunks = 4;                  // 16-byte chunks each thread keeps in registers

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

// LDS pitch in bytes of one row of f32 squares.
__host__ __device__ inline int norm_pitch(int hidden) { return hidden * 4 + 16; }

template <typename T>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a, int rows_per_wg) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int VEC = 16 / (int)sizeof(T);
  auto rnd = [](float v) { return BF ? bf16_round(v) : v; };
  extern __shared__ __align__(16) char sq_lds[];
  __shared__ float msh[kNormRows], ysh[kNormRows];
  __shared__ int min_exp[kNormRows], fast_row[kNormRows];
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
  const int nrows = (int)min<int64_t>(rows_per_wg, a.rows - r0);
  const int nc = a.hidden / VEC;
  const int pitch = norm_pitch(a.hidden);
  const int tid = threadIdx.x;
  const int total = nrows * nc;  // <= kNormThreads * kNormChunks (launcher)
  if (tid < kNormRows) min_exp[tid] = 0;
  __syncthreads();

  // chunk b of this thread is i = tid + b * kNormThreads
  u32x4 cx[kNormChunks];
  {
    u32x4 ch[kNormChunks];
#pragma unroll
    for (int b = 0; b < kNormChunks; ++b) {
      const int i = tid + b * kNormThreads;
      if (i < total) {
        const int64_t r = r0 + i / nc;
        const int k = i % nc;
        cx[b] = *(const u32x4*)((const T*)a.x + r * a.x_st + k * VEC);
        if (a.h) ch[b] = *(const u32x4*)((const T*)a.h + r * a.h_st + k * VEC);
      }
    }
#pragma unroll
    for (int b = 0; b < kNormChunks; ++b) {
      const int i = tid + b * kNormThreads;
      if (i < total) {
        const int rr = i / nc, k = i % nc;
        float xs[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) xs[j] = a.h ? rnd(elem<T>(cx[b], j) + elem<T>(ch[b], j)) : elem<T>(cx[b], j);
        if (a.h) {
          cx[b] = pack<T>(xs);
          *(u32x4*)((T*)a.x_out + (r0 + rr) * a.xo_st + k * VEC) = cx[b];
        }
        int me = 0;
        float* sq = (float*)(sq_lds + rr * pitch) + k * VEC;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          sq[j] = xs[j] * xs[j];
          me = min(me, __builtin_amdgcn_frexp_expf(xs[j]));
        }
        if (me < 0) atomicMin(&min_exp[rr], me);
      }
    }
  }
  __syncthreads();

  if (tid < nrows) {
    const float* row = (const float*)(sq_lds + tid * pitch);
    float s = 0.0f;
#pragma unroll 8
    for (int k = 0; k < a.hidden / 4; ++k) {
      const f32x4 q = *(const f32x4*)(row + 4 * k);
      s += q[0];
      s += q[1];
      s += q[2];
      s += q[3];
    }
    const float m = rnd(sqrtf(s / (float)a.hidden + a.eps));
    msh[tid] = m;
    ysh[tid] = 1.0f / m;
    fast_row[tid] = min_exp[tid] >= -95 && s <= 0x1p120f && m >= 0x1p-20f && m <= 0x1p20f;
  }
  __syncthreads();

#pragma unroll
  for (int b = 0; b < kNormChunks; ++b) {
    const int i = tid + b * kNormThreads;
    if (i < total) {
      const int rr = i / nc, k = i % nc;
      const float m = msh[rr], y = ysh[rr];
      const bool fast = fast_row[rr];
      const u32x4 cw = *(const u32x4*)((const T*)a.w + k * VEC);
      float ys[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float x = elem<T>(cx[b], j);
        float q;
        if (fast) {
          const float q0 = x * y;
          q = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, m, x), y, q0), q0);
        } else {
          q = x / m;
        }
        float w = elem<T>(cw, j);
        if (a.plus_one) w = rnd(w + 1.0f);
        ys[j] = rnd(rnd(q) * w);
      }
      *(u32x4*)((T*)a.y + (r0 + rr) * a.y_st + k * VEC) = pack<T>(ys);
    }
  }
}

constexpr int kWaveNormRows = 4;  // rows (waves) per workgroup of the wave kernel

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// One wave per row, lane l holding chunks l, l + 64, ... (NCH at most).
// Every lane loads all NCH chunks of x, h and the weight at once (indices
// clamped to the row, so the loads are unconditional and all in flight
// together); chunks past the row are neither summed nor stored.  The
// residual is a template parameter and the division path is chosen once
// per row, so no branch sits inside the element loops.
template <typename T, int NCH, bool RES>
__global__ __launch_bounds__(kWaveNormRows * 64) void rms_norm_wave_kernel(NormArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int VEC = 16 / (int)sizeof(T);
  auto rnd = [](float v) { return BF ? bf16_round(v) : v; };
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kWaveNormRows + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  const int nc = a.hidden / VEC;
  u32x4 cx[NCH], ch[NCH], cw[NCH];
#pragma unroll
  for (int b = 0; b < NCH; ++b) {
    const int k = min(lane + 64 * b, nc - 1);
    cx[b] = *(const u32x4*)((const T*)a.x + r * a.x_st + k * VEC);
    if constexpr (RES) ch[b] = *(const u32x4*)((const T*)a.h + r * a.h_st + k * VEC);
    cw[b] = *(const u32x4*)((const T*)a.w + k * VEC);
  }
  float s = 0.0f;
  int me = 0;
#pragma unroll
  for (int b = 0; b < NCH; ++b) {
    const int k = lane + 64 * b;
    const bool in_row = k < nc;
    float xs[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) xs[j] = RES ? rnd(elem<T>(cx[b], j) + elem<T>(ch[b], j)) : elem<T>(cx[b], j);
    if constexpr (RES) {
      cx[b] = pack<T>(xs);
      if (in_row) *(u32x4*)((T*)a.x_out + r * a.xo_st + k * VEC) = cx[b];
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float sj = __builtin_fmaf(xs[j], xs[j], s);
      const int mj = min(me, __builtin_amdgcn_frexp_expf(xs[j]));
      s = in_row ? sj : s;
      me = in_row ? mj : me;
    }
  }
  s = wave_sum_f32(s);
  me = wave_min_i32(me);
  const float m = rnd(sqrtf(s / (float)a.hidden + a.eps));
  const float y = 1.0f / m;
  const bool fast = me >= -95 && s <= 0x1p120f && m >= 0x1p-20f && m <= 0x1p20f;
  auto norm_row = [&](auto fast_c) {
#pragma unroll
    for (int b = 0; b < NCH; ++b) {
      const int k = lane + 64 * b;
      float ys[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float x = elem<T>(cx[b], j);
        float q;
        if constexpr (decltype(fast_c)::value) {
          const float q0 = x * y;
          q = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, m, x), y, q0), q0);
        } else {
          q = x / m;
        }
        const float w0 = elem<T>(cw[b], j);
        const float w = a.plus_one ? rnd(w0 + 1.0f) : w0;
        ys[j] = rnd(rnd(q) * w);
      }
      if (k < nc) *(u32x4*)((T*)a.y + r * a.y_st + k * VEC) = pack<T>(ys);
    }
  };
  if (fast)
    norm_row(std::true_type{});
  else
    norm_row(std::false_type{});
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

// bf16 with the SiLU table: up to kSwigluBlocks workgroups, each filling
// the table once and then taking rows blockIdx.x, blockIdx.x + gridDim.x, ...;
// a thread loads kSwigluAhead chunks of g and u of a row (indices clamped to
// the row, so the loads are unconditional) before computing them.  A chunk
// slot whose gate values are not all in the table takes silu_bf16 for the
// whole wave.  Bit-identical to swiglu_kernel<bf16>.
constexpr int kSwigluThreads = 256;
constexpr int kSwigluAhead = 4;
constexpr int kSwigluBlocks = 1024;  // four workgroups per CU, 23 KB of table each
__global__ __launch_bounds__(kSwigluThreads) void swiglu_table_kernel(SwigluArgs a) {
  constexpr int VEC = 8;
  __shared__ float silu_tab[kSiluEntries];
  silu_fill(silu_tab, kSwigluThreads);
  __syncthreads();
  const int nc = a.inter / VEC;
  for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
    const uint16_t* gr = (const uint16_t*)a.g + r * a.in_st;
    const uint16_t* ur = (const uint16_t*)a.u + r * a.in_st;
    uint16_t* orow = (uint16_t*)a.out + r * a.out_st;
    for (int k0 = threadIdx.x; k0 < nc; k0 += kSwigluThreads * kSwigluAhead) {
      u32x4 cg[kSwigluAhead], cu[kSwigluAhead];
#pragma unroll
      for (int u = 0; u < kSwigluAhead; ++u) {
        const int k = min(k0 + u * kSwigluThreads, nc - 1);
        cg[u] = *(const u32x4*)(gr + k * VEC);
        cu[u] = *(const u32x4*)(ur + k * VEC);
      }
#pragma unroll
      for (int u = 0; u < kSwigluAhead; ++u) {
        const int k = k0 + u * kSwigluThreads;
        uint32_t slot[VEC];
        bool hit = true;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          slot[j] = silu_slot(elem<uint16_t>(cg[u], j));
          hit = hit && slot[j] < (uint32_t)kSiluEntries;
        }
        float o[VEC];
        if (__all(hit)) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) o[j] = bf16_round(silu_tab[slot[j]] * elem<uint16_t>(cu[u], j));
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) o[j] = bf16_round(silu_bf16(elem<uint16_t>(cg[u], j)) * elem<uint16_t>(cu[u], j));
        }
        if (k < nc) *(u32x4*)(orow + k * VEC) = pack<uint16_t>(o);
      }
    }
  }
}



// ---------------------------------------------------------------------------
// Debiased readout scores (Service::run_debiased's averaging,
// crates/cev-runtime/src/service.rs:330-345, with math::log_softmax,
// crates/cev-core/src/math.rs:14-18).  One wave per question; lane p holds
// position p of a variant's logits (k <= 64 options).  log_softmax in f64:
// m = the f32 max, lse = m + ln(sum_j e^(z_j - m)) summed in position order
// like the reference's iterator, lp_p = z_p - lse.  Every variant adds
// (lp_p - base_p) / n to the score of option order[p], variants in span
// order; base is the calibration twin's log_softmax (0 without one).
struct DebiasArgs {
  const int32_t* span_begin;
  const int32_t* span_len;
  const int32_t* n_options;
  const float* logits;
  const float* calib;
  const int32_t* order;
  float* scores;
  int32_t n_variants, ld;
};

__device__ __forceinline__ double readlane_f64(double x, int j) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, j), hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), j);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// log_softmax at this lane's position of a k-wide row (lanes >= k: unused)
__device__ __forceinline__ double log_softmax_lane(float z, int k, int lane) {
  float m = -INFINITY;
  for (int j = 0; j < k; ++j) m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, z), j)));
  const double m64 = (double)m;
  const double e = lane < k ? exp((double)z - m64) : 0.0;
  double sum = 0.0;
  for (int j = 0; j < k; ++j) sum += readlane_f64(e, j);
  return (double)z - (m64 + log(sum));
}

__global__ __launch_bounds__(64) void debias_kernel(DebiasArgs a) {
  __shared__ double score[64];
  const int q = blockIdx.x, lane = threadIdx.x;
  score[lane] = 0.0;
  const int k = a.n_options[q], b = a.span_begin[q], n = a.span_len[q];
  float* out = a.scores + (int64_t)q * a.ld;
  // a span outside the variants or an option count outside [1, min(ld, 64)]:
  // the question's scores are NaN (a launch cannot return an error)
  const bool span_ok = k >= 1 && k <= min(a.ld, 64) && n >= 1 && b >= 0 && b <= a.n_variants - n;
  if (!span_ok) {
    if (lane < a.ld) out[lane] = __builtin_nanf("");
    return;
  }
  bool order_ok = true;
  for (int v = b; v < b + n; ++v) {
    const int64_t row = (int64_t)v * a.ld;
    const float z = lane < k ? a.logits[row + lane] : 0.0f;
    double d = log_softmax_lane(z, k, lane);
    if (a.calib) d -= log_softmax_lane(lane < k ? a.calib[row + lane] : 0.0f, k, lane);
    const int o = lane < k ? a.order[row + lane] : -1;
    // order must be a permutation of 0..k-1: every option is named by
    // exactly one of the k lanes (a repeated index leaves another unnamed)
    for (int j = 0; j < k; ++j) order_ok &= __popcll(__ballot(o == j)) == 1;
    // each option then gets one lane's term per variant; the barrier keeps
    // variants in order (LDS work of one wave)
    if (lane < k && o >= 0 && o < k) score[o] += d / (double)n;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const bool all_ok = __all(order_ok);
  if (lane < k) out[lane] = all_ok ? (float)score[lane] : __builtin_nanf("");
}

}  // namespace

namespace {

int32_t check_norm(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h, int64_t h_stride,
                   void* x_out, int64_t x_out_stride, const void* w, float eps, void* y, int64_t y_stride) {
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
  return CEV_OK;
}

int32_t rms_norm_seq(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h, int64_t h_stride,
                     void* x_out, int64_t x_out_stride, const void* w, float eps, int32_t weight_plus_one, void* y, int64_t y_stride,
                     cev_stream stream) {
  const int vec = dtype == CEV_BF16 ? 8 : 4;
  NormArgs a{x, h, x_out, w, y, rows, x_stride, h_stride, x_out_stride, y_stride, hidden, weight_plus_one, eps};
  const int pitch = norm_pitch(hidden);
  const int rows_per_wg = std::min({kNormRows, kNormLdsBytes / pitch, kNormThreads * kNormChunks / (hidden / vec)});
  CEV_CHECK_ARG(rows_per_wg >= 1, "cev_rms_norm: hidden %d too large for one row in LDS", hidden);
  const int64_t grid = (rows + rows_per_wg - 1) / rows_per_wg;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_rms_norm: too many rows");
  hipStream_t s = (hipStream_t)stream;
  const size_t lds = (size_t)rows_per_wg * pitch;
  if (dtype == CEV_BF16)
    hipLaunchKernelGGL(rms_norm_kernel<uint16_t>, dim3((unsigned)grid), dim3(kNormThreads), lds, s, a, rows_per_wg);
  else
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)grid), dim3(kNormThreads), lds, s, a, rows_per_wg);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_rms_norm launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

template <typename T>
int32_t launch_wave_norm(const NormArgs& a, int nch, hipStream_t s) {
  const int64_t grid = (a.rows + kWaveNormRows - 1) / kWaveNormRows;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_rms_norm: too many rows");
  const dim3 g((unsigned)grid), b(kWaveNormRows * 64);
  const bool res = a.h != nullptr;
  if (nch <= 4)
    hipLaunchKernelGGL(res ? (rms_norm_wave_kernel<T, 4, true>) : (rms_norm_wave_kernel<T, 4, false>), g, b, 0, s, a);
  else if (nch <= 8)
    hipLaunchKernelGGL(res ? (rms_norm_wave_kernel<T, 8, true>) : (rms_norm_wave_kernel<T, 8, false>), g, b, 0, s, a);
  else
    hipLaunchKernelGGL(res ? (rms_norm_wave_kernel<T, 16, true>) : (rms_norm_wave_kernel<T, 16, false>), g, b, 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_rms_norm launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

}  // namespace

extern "C" int32_t cev_rms_norm(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h,
                                int64_t h_stride, void* x_out, int64_t x_out_stride, const void* w, float eps, int32_t weight_plus_one,
                                void* y, int64_t y_stride, cev_stream stream) {
  int32_t rc = check_norm(dtype, rows, hidden, x, x_stride, h, h_stride, x_out, x_out_stride, w, eps, y, y_stride);
  if (rc || rows == 0) return rc;
  const int vec = dtype == CEV_BF16 ? 8 : 4;
  const int nch = (hidden / vec + 63) / 64;  // 16-byte chunks per lane
  if (nch > 16)  // rows wider than 16 chunks per lane: the sequential-sum kernel
    return rms_norm_seq(dtype, rows, hidden, x, x_stride, h, h_stride, x_out, x_out_stride, w, eps, weight_plus_one, y, y_stride, stream);
  NormArgs a{x, h, x_out, w, y, rows, x_stride, h_stride, x_out_stride, y_stride, hidden, weight_plus_one, eps};
  if (dtype == CEV_BF16) return launch_wave_norm<uint16_t>(a, nch, (hipStream_t)stream);
  return launch_wave_norm<float>(a, nch, (hipStream_t)stream);
}

extern "C" int32_t cev_rms_norm_seq(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h,
                                    int64_t h_stride, void* x_out, int64_t x_out_stride, const void* w, float eps, int32_t weight_plus_one,
                                    void* y, int64_t y_stride, cev_stream stream) {
  int32_t rc = check_norm(dtype, rows, hidden, x, x_stride, h, h_stride, x_out, x_out_stride, w, eps, y, y_stride);
  if (rc || rows == 0) return rc;
  return rms_norm_seq(dtype, rows, hidden, x, x_stride, h, h_stride, x_out, x_out_stride, w, eps, weight_plus_one, y, y_stride, stream);
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
    hipLaunchKernelGGL(swiglu_table_kernel, dim3((unsigned)std::min<int64_t>(rows, kSwigluBlocks)), dim3(kSwigluThreads), 0, s, a);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3((unsigned)grid), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_swiglu launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

extern "C" int32_t cev_debias_scores(int32_t n_questions, int32_t n_variants, const int32_t* span_begin, const int32_t* span_len,
                                     const int32_t* n_options, const float* logits, const float* calib, const int32_t* order, int32_t ld,
                                     float* scores, cev_stream stream) {
  CEV_CHECK_ARG(n_questions >= 0 && n_variants >= 0, "cev_debias_scores: negative count");
  CEV_CHECK_ARG(ld >= 1 && ld <= 64, "cev_debias_scores: row width %d outside [1, 64]", ld);
  if (n_questions == 0) return CEV_OK;
  CEV_CHECK_ARG(span_begin && span_len && n_options && logits && order && scores, "cev_debias_scores: null buffer");
  DebiasArgs a{span_begin, span_len, n_options, logits, calib, order, scores, n_variants, ld};
  hipLaunchKernelGGL(debias_kernel, dim3((unsigned)n_questions), dim3(64), 0, (hipStream_t)stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_debias_scores launch: %s", hipGetErrorString(e));
  return CEV_OK;
}
