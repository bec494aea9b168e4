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
// Three work splits, all summing each vector's squares in element order so
// the sum matches the reference's sequential f32 sum bit for bit:
//   qknorm_rope_lane_kernel (full rotary or a quarter of it, 16-byte aligned
//     rows): one lane per vector (token, head).  A wave reads its 64 vectors
//     with whole 128-byte lines and hands each lane its own vector through a
//     per-wave LDS tile; the lane sums, normalises and rotates the pairs
//     (i, i + rot/2) in registers, and the results go back out through the
//     tile the same way: one dependent add chain of D per lane, no
//     workgroup barrier after the weights.
//   qknorm_rope_quad_kernel (the same shapes, calls under 16,384 vectors):
//     four lanes per vector, the sum handed from lane to lane in order.
//   qknorm_rope_kernel (any other shape): a wave normalises 8 vectors at a
//     time; lanes load coalesced, the squares go through LDS and lanes 0..7
//     each sum one vector.
#include <algorithm>

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
  // Optional: token i's k (and v) rows go to row slots[i] of k_out (v_out)
  // instead of row i; v rows are copied unchanged by the workgroups from
  // qk_blocks on.
  const int32_t* slots;
  int32_t n_slots;
  int32_t qk_blocks;
  const void* v_in;
  void* v_out;
  int64_t vi_st, vi_sh, vo_st, vo_sh;
};

// Output row of token tk's k and v: slots[tk] when the caller maps tokens to
// cache slots, else tk; a slot outside [0, n_slots) stores nothing.
__device__ __forceinline__ int64_t kv_row(const QkArgs& a, int tk) {
  if (!a.slots) return tk;
  const int s = a.slots[tk];
  return (s >= 0 && s < a.n_slots) ? (int64_t)s : -1;
}

// The v part of a call (workgroups from a.qk_blocks on): every v row copied
// to its output row in 16-byte chunks, grid-strided.
template <typename T, int D>
__device__ void copy_v_rows(const QkArgs& a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int NCH = D / VEC;
  const int64_t total = (int64_t)a.t * a.hkv * NCH;
  const int64_t stride = (int64_t)(gridDim.x - a.qk_blocks) * blockDim.x;
  for (int64_t i = (int64_t)(blockIdx.x - a.qk_blocks) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t vr = i / NCH;
    const int ch = (int)(i % NCH);
    const int tk = (int)(vr / a.hkv), h = (int)(vr % a.hkv);
    const int64_t r = kv_row(a, tk);
    if (r < 0) continue;
    const uint4 v = *(const uint4*)((const T*)a.v_in + tk * a.vi_st + h * a.vi_sh + ch * VEC);
    *(uint4*)((T*)a.v_out + r * a.vo_st + h * a.vo_sh + ch * VEC) = v;
  }
}

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
  if ((int)blockIdx.x >= a.qk_blocks) {
    copy_v_rows<T, D>(a);
    return;
  }
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
      const int64_t r = kv_row(a, tk);
      dst[j] = r >= 0 ? (T*)a.k_out + r * a.ko_st + h * a.ko_sh : nullptr;
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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Element j of a 16-byte chunk: bf16 packs two per dword (low half first).
template <typename T>
__device__ __forceinline__ float chunk_get(const u32x4& c, int j) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w = c[j >> 1];
    return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(c[j]);
  }
}
// Elements 2i, 2i+1 of a chunk from two values: bf16 rounds both to nearest
// even and packs them (one v_cvt_pk_bf16_f32); f32 stores them as they are.
template <typename T>
__device__ __forceinline__ void chunk_set2(u32x4& c, int i, float lo, float hi) {
  if constexpr (sizeof(T) == 2) {
    const __bf16 l = (__bf16)lo, h = (__bf16)hi;
    c[i] = (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
  } else {
    c[2 * i] = __float_as_uint(lo);
    c[2 * i + 1] = __float_as_uint(hi);
  }
}

constexpr int kLaneThreads = 256;
constexpr int kStageRow = 144;      // bytes per vector row of a staging tile: 128 + 16 pad

// A pointer into global memory (loads and stores through it are global, not
// flat, instructions).
template <typename V>
using gptr = __attribute__((address_space(1))) V*;

// The value of lane src's x (a 64-bit value in two permutes).
__device__ __forceinline__ uint64_t shfl_u64(uint64_t x, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)x, src, 64), hi = (uint32_t)__shfl((int)(uint32_t)(x >> 32), src, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Waves per SIMD the register budget is held to: the packed vector takes
// D * sizeof(T) / 16 * 4 registers per lane.
template <typename T, int D>
constexpr int lane_waves() { return D * (int)sizeof(T) >= 512 ? 2 : 3; }

template <typename T, int D, int ROT, int TPB>
__global__ __launch_bounds__(TPB) __attribute__((amdgpu_waves_per_eu(lane_waves<T, D>()))) void qknorm_rope_lane_kernel(
    QkArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int VEC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int NC = D / VEC;               // chunks per vector
  constexpr int HALF = ROT / 2;
  constexpr int HC = HALF / VEC;            // chunks in the first rotary half
  static_assert(HALF % VEC == 0 && ROT <= D, "rotary halves are whole chunks");
  auto rnd = [](float x) { return BF ? bf16_round(x) : x; };
  __shared__ __align__(16) float weff[2][D];  // the norm's weights, q's then k's
  // per wave: 64 vectors x 128 bytes (one staging round) + 16 bytes of pad
  constexpr int NR = NC / 8;  // staging rounds
  static_assert(NC % 8 == 0, "whole staging rounds");
  __shared__ __align__(16) char stage[TPB / 64][64 * kStageRow];
  if ((int)blockIdx.x >= a.qk_blocks) {
    copy_v_rows<T, D>(a);
    return;
  }

  const int64_t nq = (int64_t)a.t * a.hq;
  const int64_t total = nq + (int64_t)a.t * a.hkv;
  const int64_t v = (int64_t)blockIdx.x * TPB + threadIdx.x;
  // Lanes past the last vector redo the last one, so that they take part in
  // the staging exchange, and store nothing.
  const bool valid = v < total;
  const int64_t vv = valid ? v : total - 1;
  const T* src;
  T* dst;
  int tk;
  const bool is_q = vv < nq;
  if (is_q) {
    tk = (int)(vv / a.hq);
    const int h = (int)(vv % a.hq);
    src = (const T*)a.q_in + tk * a.qi_st + h * a.qi_sh;
    dst = (T*)a.q_out + tk * a.qo_st + h * a.qo_sh;
  } else {
    const int64_t vk = vv - nq;
    tk = (int)(vk / a.hkv);
    const int h = (int)(vk % a.hkv);
    src = (const T*)a.k_in + tk * a.ki_st + h * a.ki_sh;
    dst = (T*)a.k_out + h * a.ko_sh;  // the slot row is added below
  }
  // Loads the epilogue needs go out before the staging loads, so that no
  // dependent load waits behind them: the token's position and, for k, its
  // cache slot (every lane reads one; q lanes ignore theirs).
  const int p = a.pos[tk];
  const int slot = a.slots ? a.slots[tk] : tk;
  const float* wl = weff[is_q ? 0 : 1];
  const int lane = threadIdx.x & 63;
  char* st = stage[threadIdx.x >> 6];
  u32x4 c[NC];
  {
    // Staged load: in round q every instruction reads 128 bytes (chunks
    // 8q .. 8q+7) of 8 vectors, lane l taking vector 8i + l/8, chunk l%8;
    // the LDS tile then hands each lane its own vector.
    const uint64_t sp = (uint64_t)src;
    const int sub = lane >> 3, kc = lane & 7;
    gptr<const u32x4> vp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vp[i] = (gptr<const u32x4>)shfl_u64(sp, 8 * i + sub) + kc;
    // The first two rounds' loads go out before the workgroup's weight
    // loads, and each later round's two rounds ahead of its exchange (the LDS
    // syncs fence memory operations), so the weights and a vector cost about
    // one memory latency, not one per round.
    u32x4 g0[8], g1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) g0[i] = vp[i][0];
    if (NR > 1) {
#pragma unroll
      for (int i = 0; i < 8; ++i) g1[i] = vp[i][8];
    }
    // The weights as the norm multiplies them (1 + w rounded to the dtype
    // for the zero-centred form), once per workgroup: q's then k's.
    // The loads are unconditional (a side with no heads reads the other
    // side's weights and uses 0), so none waits behind a branch.
    constexpr int WN = (2 * D + TPB - 1) / TPB;
    const T* wsafe = a.hq > 0 ? (const T*)a.w_q : (const T*)a.w_k;
    float wraw[WN];
    bool whave[WN];
#pragma unroll
    for (int u = 0; u < WN; ++u) {
      const int i = threadIdx.x + u * TPB;
      whave[u] = i < 2 * D && (i < D ? a.hq > 0 : a.hkv > 0);
      const T* wp = whave[u] ? (i < D ? (const T*)a.w_q : (const T*)a.w_k) + i % D : wsafe;
      if constexpr (BF)
        wraw[u] = bf16_from_bits(*(const uint16_t*)wp);
      else
        wraw[u] = *(const float*)wp;
    }
#pragma unroll
    for (int u = 0; u < WN; ++u) {
      const int i = threadIdx.x + u * TPB;
      if (i < 2 * D) {
        const float w = a.plus_one ? rnd(wraw[u] + 1.0f) : wraw[u];
        weff[i / D][i % D] = whave[u] ? w : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      u32x4* g = q % 2 == 0 ? g0 : g1;
#pragma unroll
      for (int i = 0; i < 8; ++i) *(u32x4*)(st + (8 * i + sub) * kStageRow + 16 * kc) = g[i];
      wave_lds_sync();
#pragma unroll
      for (int k = 0; k < 8; ++k) c[8 * q + k] = *(const u32x4*)(st + lane * kStageRow + 16 * k);
      wave_lds_sync();
      if (q + 2 < NR) {
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = vp[i][8 * (q + 2)];
      }
    }
  }
  if (!is_q) {
    const bool slot_ok = !a.slots || (slot >= 0 && slot < a.n_slots);
    dst = slot_ok ? dst + (int64_t)slot * a.ko_st : nullptr;
  }

  float sum2 = 0.0f;
  int min_exp = 0;  // smallest frexp exponent of a nonzero element (0 for 0)
#pragma unroll
  for (int k = 0; k < NC; ++k)
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float x = chunk_get<T>(c[k], j);
      sum2 += x * x;
      min_exp = min(min_exp, __builtin_amdgcn_frexp_expf(x));
    }
  const float m = rnd(sqrtf(sum2 / (float)D + a.eps));
  // x / m, correctly rounded, for every element.  With y = RN(1/m),
  // q0 = RN(x y) and the exact residual r = x - q0 m, RN(q0 + r y) is the
  // correctly rounded quotient (Markstein) as long as r cannot underflow or
  // overflow: every nonzero |x| in [2^-96, 2^60] (sum2 <= 2^120 bounds the
  // top) and m in [2^-20, 2^20], checked for the whole wave; otherwise the
  // wave takes the IEEE division.  copysign keeps the sign of -0 / m.
  const bool fast = min_exp >= -95 && sum2 <= 0x1p120f && m >= 0x1p-20f && m <= 0x1p20f;
  const float y = 1.0f / m;
  const bool p_ok = p >= 0 && p < a.n_pos;
  const T* crow = (const T*)a.cos_t + (int64_t)(p_ok ? p : 0) * HALF;
  const T* srow = (const T*)a.sin_t + (int64_t)(p_ok ? p : 0) * HALF;

  // The chunks pass through an empty asm so the compiler unpacks them again
  // below instead of keeping all D unpacked values of the sum live.
#pragma unroll
  for (int k = 0; k < NC; ++k) asm volatile("" : "+v"(c[k]));

  // y = dtype(dtype(x / m) * w) on chunk k, then rotate-half on the pairs
  // (i, i + ROT/2) of the first ROT elements; a position outside the table
  // yields NaN there instead of a stray read.
  auto pair = [&](auto fast_c, u32x4& c0, u32x4& c1, int k, const u32x4& cc, const u32x4& sc) {
    constexpr bool FAST = decltype(fast_c)::value;
    auto quot = [&](float x) {
      if constexpr (FAST) {
        const float q0 = x * y;
        const float r = __builtin_fmaf(-q0, m, x);
        return __builtin_copysignf(__builtin_fmaf(r, y, q0), q0);
      } else {
        return x / m;
      }
    };
    float r0[VEC], r1[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const f32x4 w0 = *(const f32x4*)(wl + k * VEC + (j & ~3));
      const f32x4 w1 = *(const f32x4*)(wl + (k + HC) * VEC + (j & ~3));
      const float y0 = rnd(rnd(quot(chunk_get<T>(c0, j))) * w0[j & 3]);
      const float y1 = rnd(rnd(quot(chunk_get<T>(c1, j))) * w1[j & 3]);
      const float co = p_ok ? chunk_get<T>(cc, j) : __builtin_nanf("");
      const float si = p_ok ? chunk_get<T>(sc, j) : __builtin_nanf("");
      r0[j] = rnd(y0 * co) - rnd(y1 * si);
      r1[j] = rnd(y0 * si) + rnd(y1 * co);
    }
#pragma unroll
    for (int i = 0; i < VEC / 2; ++i) {
      chunk_set2<T>(c0, i, r0[2 * i], r0[2 * i + 1]);
      chunk_set2<T>(c1, i, r1[2 * i], r1[2 * i + 1]);
    }
  };
  auto single = [&](auto fast_c, u32x4& c0, int k) {
    constexpr bool FAST = decltype(fast_c)::value;
    float yv[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float x = chunk_get<T>(c0, j);
      float q;
      if constexpr (FAST) {
        const float q0 = x * y;
        q = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, m, x), y, q0), q0);
      } else {
        q = x / m;
      }
      yv[j] = rnd(rnd(q) * (*(const f32x4*)(wl + k * VEC + (j & ~3)))[j & 3]);
    }
#pragma unroll
    for (int i = 0; i < VEC / 2; ++i) chunk_set2<T>(c0, i, yv[2 * i], yv[2 * i + 1]);
  };

  if (__all(fast)) {
    // the table chunks of pair k are loaded TPD pairs ahead, so their
    // latency hides behind the pairs in between
    constexpr int TPD = HC < 2 ? HC : 2;
    u32x4 tcos[TPD > 0 ? TPD : 1], tsin[TPD > 0 ? TPD : 1];
#pragma unroll
    for (int k = 0; k < TPD; ++k) {
      tcos[k] = *(const u32x4*)(crow + k * VEC);
      tsin[k] = *(const u32x4*)(srow + k * VEC);
    }
#pragma unroll
    for (int k = 0; k < HC; ++k) {
      const u32x4 cc = tcos[k % TPD], sc = tsin[k % TPD];
      if (k + TPD < HC) {
        tcos[k % TPD] = *(const u32x4*)(crow + (k + TPD) * VEC);
        tsin[k % TPD] = *(const u32x4*)(srow + (k + TPD) * VEC);
      }
      pair(std::true_type{}, c[k], c[k + HC], k, cc, sc);
      // keeps each chunk's weight reads and the table loads next to their
      // use (hoisted, they take a register each and cap the waves per SIMD)
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int k = 2 * HC; k < NC; ++k) {
      single(std::true_type{}, c[k], k);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Staged store, the load's exchange in reverse: every instruction
    // writes whole 128-byte lines.  The empty asm makes each pair pack its
    // result where it is computed (sunk to the LDS writes, the unpacked
    // values of every pair would stay live at once and spill).
#pragma unroll
    for (int k = 0; k < NC; ++k) asm volatile("" : "+v"(c[k]));
    const uint64_t dp = (valid && dst) ? (uint64_t)dst : 0;
    const int sub = lane >> 3, kc = lane & 7;
    gptr<u32x4> vdst[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vdst[i] = (gptr<u32x4>)shfl_u64(dp, 8 * i + sub);
#pragma unroll
    for (int q = 0; q < NR; ++q) {
#pragma unroll
      for (int k = 0; k < 8; ++k) *(u32x4*)(st + lane * kStageRow + 16 * k) = c[8 * q + k];
      wave_lds_sync();
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32x4 val = *(const u32x4*)(st + (8 * i + sub) * kStageRow + 16 * kc);
        if (vdst[i]) vdst[i][8 * q + kc] = val;
      }
      wave_lds_sync();
    }
  } else if (valid && dst) {
    // Rare (a wave with a tiny, huge or non-finite element): IEEE division,
    // one chunk or rotary pair at a time, re-read from the input (each
    // chunk is read before its own store, so q_out may alias q_in).
#pragma unroll 1
    for (int k = 0; k < HC; ++k) {
      u32x4 c0 = *(const u32x4*)(src + k * VEC), c1 = *(const u32x4*)(src + (k + HC) * VEC);
      pair(std::false_type{}, c0, c1, k, *(const u32x4*)(crow + k * VEC), *(const u32x4*)(srow + k * VEC));
      *(u32x4*)(dst + k * VEC) = c0;
      *(u32x4*)(dst + (k + HC) * VEC) = c1;
    }
#pragma unroll 1
    for (int k = 2 * HC; k < NC; ++k) {
      u32x4 c0 = *(const u32x4*)(src + k * VEC);
      single(std::false_type{}, c0, k);
      *(u32x4*)(dst + k * VEC) = c0;
    }
  }
}


// The one-lane-per-vector kernel covers full and quarter rotary when every
// row, weight vector and table row is a whole number of 16-byte chunks.
template <typename T>
bool lane_kernel_fits(const QkArgs& a, int d) {
  const int vec = 16 / (int)sizeof(T);
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const int64_t st[] = {a.qi_st, a.qi_sh, a.ki_st, a.ki_sh, a.qo_st, a.qo_sh, a.ko_st, a.ko_sh};
  for (int64_t x : st)
    if (x % vec) return false;
  if (!(al(a.cos_t) && al(a.sin_t))) return false;
  if (a.hq && !(al(a.q_in) && al(a.q_out) && al(a.w_q))) return false;
  if (a.hkv && !(al(a.k_in) && al(a.k_out) && al(a.w_k))) return false;
  if (sizeof(T) == 4 && d == 256) return false;  // 256 registers of f32 per vector
  return a.rot == d || a.rot == d / 4;
}

// Calls with few vectors (a short suffix, small test passes) leave most
// SIMDs idle under the one-lane-per-vector split, and one lane's ~2,000
// dependent instructions then set the time.  Here a DPP quad (4 lanes)
// holds one vector, a contiguous quarter per lane.  The sum of squares still
// runs in element order: quad lane j adds its quarter to lane j-1's total.
// The rotate-half partners of full rotary sit two lanes apart (quad_perm
// lane ^ 2); a quarter rotary lies in lane 0's quarter.  Same per-element
// ops and division as the lane kernel, so the results are the same bits.
constexpr int kQuadThreads = 64;         // one wave: 16 vectors per workgroup
constexpr int64_t kQuadMaxVecs = 16384;  // calls below this use the quad split

template <typename T, int D, int ROT>
__global__ __launch_bounds__(kQuadThreads) void qknorm_rope_quad_kernel(QkArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int VEC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int E = D / 4;                  // elements per lane
  constexpr int NCL = E / VEC;              // chunks per lane
  static_assert(E % VEC == 0 && (ROT == D || ROT == D / 4), "whole chunks; full or quarter rotary");
  auto rnd = [](float x) { return BF ? bf16_round(x) : x; };
  __shared__ __align__(16) float weff[2][D];
  if ((int)blockIdx.x >= a.qk_blocks) {
    copy_v_rows<T, D>(a);
    return;
  }
  const int64_t nq = (int64_t)a.t * a.hq;
  const int64_t total = nq + (int64_t)a.t * a.hkv;
  const int j = threadIdx.x & 3;
  const int64_t v = ((int64_t)blockIdx.x * kQuadThreads + threadIdx.x) >> 2;
  // Quads past the last vector redo the last one (every lane of a quad must
  // take part in the DPP moves) and store nothing.
  const bool valid = v < total;
  const int64_t vv = valid ? v : total - 1;
  const T* src;
  T* dst;
  int tk;
  const bool is_q = vv < nq;
  if (is_q) {
    tk = (int)(vv / a.hq);
    const int h = (int)(vv % a.hq);
    src = (const T*)a.q_in + tk * a.qi_st + h * a.qi_sh;
    dst = (T*)a.q_out + tk * a.qo_st + h * a.qo_sh;
  } else {
    const int64_t vk = vv - nq;
    tk = (int)(vk / a.hkv);
    const int h = (int)(vk % a.hkv);
    src = (const T*)a.k_in + tk * a.ki_st + h * a.ki_sh;
    dst = (T*)a.k_out + h * a.ko_sh;  // the slot row is added below
  }
  // Every load the lane needs goes out before the first wait: its quarter of
  // the vector, the token's position and cache slot (q lanes ignore theirs)
  // and the workgroup's weights.  The weight loads are unconditional (a side
  // with no heads reads the other side's weights and stores 0), so none
  // waits behind a branch.
  u32x4 c[NCL];
#pragma unroll
  for (int k = 0; k < NCL; ++k) c[k] = *(const u32x4*)(src + j * E + k * VEC);
  const int p = a.pos[tk];
  const int slot = a.slots ? a.slots[tk] : tk;
  constexpr int WN = 2 * D / kQuadThreads;
  static_assert(2 * D % kQuadThreads == 0, "whole weight rounds");
  const T* wsafe = a.hq > 0 ? (const T*)a.w_q : (const T*)a.w_k;
  float wraw[WN];
#pragma unroll
  for (int u = 0; u < WN; ++u) {
    const int i = threadIdx.x + u * kQuadThreads;
    const bool have = i < D ? a.hq > 0 : a.hkv > 0;
    const T* wp = have ? (i < D ? (const T*)a.w_q : (const T*)a.w_k) + i % D : wsafe;
    if constexpr (BF)
      wraw[u] = bf16_from_bits(*(const uint16_t*)wp);
    else
      wraw[u] = *(const float*)wp;
    wraw[u] = have ? (a.plus_one ? rnd(wraw[u] + 1.0f) : wraw[u]) : 0.0f;
  }
  // the rotation's cos/sin chunks, loaded as soon as the position is known
  const bool p_ok = p >= 0 && p < a.n_pos;
  const T* crow = (const T*)a.cos_t + (int64_t)(p_ok ? p : 0) * (ROT / 2);
  const T* srow = (const T*)a.sin_t + (int64_t)(p_ok ? p : 0) * (ROT / 2);
  constexpr int NT = ROT == D ? NCL : NCL / 2;  // table chunks a lane reads
  const int tb = ROT == D ? (j & 1) * E : 0;     // table index of its first element
  u32x4 ctab[NT], stab[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    ctab[k] = *(const u32x4*)(crow + tb + k * VEC);
    stab[k] = *(const u32x4*)(srow + tb + k * VEC);
  }
#pragma unroll
  for (int u = 0; u < WN; ++u) {
    const int i = threadIdx.x + u * kQuadThreads;
    weff[i / D][i % D] = wraw[u];
  }
  __syncthreads();
  if (!is_q) {
    const bool slot_ok = !a.slots || (slot >= 0 && slot < a.n_slots);
    dst = slot_ok ? dst + (int64_t)slot * a.ko_st : nullptr;
  }
  const float* wl = weff[is_q ? 0 : 1] + j * E;

  // smallest frexp exponent of a nonzero element over the quad (0 for 0)
  int min_exp = 0;
#pragma unroll
  for (int k = 0; k < NCL; ++k)
#pragma unroll
    for (int e = 0; e < VEC; ++e) min_exp = min(min_exp, __builtin_amdgcn_frexp_expf(chunk_get<T>(c[k], e)));
  min_exp = min(min_exp, (int)dpp_u<0xB1>((uint32_t)min_exp));  // lane ^ 1
  min_exp = min(min_exp, (int)dpp_u<0x4E>((uint32_t)min_exp));  // lane ^ 2
  // the sum of squares in element order, handed from lane to lane
  float acc = 0.0f;
#pragma unroll
  for (int step = 0; step < 4; ++step) {
    const float prev = dpp_f<0x90>(acc);  // quad_perm [0, 0, 1, 2]: lane j - 1's total
    if (j == step) {
      float s = step == 0 ? 0.0f : prev;
#pragma unroll
      for (int k = 0; k < NCL; ++k)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float x = chunk_get<T>(c[k], e);
          s += x * x;
        }
      acc = s;
    }
  }
  const float sum2 = dpp_f<0xFF>(acc);  // quad_perm [3, 3, 3, 3]: lane 3 holds the total
  const float m = rnd(sqrtf(sum2 / (float)D + a.eps));
  const bool fast = min_exp >= -95 && sum2 <= 0x1p120f && m >= 0x1p-20f && m <= 0x1p20f;
  const float y = 1.0f / m;

  auto body = [&](auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    // dtype(dtype(x / m) * w) for element e of chunk k
    auto norm = [&](const u32x4& ck, int k, int e) {
      const float x = chunk_get<T>(ck, e);
      float q;
      if constexpr (FAST) {
        const float q0 = x * y;
        q = __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, m, x), y, q0), q0);
      } else {
        q = x / m;
      }
      return rnd(rnd(q) * wl[k * VEC + e]);
    };
    if constexpr (ROT == D) {
      // lane j < 2 holds x_i of the pair (x_i, x_{i + D/2}), lane j + 2 the
      // other: r = dtype(ya * ca) + dtype(yb * cb) gives
      //   x_i'         = dtype(x_i c) - dtype(x_{i+D/2} s)   (j < 2),
      //   x_{i+D/2}'   = dtype(x_i s) + dtype(x_{i+D/2} c)   (j >= 2).
      const bool first = j < 2;
#pragma unroll
      for (int k = 0; k < NCL; ++k) {
        float yo[VEC], yp[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) yo[e] = norm(c[k], k, e);
#pragma unroll
        for (int e = 0; e < VEC; ++e) yp[e] = dpp_f<0x4E>(yo[e]);  // the partner's (lane ^ 2)
        const u32x4 cc = ctab[k], sc = stab[k];
        float r[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float co = p_ok ? chunk_get<T>(cc, e) : __builtin_nanf("");
          const float si = p_ok ? chunk_get<T>(sc, e) : __builtin_nanf("");
          const float ya = first ? yo[e] : yp[e];
          const float yb = first ? yp[e] : yo[e];
          const float ca = first ? co : si, cb = first ? -si : co;
          r[e] = rnd(ya * ca) + rnd(yb * cb);
        }
#pragma unroll
        for (int i = 0; i < VEC / 2; ++i) chunk_set2<T>(c[k], i, r[2 * i], r[2 * i + 1]);
      }
    } else {
      // quarter rotary: the pairs (i, i + E/2) of lane 0's quarter
      constexpr int HC = NCL / 2;
      if (j == 0) {
#pragma unroll
        for (int k = 0; k < HC; ++k) {
          const u32x4 cc = ctab[k], sc = stab[k];
          float r0[VEC], r1[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float y0 = norm(c[k], k, e), y1 = norm(c[k + HC], k + HC, e);
            const float co = p_ok ? chunk_get<T>(cc, e) : __builtin_nanf("");
            const float si = p_ok ? chunk_get<T>(sc, e) : __builtin_nanf("");
            r0[e] = rnd(y0 * co) - rnd(y1 * si);
            r1[e] = rnd(y0 * si) + rnd(y1 * co);
          }
#pragma unroll
          for (int i = 0; i < VEC / 2; ++i) {
            chunk_set2<T>(c[k], i, r0[2 * i], r0[2 * i + 1]);
            chunk_set2<T>(c[k + HC], i, r1[2 * i], r1[2 * i + 1]);
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < NCL; ++k) {
          float r[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) r[e] = norm(c[k], k, e);
#pragma unroll
          for (int i = 0; i < VEC / 2; ++i) chunk_set2<T>(c[k], i, r[2 * i], r[2 * i + 1]);
        }
      }
    }
  };
  if (__all(fast))
    body(std::true_type{});
  else
    body(std::false_type{});
  if (valid && dst) {
#pragma unroll
    for (int k = 0; k < NCL; ++k) *(u32x4*)(dst + j * E + k * VEC) = c[k];
  }
}

// Workgroups that copy v after the q/k ones: one 16-byte chunk per thread,
// at most kVBlocks workgroups striding over the rest.
constexpr int64_t kVBlocks = 2048;
template <typename T>
int64_t v_blocks(const QkArgs& a, int d, int tpb) {
  if (!a.v_in) return 0;
  const int64_t chunks = (int64_t)a.t * a.hkv * (d / (16 / (int)sizeof(T)));
  return std::min<int64_t>(kVBlocks, (chunks + tpb - 1) / tpb);
}

template <typename T>
int32_t launch_quad(QkArgs a, int d, int64_t vecs, hipStream_t s) {
  const int64_t qk = (4 * vecs + kQuadThreads - 1) / kQuadThreads;
  a.qk_blocks = (int32_t)qk;
  const int64_t grid = qk + v_blocks<T>(a, d, kQuadThreads);
  const dim3 g((unsigned)grid), b(kQuadThreads);
  if (d == 128 && a.rot == 128)
    hipLaunchKernelGGL((qknorm_rope_quad_kernel<T, 128, 128>), g, b, 0, s, a);
  else if (d == 128)
    hipLaunchKernelGGL((qknorm_rope_quad_kernel<T, 128, 32>), g, b, 0, s, a);
  else if constexpr (sizeof(T) == 2) {
    if (a.rot == 256)
      hipLaunchKernelGGL((qknorm_rope_quad_kernel<T, 256, 256>), g, b, 0, s, a);
    else
      hipLaunchKernelGGL((qknorm_rope_quad_kernel<T, 256, 64>), g, b, 0, s, a);
  } else {
    return cev_fail(CEV_ERR_UNSUPPORTED, "qknorm_rope: no quad kernel for f32 at d = %d", d);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "qknorm_rope launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

template <typename T, int TPB>
int32_t launch_lane(QkArgs a, int d, int64_t vecs, hipStream_t s) {
  const int64_t qk = (vecs + TPB - 1) / TPB;
  if (qk > INT32_MAX / 2) return cev_fail(CEV_ERR_UNSUPPORTED, "qknorm grid too large");
  a.qk_blocks = (int32_t)qk;
  const int64_t grid = qk + v_blocks<T>(a, d, TPB);
  const dim3 g((unsigned)grid), b(TPB);
  if (d == 128 && a.rot == 128)
    hipLaunchKernelGGL((qknorm_rope_lane_kernel<T, 128, 128, TPB>), g, b, 0, s, a);
  else if (d == 128)
    hipLaunchKernelGGL((qknorm_rope_lane_kernel<T, 128, 32, TPB>), g, b, 0, s, a);
  else if constexpr (sizeof(T) == 2) {
    if (a.rot == 256)
      hipLaunchKernelGGL((qknorm_rope_lane_kernel<T, 256, 256, TPB>), g, b, 0, s, a);
    else
      hipLaunchKernelGGL((qknorm_rope_lane_kernel<T, 256, 64, TPB>), g, b, 0, s, a);
  } else {
    return cev_fail(CEV_ERR_UNSUPPORTED, "qknorm_rope: no lane kernel for f32 at d = %d", d);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "qknorm_rope launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

template <typename T>
int32_t launch_qk(QkArgs a, int d, hipStream_t s) {
  const int64_t vecs = (int64_t)a.t * (a.hq + a.hkv);
  if (vecs == 0) return CEV_OK;
  if (lane_kernel_fits<T>(a, d)) {
    if (vecs < kQuadMaxVecs) return launch_quad<T>(a, d, vecs, s);
    // One-wave workgroups for a short call (under 64 workgroups of 256
    // lanes), which then spreads over more CUs.
    if (vecs < (int64_t)kLaneThreads * 64) return launch_lane<T, 64>(a, d, vecs, s);
    return launch_lane<T, kLaneThreads>(a, d, vecs, s);
  }
  const int64_t per_wg = (int64_t)WAVES * VPW;
  const int64_t qk = (vecs + per_wg - 1) / per_wg;
  if (qk > INT32_MAX / 2) return cev_fail(CEV_ERR_UNSUPPORTED, "qknorm grid too large");
  a.qk_blocks = (int32_t)qk;
  const int64_t grid = qk + v_blocks<T>(a, d, WAVES * 64);
  if (d == 128)
    hipLaunchKernelGGL((qknorm_rope_kernel<T, 128>), dim3((unsigned)grid), dim3(WAVES * 64), 0, s, a);
  else
    hipLaunchKernelGGL((qknorm_rope_kernel<T, 256>), dim3((unsigned)grid), dim3(WAVES * 64), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "qknorm_rope launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

}  // namespace

namespace {

int32_t qknorm_rope_impl(const cev_qknorm_desc* d, const void* q_in, const void* k_in, const void* v_in, int64_t vi_st, int64_t vi_sh,
                         const void* w_q, const void* w_k, const int32_t* pos, const void* cos_t, const void* sin_t, const int32_t* slots,
                         int32_t n_slots, void* q_out, void* k_out, void* v_out, int64_t vo_st, int64_t vo_sh, cev_stream stream) {
  CEV_CHECK_ARG(d != nullptr, "cev_qknorm_rope: null descriptor");
  if (d->dtype != CEV_F32 && d->dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_qknorm_rope: dtype %d", d->dtype);
  if (d->head_dim != 128 && d->head_dim != 256) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_qknorm_rope: head_dim %d", d->head_dim);
  CEV_CHECK_ARG(d->t >= 0 && d->n_q_heads >= 0 && d->n_kv_heads >= 0, "cev_qknorm_rope: negative sizes");
  CEV_CHECK_ARG(d->rotary_dim >= 2 && d->rotary_dim % 2 == 0 && d->rotary_dim <= d->head_dim, "cev_qknorm_rope: rotary_dim %d",
                d->rotary_dim);
  CEV_CHECK_ARG(d->n_pos >= 1, "cev_qknorm_rope: empty cos/sin table");
  CEV_CHECK_ARG(d->eps >= 0.0f, "cev_qknorm_rope: negative eps");
  CEV_CHECK_ARG(!slots || n_slots >= 0, "cev_qknorm_rope: negative slot count");
  if (d->t == 0 || d->n_q_heads + d->n_kv_heads == 0) return CEV_OK;
  CEV_CHECK_ARG(pos && cos_t && sin_t, "cev_qknorm_rope: null pos or table");
  CEV_CHECK_ARG(d->n_q_heads == 0 || (q_in && q_out && w_q), "cev_qknorm_rope: null q buffers");
  CEV_CHECK_ARG(d->n_kv_heads == 0 || (k_in && k_out && w_k), "cev_qknorm_rope: null k buffers");
  if (v_in || v_out) {
    CEV_CHECK_ARG(v_in && v_out && d->n_kv_heads > 0, "cev_qknorm_rope_kv: v_in and v_out go together, with kv heads");
    const int64_t vec = d->dtype == CEV_BF16 ? 8 : 4;
    CEV_CHECK_ARG(((uintptr_t)v_in & 15) == 0 && ((uintptr_t)v_out & 15) == 0 && vi_st % vec == 0 && vi_sh % vec == 0 &&
                      vo_st % vec == 0 && vo_sh % vec == 0 && vi_st >= 0 && vi_sh >= 0 && vo_st >= 0 && vo_sh >= 0,
                  "cev_qknorm_rope_kv: v rows must be 16-byte aligned");
  }
  QkArgs a{};
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
  a.slots = slots;
  a.n_slots = n_slots;
  a.qk_blocks = INT32_MAX;
  a.v_in = v_in;
  a.v_out = v_out;
  a.vi_st = vi_st;
  a.vi_sh = vi_sh;
  a.vo_st = vo_st;
  a.vo_sh = vo_sh;
  hipStream_t s = (hipStream_t)stream;
  if (d->dtype == CEV_BF16) return launch_qk<uint16_t>(a, d->head_dim, s);
  return launch_qk<float>(a, d->head_dim, s);
}

}  // namespace

extern "C" int32_t cev_qknorm_rope(const cev_qknorm_desc* d, const void* q_in, const void* k_in, const void* w_q, const void* w_k,
                                   const int32_t* pos, const void* cos_t, const void* sin_t, void* q_out, void* k_out, cev_stream stream) {
  return qknorm_rope_impl(d, q_in, k_in, nullptr, 0, 0, w_q, w_k, pos, cos_t, sin_t, nullptr, 0, q_out, k_out, nullptr, 0, 0, stream);
}

extern "C" int32_t cev_qknorm_rope_kv(const cev_qknorm_desc* d, const void* q_in, const void* k_in, const void* v_in, int64_t vi_stride_t,
                                      int64_t vi_stride_h, const void* w_q, const void* w_k, const int32_t* pos, const void* cos_t,
                                      const void* sin_t, const int32_t* slots, int32_t n_slots, void* q_out, void* k_out, void* v_out,
                                      int64_t vo_stride_t, int64_t vo_stride_h, cev_stream stream) {
  return qknorm_rope_impl(d, q_in, k_in, v_in, vi_stride_t, vi_stride_h, w_q, w_k, pos, cos_t, sin_t, slots, n_slots, q_out, k_out, v_out,
                          vo_stride_t, vo_stride_h, stream);
}
