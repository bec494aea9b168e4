// Packed-prefill attention for gfx950: the replacement for Attention::attend
// (crates/cev-model/src/qwen3.rs:206-220, crates/cev-model/src/qwen35.rs:563-579)
// with the block-offset table in place of the dense mask.
//
// Design (one workgroup = one tile of query rows x one KV head [x one part
// of the tile's key stream when it is split]):
//   - the 8 waves x 32 query slots of a workgroup hold 256/g rows x the g
//     query heads of one KV head's GQA group (slot -> row slot/g, head
//     slot%g), so a K/V key tile staged in LDS once is scored by 256 queries;
//   - scores are computed transposed, S^T = K . Q^T, on 32x32 MFMA tiles: a
//     lane then holds 16 keys of ONE query row, and the softmax row max and
//     row sum reduce inside the lane plus one permlane32 swap;
//   - online softmax in base 2 (exp2(q.k * scale * log2 e - m)), f32 state,
//     O rescaled only when a row max grows by more than 2^kRescale;
//   - O^T = V^T . P^T accumulates on MFMA with P kept in registers as the B
//     operand (its K slots follow the S^T register order);
//   - K/V key tiles stream through LDS ahead of the one being scored: bf16
//     chunks go from HBM straight into a four-deep LDS ring (buffer_load ...
//     lds), f32 chunks are double-buffered through registers;
//   - the key ranges a tile visits come from the plan: spans are unmasked,
//     local keys are masked per row from the row's [lo, hi) + diag;
//   - blockIdx -> (tile, part, kv head) with the kv head fastest, so the
//     workgroups of one XCD (dispatched round-robin over the 8 XCDs) share a
//     KV head and its K/V stream stays in that XCD's L2;
//   - a split tile writes (unnormalised O, m, l) per row and head to the
//     workspace and attn_merge_kernel combines the parts.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "cev_device.h"
#include "cev_internal.h"
#include "cev_plan.h"

namespace {

struct AttnArgs {
  const void* q;
  const void* kc;
  const void* vc;
  const void* kn;
  const void* vn;
  const void* gate;
  void* out;
  char* ws;  // split records: outputs, then (m, l) pairs (cev_plan.h)
  const int32_t* plan;
  int64_t q_st, q_sh, kc_ss, kc_sh, vc_ss, vc_sh, kn_st, kn_sh, vn_st, vn_sh, g_st, g_sh, o_st, o_sh;
  int32_t n_tiles, t, s_cache, hq, hkv, g, has_gate, n_splits, tile_rows;
  int32_t rows_dense;  // the host plan's tiles cover rows [0, t) in order, each row once
  float scale_log2;
  uint32_t plan_sig;  // signature of the host plan this launch was validated with
};

constexpr float kRescale = 8.0f;
// Largest sum of a lane's 16 probabilities of one sub-tile that the d = 128
// loop accepts before it moves the row's max (so p < 2^16 there).
constexpr float kMaxP = 65536.0f;
constexpr float kLog2MaxP = 16.0f;  // log2(kMaxP)

// The plan header on the device must be the host plan's (same signature,
// same launch shape).  A device plan that is not a copy of the validated
// host plan is never followed: the attention kernels fill the whole output
// with NaN instead (poison_output) and the merge pass writes nothing, so a
// stale device plan shows in the result rather than leaving rows unwritten.
// The header is read at once and every field compared (no short-circuit,
// which would make each field a dependent load).
// The header stays in h for the offsets the kernel reads next.
__device__ __forceinline__ bool header_ok(const AttnArgs& a, const cev_plan_header& h) {
  // the section offsets follow the header in order (this also loads them
  // with the other fields)
  constexpr int32_t kHeaderWords = (int32_t)(sizeof(cev_plan_header) / 4);
  return (h.magic == CEV_PLAN_MAGIC) & ((uint32_t)h.sig == a.plan_sig) & (h.n_tiles == a.n_tiles) & (h.t == a.t) &
         (h.s_cache == a.s_cache) & (h.n_splits == a.n_splits) & (h.tiles_off >= kHeaderWords) & (h.segs_off >= h.tiles_off) &
         (h.rows_off >= h.segs_off);
}
__device__ __forceinline__ bool plan_ok(const AttnArgs& a, cev_plan_header& h) {
  h = *(const cev_plan_header*)a.plan;
  return header_ok(a, h);
}

// Workgroup b of the grid writes NaN over output rows [b t / G, (b+1) t / G)
// of every query head (the launcher validated the output strides).
template <typename T, int D>
__device__ void poison_output(const AttnArgs& a) {
  const int64_t G = gridDim.x;
  const int64_t r0 = (int64_t)blockIdx.x * a.t / G, r1 = (int64_t)(blockIdx.x + 1) * a.t / G;
  const int64_t per_row = (int64_t)a.hq * D;
  for (int64_t i = threadIdx.x; i < (r1 - r0) * per_row; i += blockDim.x) {
    const int64_t r = r0 + i / per_row, h = (i % per_row) / D, e = i % D;
    ((T*)a.out)[r * a.o_st + h * a.o_sh + e] = (T)__builtin_nanf("");
  }
}

// Clamps a segment to the key buffer it starts in.
__device__ __forceinline__ int4 clamp_seg(int4 sg, int s_cache, int t) {
  sg.x = max(sg.x, 0);
  const int lim = sg.x < s_cache ? s_cache : s_cache + t;
  sg.y = min(sg.y, lim);
  return sg;
}

__device__ __forceinline__ float gate_value(float o, float g, bool bf16) {
  // out * sigmoid(g), each op in the model dtype (qwen35.rs:556-558)
  if (bf16) {
    float e = bf16_round(expf(-g));
    float den = bf16_round(e + 1.0f);
    // bf16(1 / den) from the hardware reciprocal (1 ulp): den = D 2^p with
    // D an 8-bit integer, a bf16 rounding midpoint is M 2^q with M an odd
    // 9-bit integer, and D M is never a power of two, so 1 / den lies at
    // least 2^-17 (relative) from every midpoint and a 2^-23 error cannot
    // change its bf16 rounding.  Below 2^-126 (den > 2^126) the reciprocal
    // is an f32 denormal, which the division still gives exactly.
    float sg = bf16_round(den < 0x1p126f ? __builtin_amdgcn_rcpf(den) : 1.0f / den);
    return bf16_round(bf16_round(o) * sg);
  }
  return o * (1.0f / (expf(-g) + 1.0f));
}

__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The larger of x and its value in lane ^ 16 (within each 32-lane half).
__device__ __forceinline__ float pair16_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// x plus its value in lane ^ 16 (within each 32-lane half).
__device__ __forceinline__ float pair16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 lds_read_tr(const __bf16* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

// --------------------------------------------------------------------------
// Per-dtype MFMA fragments.
//
// bf16 (v_mfma_f32_32x32x16_bf16): Q as the B operand, 8 head-dim values per
// lane per step; P converted to bf16 B operands whose K slot 8u + j of half
// h is S^T register 8h + j (key 16h + 8(j/4) + 4u + j%4 of a sub-tile); the
// V^T A operand comes from ds_read_b64_tr_b16 on the key-major V tile.
//
// f32 (v_mfma_f32_32x32x2_f32, full f32 products): the head-dim order of
// the QK^T K slots is permuted (d = 8k + 4u + r) so a lane reads 4
// consecutive floats for 4 steps; one K=2 PV step per S^T register.
//
// Both expose the work as small steps so the main loop can interleave the
// MFMAs of one sub-tile with the VALU work of another:
//   qk_step(st), st < NQK   - builds one 32x32 S^T sub-tile;
//   pv_step(j),  j < NPV    - adds one sub-tile's V^T . P^T to O;
//   make_p                  - probabilities -> PV operand, plus their sum.
template <typename T, int D>
struct Frag;

#ifndef CEV_VPAD_BF16
#define CEV_VPAD_BF16 32
#endif

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int D>
struct Frag<__bf16, D> {
  static constexpr int BN = D == 128 ? 64 : 32;
  static constexpr int PAD = 8;
  static constexpr int VPAD = CEV_VPAD_BF16;
  static constexpr int VEC = 8;
  static constexpr int NQK = D / 16;
  static constexpr int NPV = 2 * (D / 32);
  typedef bf16x8 Vec;
  struct P {
    bf16x8 h[2];
  };
  bf16x8 q[D / 16];

  __device__ __forceinline__ void load_q(const __bf16* qp, bool ok, int u) {
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      bf16x8 z = {};
      q[s] = ok ? *(const bf16x8*)(qp + 16 * s + 8 * u) : z;
    }
  }
  // q * c rounded to bf16: the QK^T MFMAs then give scores already in the
  // base-2 units of the softmax (c = scale * log2 e).
  __device__ __forceinline__ void scale_q(float c) {
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) q[s][e] = (__bf16)((float)q[s][e] * c);
  }

  // K operand of QK step st: key kt*32 + n, head-dim values 16st + 8u ..
  template <int RS>
  __device__ __forceinline__ static bf16x8 k_frag(const __bf16* sK, int kt, int st, int n, int u) {
    return *(const bf16x8*)&sK[(kt * 32 + n) * RS + 16 * st + 8 * u];
  }
  __device__ __forceinline__ void qk_mfma(const bf16x8& af, int st, f32x16& s) const {
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, q[st], s, 0, 0, 0);
  }
  template <int RS>
  __device__ __forceinline__ void qk_step(const __bf16* sK, int kt, int st, int n, int u, f32x16& s) const {
    qk_mfma(k_frag<RS>(sK, kt, st, n, u), st, s);
  }

  // The row sum is taken over the bf16 probabilities PV multiplies, on the
  // dot-product unit (two products per instruction).
  __device__ __forceinline__ static void make_p(const f32x16& e, P& p, float& rs) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) p.h[h][j] = (__bf16)e[8 * h + j];
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 8; j += 2) rs = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{p.h[h][j], p.h[h][j + 1]}, one, rs, false);
  }

  // Step j = h * (D/32) + dt: o[dt] += V^T(keys of half h) . P^T(half h).
  // Lane (group g16 = lane/16, i = lane%16) reads row kb + i/4, columns
  // d0 + 4(i%4) .. +3; the transpose load hands it 4 consecutive keys of
  // head-dim column d0 + i.
  template <int RS>
  __device__ __forceinline__ static bf16x8 v_frag(const __bf16* sV, int kt, int j, int lane, int u) {
    const int h = j / (D / 32), dt = j % (D / 32);
    const int tr_row = (lane & 15) >> 2;
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const __bf16* vp = sV + (kt * 32 + 16 * h + 4 * u + tr_row) * RS + dt * 32 + tr_col;
    const bf16x4 lo = lds_read_tr(vp);
    const bf16x4 hi = lds_read_tr(vp + 8 * RS);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  __device__ __forceinline__ static void pv_mfma(const bf16x8& af, int j, const P& p, f32x16* o) {
    const int h = j / (D / 32), dt = j % (D / 32);
    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, p.h[h], o[dt], 0, 0, 0);
  }
  template <int RS>
  __device__ __forceinline__ void pv_step(const __bf16* sV, int kt, int j, int lane, int u, const P& p, f32x16* o) const {
    pv_mfma(v_frag<RS>(sV, kt, j, lane, u), j, p, o);
  }
};

template <int D>
struct Frag<float, D> {
  static constexpr int BN = 32;
  static constexpr int PAD = 4;
  static constexpr int VPAD = 4;
  static constexpr int VEC = 4;
  static constexpr int NQK = D / 8;
  static constexpr int NPV = 16;
  typedef f32x4 Vec;
  struct P {
    f32x16 v;
  };
  f32x4 q[D / 8];

  __device__ __forceinline__ void load_q(const float* qp, bool ok, int u) {
#pragma unroll
    for (int k = 0; k < D / 8; ++k) q[k] = ok ? *(const f32x4*)(qp + 8 * k + 4 * u) : f32x4{};
  }

  template <int RS>
  __device__ __forceinline__ void qk_step(const float* sK, int kt, int k, int n, int u, f32x16& s) const {
    const f32x4 af = *(const f32x4*)&sK[(kt * 32 + n) * RS + 8 * k + 4 * u];
#pragma unroll
    for (int r = 0; r < 4; ++r) s = __builtin_amdgcn_mfma_f32_32x32x2f32(af[r], q[k][r], s, 0, 0, 0);
  }

  __device__ __forceinline__ static void make_p(const f32x16& e, P& p, float& rs) {
    p.v = e;
#pragma unroll
    for (int i = 0; i < 16; ++i) rs += e[i];
  }

  template <int RS>
  __device__ __forceinline__ void pv_step(const float* sV, int kt, int i, int lane, int u, const P& p, f32x16* o) const {
    const int n = lane & 31;
    const int key = kt * 32 + 8 * (i >> 2) + 4 * u + (i & 3);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(sV[key * RS + dt * 32 + n], p.v[i], o[dt], 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ void store_vec4(T* p, const float* v);
template <>
__device__ __forceinline__ void store_vec4<__bf16>(__bf16* p, const float* v) {
  bf16x4 r = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
  *(bf16x4*)p = r;
}
template <>
__device__ __forceinline__ void store_vec4<float>(float* p, const float* v) {
  *(f32x4*)p = f32x4{v[0], v[1], v[2], v[3]};
}

template <typename T>
__device__ __forceinline__ void load_vec4(const T* p, float* v);
template <>
__device__ __forceinline__ void load_vec4<__bf16>(const __bf16* p, float* v) {
  const bf16x4 g = *(const bf16x4*)p;
  for (int e = 0; e < 4; ++e) v[e] = (float)g[e];
}
template <>
__device__ __forceinline__ void load_vec4<float>(const float* p, float* v) {
  const f32x4 g = *(const f32x4*)p;
  for (int e = 0; e < 4; ++e) v[e] = g[e];
}

// Four values of a record's output as loaded (bf16x4 or f32x4) and their
// f32 form.
template <typename T>
using VecOf = typename std::conditional<sizeof(T) == 2, bf16x4, f32x4>::type;
// E values of T as one load or store: bf16x8 for E = 8, else VecOf<T>.
template <typename T, int E>
using VecN = typename std::conditional<E == 8, bf16x8, VecOf<T>>::type;
__device__ __forceinline__ f32x4 to_f32x4(const bf16x4& v) { return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]}; }
__device__ __forceinline__ f32x4 to_f32x4(const f32x4& v) { return v; }

// The normalised, optionally gated output of one query slot (row, head):
// lane half ue holds columns 32 dt + 8 q4 + 4 ue .. +3 of o[dt].  bf16
// layers multiply by 1/l (the result is rounded to bf16), f32 layers divide
// by l.  The gate's loads are all issued before the first store, so each of
// the row's output lines is written in one burst; with one load round trip
// between stores, lines sat half written in L2 and went to HBM twice.
template <typename T, int D>
__device__ __forceinline__ void store_output(const AttnArgs& a, int row, int head, int ue, const f32x16* o, float l) {
  constexpr int NDT = D / 32;
  constexpr bool BF = sizeof(T) == 2;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  T* op = (T*)a.out + (int64_t)row * a.o_st + (int64_t)head * a.o_sh;
  auto value = [&](int dt, int i) { return BF ? o[dt][i] * inv : (l > 0.0f ? o[dt][i] / l : 0.0f); };
  if (a.has_gate) {
    const T* gp = (const T*)a.gate + (int64_t)row * a.g_st + (int64_t)head * a.g_sh;
    VecOf<T> graw[NDT][4];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) graw[dt][q4] = *(const VecOf<T>*)(gp + dt * 32 + 8 * q4 + 4 * ue);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4 gv = to_f32x4(graw[dt][q4]);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gate_value(value(dt, 4 * q4 + e), gv[e], BF);
        store_vec4<T>(op + dt * 32 + 8 * q4 + 4 * ue, v);
      }
  } else {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = value(dt, 4 * q4 + e);
        store_vec4<T>(op + dt * 32 + 8 * q4 + 4 * ue, v);
      }
  }
}

// Index of record (row, head, part) in the split workspace.
__device__ __forceinline__ int64_t record_index(const AttnArgs& a, int row, int head, int part) {
  return ((int64_t)row * a.hq + head) * a.n_splits + part;
}
// Output of record i, and the (m, l) region that follows all outputs.
template <typename T, int D>
__device__ __forceinline__ T* record_out(const AttnArgs& a, int64_t i) {
  return (T*)a.ws + i * D;
}
template <typename T, int D>
__device__ __forceinline__ float2* record_ml(const AttnArgs& a) {
  return (float2*)(a.ws + (int64_t)a.t * a.hq * a.n_splits * D * (int64_t)sizeof(T));
}

// Writes this lane's share of partial record (row, head, part): output
// values d .. d+3 of every (dt, q4) slice (d = 32 dt + 8 q4 + 4u), then m
// and l from the lane with u == 0.
template <typename T, int D>
__device__ __forceinline__ void write_record(const AttnArgs& a, int row, int head, int part, const f32x16* o, int u, float m, float l) {
  const int64_t i = record_index(a, row, head, part);
  T* rec = record_out<T, D>(a, i);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = dt * 32 + 8 * q4 + 4 * u;
      const float v[4] = {o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]};
      store_vec4<T>(rec + d, v);
    }
  if (u == 0) record_ml<T, D>(a)[i] = make_float2(m, l);
}

// Word 3 of a raw buffer resource on gfx9: 32-bit data format, no swizzle.
constexpr int kBufferWord3 = 0x00020000;

// Values the compiler cannot prove wave-uniform (they come through vector
// loads of the plan) but are: readfirstlane moves them to SGPRs, where a
// buffer resource must live.
__device__ __forceinline__ int uniform_i32(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Keeps a value computed where it stands: sched_barrier only fences the
// machine scheduler, and without a use the IR passes sink the row max and
// row sum past the MFMAs they are meant to overlap.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// One BN-key chunk of a tile's key stream: keys key0 .. key0 + BN, the first
// nvalid of them inside the segment; local != 0 when the segment's keys are
// masked per row.
struct Chunk {
  int key0, nvalid, local;
};

// Cursor over the BN-key chunks of a tile's segments.  The current segment,
// clamped, stays in SGPRs; the plan is read only when the cursor enters a
// new segment (readfirstlane tells the compiler these vector-loaded values
// are wave-uniform).
template <int BN>
struct ChunkCursor {
  const int4* segs;
  int nseg, s_cache, t;
  int si, k0;
  int4 cur;

  __device__ __forceinline__ int4 seg(int i) const {
    const int4 sg = clamp_seg(segs[i], s_cache, t);
    return make_int4(uniform_i32(sg.x), uniform_i32(sg.y), uniform_i32(sg.z), 0);
  }
  // Positions the cursor on chunk c of the tile's stream.
  __device__ __forceinline__ void seek(int c) {
    si = 0;
    k0 = 0;
    cur = make_int4(0, 0, 0, 0);
    for (; si < nseg; ++si) {
      cur = seg(si);
      const int nch = (max(0, cur.y - cur.x) + BN - 1) / BN;
      if (c < nch) {
        k0 = c * BN;
        return;
      }
      c -= nch;
    }
  }
  __device__ __forceinline__ bool valid() const { return si < nseg; }
  __device__ __forceinline__ void next() {
    k0 += BN;
    if (cur.x + k0 < cur.y) return;
    k0 = 0;
    for (++si; si < nseg; ++si) {
      cur = seg(si);
      if (cur.y > cur.x) return;
    }
  }
  __device__ __forceinline__ Chunk here() const {
    Chunk ch{0, 0, 0};
    if (si < nseg) {
      ch.key0 = cur.x + k0;
      ch.nvalid = max(0, min(BN, cur.y - ch.key0));
      ch.local = cur.z;
    }
    return ch;
  }
};

// K/V rows of one KV head (cache rows [0, s_cache), then the new rows),
// fetched with buffer loads whose byte range ends at a chunk's last valid
// key: rows past it read as zero.
template <typename T>
struct KvSource {
  uint64_t kc, vc, kn, vn;         // row 0 of this head
  int kc_rb, vc_rb, kn_rb, vn_rb;  // row strides in bytes
  int s_cache;

  __device__ __forceinline__ void init(const AttnArgs& a, int kvh) {
    kc = (uint64_t)((const T*)a.kc + kvh * a.kc_sh);
    vc = (uint64_t)((const T*)a.vc + kvh * a.vc_sh);
    kn = (uint64_t)((const T*)a.kn + kvh * a.kn_sh);
    vn = (uint64_t)((const T*)a.vn + kvh * a.vn_sh);
    kc_rb = (int)(a.kc_ss * (int64_t)sizeof(T));
    vc_rb = (int)(a.vc_ss * (int64_t)sizeof(T));
    kn_rb = (int)(a.kn_st * (int64_t)sizeof(T));
    vn_rb = (int)(a.vn_st * (int64_t)sizeof(T));
    s_cache = a.s_cache;
  }
  // Buffer resources for chunk ch and the row strides they use.
  __device__ __forceinline__ void rsrc(const Chunk& ch, __amdgpu_buffer_rsrc_t& rk, __amdgpu_buffer_rsrc_t& rv, int& kr, int& vr) const {
    const bool cached = ch.key0 < s_cache;
    kr = uniform_i32(cached ? kc_rb : kn_rb);
    vr = uniform_i32(cached ? vc_rb : vn_rb);
    const int64_t row0 = cached ? ch.key0 : ch.key0 - s_cache;
    const uint64_t kp = uniform_u64((cached ? kc : kn) + (uint64_t)(row0 * kr));
    const uint64_t vp = uniform_u64((cached ? vc : vn) + (uint64_t)(row0 * vr));
    rk = __builtin_amdgcn_make_buffer_rsrc((void*)kp, (short)0, uniform_i32(ch.nvalid * kr), kBufferWord3);
    rv = __builtin_amdgcn_make_buffer_rsrc((void*)vp, (short)0, uniform_i32(ch.nvalid * vr), kBufferWord3);
  }
};

// Loads this thread's share of chunk ch (NLD 16-byte vectors per tensor).
template <typename T, int D, int NLD, int NT, typename Vec>
__device__ __forceinline__ void load_chunk(const KvSource<T>& src, const Chunk& ch, int tid, Vec* kreg, Vec* vreg) {
  constexpr int VEC = 16 / sizeof(T);
  __amdgpu_buffer_rsrc_t rk, rv;
  int kr, vr;
  src.rsrc(ch, rk, rv, kr, vr);
#pragma unroll
  for (int r = 0; r < NLD; ++r) {
    const int v = tid + r * NT;
    const int key = v / (D / VEC), col = (v % (D / VEC)) * VEC;
    kreg[r] = __builtin_bit_cast(Vec, __builtin_amdgcn_raw_buffer_load_b128(rk, key * kr + col * (int)sizeof(T), 0, 0));
    vreg[r] = __builtin_bit_cast(Vec, __builtin_amdgcn_raw_buffer_load_b128(rv, key * vr + col * (int)sizeof(T), 0, 0));
  }
}

// Query slot (wave, n = lane % 32) of a workgroup over tile rows [r0, r0 +
// len) and KV head kvh holds tile row slot / g and query head slot % g: the
// valid rows of a short tile fill the first waves.
struct SlotRow {
  int row, head, u;
  bool ok;
};
__device__ __forceinline__ SlotRow slot_row(int lane, int wave, int kvh, int g, int r0, int len, int t) {
  const int slot = wave * 32 + (lane & 31);
  const int rit = slot / g;
  SlotRow sr;
  sr.ok = rit < len && r0 + rit < t;
  sr.row = sr.ok ? r0 + rit : 0;
  sr.head = kvh * g + slot % g;
  sr.u = lane >> 5;
  return sr;
}

// This lane's id, computed afresh (opaque to common-subexpression elimination).
__device__ __forceinline__ int fresh_lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// --------------------------------------------------------------------------
// bf16, d = 128: the MFMA and VALU halves of consecutive 32-key sub-tiles
// overlap inside each wave (the loop below says how).  Two waves share a
// SIMD at 256 VGPRs, and the per-chunk barrier keeps them in step, so a
// wave cannot rely on the other one to fill its idle issue slots.
//
// K/V chunks go from HBM straight into LDS (buffer_load ... lds), NBUF
// chunk buffers deep, so up to NBUF-2 chunks are in flight per workgroup
// without holding registers.  Tiles are unpadded, 256 bytes a key row, with
// the 16-byte column blocks of a row permuted so the operand reads are free
// of bank conflicts:
//   K: block c of row r at slot c ^ (r & 15)   (ds_read_b128, one key row
//      per lane, 16 rows per 256 bytes read)
//   V: block c of row r at slot c ^ 4(r & 3)   (ds_read_b64_tr_b16, four
//      rows x four blocks per 16 lanes)
namespace pipe {
constexpr int kBuf = 4;             // chunk buffers
constexpr int kAhead = kBuf - 1;    // chunk i + kAhead is fetched in iteration i
constexpr int kRowBytes = 256;      // one bf16 key row of d = 128
constexpr int kTileBytes = 64 * kRowBytes;
constexpr int kVBase = kBuf * kTileBytes;  // K tiles first, then V tiles

__device__ __forceinline__ int k_slot(int blk, int row) { return blk ^ (row & 15); }
__device__ __forceinline__ int v_slot(int blk, int row) { return blk ^ ((row & 3) << 2); }

// Workgroup barrier after this wave's LDS operations have completed; global
// loads may still be in flight.  The asm is a compiler memory barrier too.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// V^T operand reads.  The compiler places an s_waitcnt vmcnt(0) before
// every ds_read_b64_tr_b16 it emits while an LDS DMA is in flight (it
// cannot tell the buffers apart), which would drain the whole fetch
// pipeline once per sub-tile.  These reads are issued from asm instead;
// buffer reuse is ordered by the explicit vmcnt wait and barrier at the end
// of each iteration, and wait_tr() below makes a fragment's registers
// depend on the reads having returned.
template <int OFF>
__device__ __forceinline__ i32x2 read_tr(int vaddr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  i32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(vaddr), "i"(OFF) : "memory");
  return r;
}
// The K operand reads go through asm as well, so that every LDS read in the
// loop body is one whose position the waits below can count.
template <int OFF>
__device__ __forceinline__ i32x4 read_b128(int vaddr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(vaddr), "i"(OFF) : "memory");
  return r;
}
// One K operand fragment: a 16-byte read per lane.  Two 8-byte reads of
// the same bytes measured no faster; the reads are bound by LDS bytes.
typedef i32x4 KFrag;
// LDS returns in order: once at most N LGKM operations are outstanding,
// every LDS read issued before the last N LDS reads has landed (an older
// scalar load still in flight only makes the wait stricter).
template <int N>
__device__ __forceinline__ void wait_tr(i32x2& lo, i32x2& hi) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(lo), "+v"(hi) : "i"(N));
}
template <int N>
__device__ __forceinline__ void wait_b128(i32x4& r) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}

// Issue order of the LDS reads of one sub-tile body (NQK = 8 QK units, then
// NPV = 8 PV units), K reads KPF and V fragments VPF ahead of their MFMA.
// QK unit u waits for K read u, then issues K read u + KPF (if any) and, in
// its last VPF units, the two reads of V fragment u - (8 - VPF).  PV unit j
// waits for V fragment j, then issues V fragment j + VPF (if any) and, in
// its last KPF units, K read j - (8 - KPF) of the next body.  The wait of
// each unit is the number of LDS reads issued after the one it needs; the
// count below replays one steady-state body.
struct ReadSchedule {
  int wait_a[8], wait_b[8];
};
constexpr ReadSchedule read_schedule(int kpf, int vpf) {
  ReadSchedule r{};
  int kpos[8] = {}, vhi[8] = {};
  int pos = 0;
  // the previous body's PV units: V reads of that body, then this body's
  // first kpf K reads
  for (int j = 0; j < 8; ++j) {
    if (j + vpf < 8) pos += 2;
    if (j >= 8 - kpf) kpos[j - (8 - kpf)] = pos++;
  }
  for (int u = 0; u < 8; ++u) {
    r.wait_a[u] = pos - kpos[u] - 1;
    if (u + kpf < 8) kpos[u + kpf] = pos++;
    if (u >= 8 - vpf) {
      vhi[u - (8 - vpf)] = pos + 1;
      pos += 2;
    }
  }
  for (int j = 0; j < 8; ++j) {
    r.wait_b[j] = pos - vhi[j] - 1;
    if (j + vpf < 8) {
      vhi[j + vpf] = pos + 1;
      pos += 2;
    }
    if (j >= 8 - kpf) ++pos;
  }
  return r;
}
constexpr bool waits_in_range(const ReadSchedule& r) {
  for (int i = 0; i < 8; ++i)
    if (r.wait_a[i] < 0 || r.wait_a[i] > 15 || r.wait_b[i] < 0 || r.wait_b[i] > 15) return false;
  return true;
}
// The loop's two forms.  Staggered (STAG): waves 4-7 run one region ahead of
// waves 0-3; on the 32k-key prefill with all 8 waves busy it ran 1.4 %
// faster than in step, and four K and two V fragments ahead ran 0.5 %
// faster there than three and three.  In step, three and three: a tile with
// at most 4 busy waves (a short block, the KV-streaming shape) has nothing
// to stagger, and there the staggered form's code ran 3 % slower.
template <bool STAG>
struct Schedule {
  static constexpr int KPF = STAG ? 4 : 3;  // K fragments in flight ahead of their MFMA
  static constexpr int VPF = STAG ? 2 : 3;  // V fragments in flight ahead of their MFMA
  static_assert(KPF >= 1 && KPF <= 8 && VPF >= 1 && VPF <= 8, "prefetch depths");
  static constexpr ReadSchedule reads = read_schedule(KPF, VPF);
  static_assert(waits_in_range(reads), "lgkmcnt range");
  static constexpr int wait_a(int st) { return reads.wait_a[st]; }
  static constexpr int wait_b(int j) { return reads.wait_b[j]; }
};
static_assert(Schedule<false>::wait_a(0) == 2 && Schedule<false>::wait_a(5) == 2 && Schedule<false>::wait_a(6) == 3 &&
                  Schedule<false>::wait_a(7) == 4 && Schedule<false>::wait_b(0) == 4 && Schedule<false>::wait_b(4) == 4 &&
                  Schedule<false>::wait_b(5) == 4 && Schedule<false>::wait_b(6) == 3 && Schedule<false>::wait_b(7) == 2,
              "wait counts at three fragments ahead");
static_assert(Schedule<true>::wait_a(0) == 5 && Schedule<true>::wait_a(1) == 3 && Schedule<true>::wait_a(5) == 2 &&
                  Schedule<true>::wait_a(6) == 1 && Schedule<true>::wait_a(7) == 2 && Schedule<true>::wait_b(0) == 2 &&
                  Schedule<true>::wait_b(5) == 3 && Schedule<true>::wait_b(6) == 4 && Schedule<true>::wait_b(7) == 2,
              "wait counts at four K and two V fragments ahead");
}  // namespace pipe

template <typename T, int D, bool STAG>
__global__ __launch_bounds__(kAttnWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_kernel_pipe(AttnArgs a) {
  using F = Frag<T, D>;
  using P = typename F::P;
  constexpr int BN = F::BN;
  constexpr int NKT = BN / 32;    // 32-key sub-tiles per chunk
  constexpr int NDT = D / 32;     // 32-wide slices of the head dim
  static_assert(sizeof(T) == 2 && D == 128 && BN == 64 && kAttnWaves == 8, "the pipelined loop is sized for bf16, d = 128");
  static_assert(F::NQK == 8 && F::NPV == 8, "unit layout below");
  using namespace pipe;
  using Sched = Schedule<STAG>;
  __shared__ __align__(16) char lds[2 * kBuf * kTileBytes];

  cev_plan_header ph;
  if (!plan_ok(a, ph)) {
    poison_output<T, D>(a);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform_i32(tid >> 6);
  const int n = lane & 31, u = lane >> 5;
  const int kvh = blockIdx.x % a.hkv;
  const int item = blockIdx.x / a.hkv;
  const int tile = item / a.n_splits, part = item % a.n_splits;
  const int4* tdp = (const int4*)(a.plan + ph.tiles_off) + 2 * tile;
  const int4 td = tdp[0];
  const int n_chunks = tdp[1].x;
  const int4* segs = (const int4*)(a.plan + ph.segs_off) + td.z;
  const int nseg = td.w;
  const int4* rows = (const int4*)(a.plan + ph.rows_off);
  // Query slot (wave, n) holds row slot / g of the tile, query head slot % g:
  // the valid rows of a short tile fill the first waves, and a wave with no
  // valid row skips the MFMA work (it still fetches its share of K/V).
  const SlotRow sr0 = slot_row(lane, wave, kvh, a.g, td.x, td.y, a.t);
  const bool row_ok = sr0.ok;
  const int row = sr0.row, head = sr0.head;
  const bool wave_active = (wave * 32) / a.g < td.y;

  // Q arrives scaled by c = scale * log2 e, so an S^T tile holds base-2
  // softmax arguments.  Each sub-tile's first QK^T MFMA starts from negm =
  // -m_run instead of zero, so the tile comes out as c q.k - m_run and the
  // probabilities are one exp2 per score.
  F fr;
  fr.load_q((const T*)a.q + (int64_t)row * a.q_st + (int64_t)head * a.q_sh, row_ok, u);
  fr.scale_q(a.scale_log2);
  int4 rv = rows[row];
  if (!row_ok) rv = make_int4(0, 0, -1, 0);

  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
  // m_set: this row has seen a visible key, and m_run is a max it reached
  // (0 until then); rows that never see one keep l = 0.
  float m_run = 0.0f, l_run = 0.0f;
  bool m_set = false;

  // ---- this part's slice of the tile's key stream: chunks [c0, c1)
  const int c0 = (int)((int64_t)part * n_chunks / a.n_splits);
  const int c1 = (int)((int64_t)(part + 1) * n_chunks / a.n_splits);
  const int nc = c1 - c0;
  ChunkCursor<BN> cursor{segs, nseg, a.s_cache, a.t, 0, 0, make_int4(0, 0, 0, 0)};
  cursor.seek(c0);
  if (nc <= 0 || !cursor.valid()) {
    // no key visible to this part: empty record / zero rows below
  } else {
    KvSource<T> kvs;
    kvs.init(a, kvh);

    // Per-lane byte offsets of the operand reads inside a tile; the
    // sub-tile, half and buffer parts are immediates.
    int koff[F::NQK], voff[NDT];
#pragma unroll
    for (int st = 0; st < F::NQK; ++st) koff[st] = n * kRowBytes + (k_slot(2 * st + u, n) << 4);
    {
      const int i = lane & 15, g16 = (lane >> 4) & 1, rr = i >> 2;
      const int blk = 2 * g16 + ((i & 3) >> 1);  // 16-byte block of the read, within a 64-byte slice
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        voff[dt] = kVBase + (4 * u + rr) * kRowBytes + (v_slot(4 * dt + blk, rr) << 4) + 8 * (i & 1);
    }
    auto k_frag = [&](int buf, int kt, int st) {
      return *(const bf16x8*)(lds + koff[st] + buf * kTileBytes + kt * 32 * kRowBytes);
    };
    // V^T fragment j (h = j / 4, head-dim slice dt = j % 4) of sub-tile KT in
    // buffer BUF: the transpose reads of rows r and r + 8.
    const int lds_base = (int)(size_t)(const __attribute__((address_space(3))) char*)lds;
    struct VFrag {
      i32x2 lo, hi;
    };
    auto v_issue = [&](auto buf_c, auto kt_c, auto j_c) {
      constexpr int BUF = decltype(buf_c)::value, KT = decltype(kt_c)::value, J = decltype(j_c)::value;
      constexpr int OFF = BUF * kTileBytes + (KT * 32 + 16 * (J / NDT)) * kRowBytes;
      const int va = lds_base + voff[J % NDT];
      return VFrag{read_tr<OFF>(va), read_tr<OFF + 8 * kRowBytes>(va)};
    };
    auto v_ready = [](VFrag& f, auto j_c) {
      wait_tr<Sched::wait_b(decltype(j_c)::value)>(f.lo, f.hi);
      const bf16x4 lo = __builtin_bit_cast(bf16x4, f.lo), hi = __builtin_bit_cast(bf16x4, f.hi);
      return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // K fragment st of sub-tile KT in buffer BUF.
    auto k_issue = [&](auto buf_c, auto kt_c, auto st_c) {
      constexpr int OFF = decltype(buf_c)::value * kTileBytes + decltype(kt_c)::value * 32 * kRowBytes;
      return read_b128<OFF>(lds_base + koff[decltype(st_c)::value]);
    };
    auto k_ready = [](KFrag& r, auto st_c) {
      wait_b128<Sched::wait_a(decltype(st_c)::value)>(r);
      return __builtin_bit_cast(bf16x8, r);
    };

    // Chunk ch into buffer buf: each wave fetches rows 8w .. 8w+7 of K and
    // of V, four rows (1 KB) per instruction; rows past the chunk's last
    // valid key read as zero.
    auto fetch = [&](const Chunk& ch, int buf) {
      __amdgpu_buffer_rsrc_t rk, rvs;
      int kr, vr;
      kvs.rsrc(ch, rk, rvs, kr, vr);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int krow = 8 * wave + 4 * r + (lane >> 4), blk = lane & 15;
        const int kdst = buf * kTileBytes + (8 * wave + 4 * r) * kRowBytes;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(lds + kdst), 16,
                                                 krow * kr + (k_slot(blk, krow) << 4), 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rvs, (__attribute__((address_space(3))) void*)(lds + kVBase + kdst), 16,
                                                 krow * vr + (v_slot(blk, krow) << 4), 0, 0, 0);
      }
    };
    constexpr int kLoadsPerChunk = 4;  // buffer_load ... lds per wave per chunk

    auto needs_mask = [](const Chunk& ch) { return ch.local != 0 || ch.nvalid < BN; };
    // Masks sub-tile kt of chunk ch in place and returns its lane-local max.
    auto mask_sub = [&](f32x16& s, int kt, const Chunk& ch) {
      // Branch-free on purpose: a short-circuit && / || here gives every
      // element its own control flow, and hipcc 7.2 then reuses the score
      // register of element 0 for `key` and drops its select.
      const bool all_rows = ch.local == 0;
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kk = kt * 32 + 8 * (i >> 2) + 4 * u + (i & 3);
        const int key = ch.key0 + kk;
        const bool vis = (kk < ch.nvalid) & (all_rows | ((key >= rv.x) & (key < rv.y)) | (key == rv.z));
        s[i] = vis ? s[i] : -INFINITY;
        mx = fmaxf(mx, s[i]);
      }
      return mx;
    };

    // Stale LDS must hold finite values: a masked key's V row is multiplied
    // by p = 0.  Zero every buffer once before the first fetch.  The
    // barrier waits for LDS writes only, so the query loads stay in flight
    // under the first fetches (__syncthreads would drain them first).
    for (int i = tid; i < 2 * kBuf * kTileBytes / 16; i += kAttnWaves * 64) *(f32x4*)(lds + 16 * i) = f32x4{};
    lds_barrier();

    // chs[k] is chunk i + k of the part; chunks past its end are empty
    // (their fetch reads no memory).
    int produced = 0;
    auto next_chunk = [&]() {
      Chunk ch{0, 0, 0};
      if (produced < nc) {
        if (produced > 0) cursor.next();
        ch = cursor.here();
      }
      ++produced;
      return ch;
    };
    Chunk chs[kAhead + 1];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      chs[k] = next_chunk();
      fetch(chs[k], k);
    }
    wait_vmcnt<kLoadsPerChunk * (kAhead - 2)>();  // chunks 0 and 1 landed
    __builtin_amdgcn_s_barrier();

    f32x16 sa, sb, negm;
    float mx = -INFINITY;  // lane-local max of the current sub-tile, relative to m_run
    if (wave_active) {
      // Sub-tile 0 scored from zero: its row max (over both lane halves of
      // the row) becomes m_run, and the tile is shifted by it.
      sa = f32x16{};
#pragma unroll
      for (int st = 0; st < F::NQK; ++st) fr.qk_mfma(k_frag(0, 0, st), st, sa);
      if (needs_mask(chs[0])) {
        mx = mask_sub(sa, 0, chs[0]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sa[i]);
      }
      const float m0 = pair_max(mx);
      m_set = m0 > -INFINITY;
      m_run = m_set ? m0 : 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sa[i] -= m_run;
      mx -= m_run;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) negm[i] = -m_run;
    // K reads in flight into the next body: the first body's are issued
    // here (sub-tile 1 of chunk 0) and waited for in full, so that its
    // counted waits see no fewer reads than a steady-state body's.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    constexpr int KPF = Sched::KPF, VPF = Sched::VPF;
    KFrag kf[KPF];
    if (wave_active) {
      static_for<KPF>([&](auto f_c) { kf[decltype(f_c)::value] = k_issue(I0{}, I1{}, f_c); });
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    // ---- main loop, software-pipelined over 32-key sub-tiles j, in two
    //   regions per sub-tile:
    //   A: scores S(j+1) = K(j+1) . Q^T on the MFMA unit while the VALU
    //      turns S(j) into probabilities, then the lazy-max check;
    //   B: O += V(j)^T . P(j) on the MFMA unit (no VALU work).
    //   Iteration i reads K of chunks i and i+1 and V of chunk i, fetches
    //   chunk i + kAhead into the buffer chunk i-1 used, and before its
    //   barrier waits for chunk i+2 to land.  In the staggered form, waves
    //   4-7 run one region ahead of waves 0-3 (they take region A of the
    //   next chunk's first sub-tile before the barrier), so the two waves of
    //   a SIMD are in opposite regions and one's softmax VALU work runs
    //   beside the other's P.V MFMAs; both groups still read only chunks i
    //   and i+1 in iteration i.
    VFrag vf[VPF];
    P p;
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    // Region A of sub-tile KT of the chunk in buffer B0.  Each unit ends in
    // a scheduling fence, so the order is the program order unit by unit:
    // one MFMA of one stream next to the VALU work of the other, with
    // operand reads KPF / VPF units ahead of their MFMA.  The part's last
    // sub-tile also scores a "next" one from a buffer of stale or zero keys,
    // never used: that keeps O out of a branch (where the compiler copies
    // all 64 accumulators).  Its last VPF units issue the first V fragments
    // of region B.
    auto region_a = [&](auto b0_c, auto kt_c) {
      constexpr int B0 = decltype(b0_c)::value, kt = decltype(kt_c)::value;
      constexpr bool last = kt + 1 == NKT;
      using BN_c = std::integral_constant<int, last ? (B0 + 1) % kBuf : B0>;  // buffer and sub-tile of the next scores
      using KTN_c = std::integral_constant<int, last ? 0 : kt + 1>;
      f32x16& s = kt % 2 == 0 ? sa : sb;
      f32x16& sn = kt % 2 == 0 ? sb : sa;
      float rs = 0.0f;
      static_for<F::NQK>([&](auto st_c) {
        constexpr int st = decltype(st_c)::value;
        if constexpr (st == 0)
          sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_ready(kf[0], st_c), fr.q[0], negm, 0, 0, 0);
        else
          fr.qk_mfma(k_ready(kf[st % KPF], st_c), st, sn);
        if constexpr (st + KPF < F::NQK) kf[st % KPF] = k_issue(BN_c{}, KTN_c{}, std::integral_constant<int, st + KPF>{});
        if constexpr (st >= F::NQK - VPF)
          vf[st - (F::NQK - VPF)] = v_issue(b0_c, kt_c, std::integral_constant<int, st - (F::NQK - VPF)>{});
        const float e0 = fast_exp2(s[2 * st]);
        const float e1 = fast_exp2(s[2 * st + 1]);
        const bf16x2 pr = {(__bf16)e0, (__bf16)e1};
        p.h[st / 4][2 * (st % 4)] = pr[0];
        p.h[st / 4][2 * (st % 4) + 1] = pr[1];
        rs = __builtin_amdgcn_fdot2_f32_bf16(pr, one, rs, false);
        pin(rs);
        __builtin_amdgcn_sched_barrier(0);
      });
      // Lazy max: S(j) came out relative to m_run, and its probabilities
      // stand as long as their row sum stays within kMaxP (O and l are f32).
      // Otherwise, or for a row with no max yet, the row moves its max (a
      // set row only when it grew by more than kRescale) and P(j) is made
      // again.  This branch issues no LDS operation, so the counted waits of
      // region B still hold.
      if (__ballot((rs > kMaxP) | !m_set)) {
        float ml = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) ml = fmaxf(ml, s[i]);
        const float delta = pair_max(ml);
        const bool move = m_set ? delta > kRescale : delta > -INFINITY;
        const float dm = move ? delta : 0.0f;
        const float alpha = m_set ? fast_exp2(-dm) : 1.0f;
        m_set = m_set | move;
        m_run += dm;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
        rs = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const bf16x2 pr = {(__bf16)fast_exp2(s[8 * h + j] - dm), (__bf16)fast_exp2(s[8 * h + j + 1] - dm)};
            p.h[h][j] = pr[0];
            p.h[h][j + 1] = pr[1];
            rs = __builtin_amdgcn_fdot2_f32_bf16(pr, one, rs, false);
          }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          sn[i] -= dm;
          negm[i] = -m_run;
        }
      }
      l_run += rs;
    };
    // Region B of sub-tile KT of the chunk in buffer B0: P.V, the next
    // region's first K reads, then the mask of the next scores (has1: the
    // part has a chunk after this one).
    auto region_b = [&](auto b0_c, auto kt_c, bool has1) {
      constexpr int B0 = decltype(b0_c)::value, kt = decltype(kt_c)::value;
      constexpr bool last = kt + 1 == NKT;
      f32x16& sn = kt % 2 == 0 ? sb : sa;
      static_for<F::NPV>([&](auto j_c) {
        constexpr int j = decltype(j_c)::value;
        F::pv_mfma(v_ready(vf[j % VPF], j_c), j, p, o);
        if constexpr (j + VPF < F::NPV) vf[j % VPF] = v_issue(b0_c, kt_c, std::integral_constant<int, j + VPF>{});
        // the next region A's first K reads: it scores sub-tile kt + 2
        if constexpr (j >= F::NPV - KPF)
          kf[j - (F::NPV - KPF)] = k_issue(std::integral_constant<int, (B0 + (kt + 2) / 2) % kBuf>{},
                                           std::integral_constant<int, (kt + 2) % 2>{},
                                           std::integral_constant<int, j - (F::NPV - KPF)>{});
        __builtin_amdgcn_sched_barrier(0);
      });
      if (!last || has1) {
        const Chunk& chn = last ? chs[1] : chs[0];
        if (needs_mask(chn)) mask_sub(sn, last ? 0 : kt + 1, chn);
      }
    };
    static_assert(NKT == 2, "two sub-tiles per chunk");
    const bool lead = STAG && wave >= kAttnWaves / 2;
    if (wave_active && lead) region_a(I0{}, I0{});
    auto step = [&](int ci, auto buf_tag) {
      constexpr int B0 = decltype(buf_tag)::value;  // buffer of chunk ci
      using B1_c = std::integral_constant<int, (B0 + 1) % kBuf>;
      const bool has1 = ci + 1 < nc;
      chs[kAhead] = next_chunk();
      fetch(chs[kAhead], (B0 + kAhead) % kBuf);
      if (wave_active) {
        if (!lead) region_a(buf_tag, I0{});
        region_b(buf_tag, I0{}, has1);
        region_a(buf_tag, I1{});
        region_b(buf_tag, I1{}, has1);
        if (lead && has1) region_a(B1_c{}, I0{});
      }
      // Chunk ci+2 (fetched in iteration ci-1) must have landed before the
      // barrier; chunk ci + kAhead may stay in flight.
      wait_vmcnt<kLoadsPerChunk * (kAhead - 2)>();
      __builtin_amdgcn_s_barrier();
#pragma unroll
      for (int k = 0; k < kAhead; ++k) chs[k] = chs[k + 1];
    };
    static_assert(kBuf == 4, "the unrolled loop below walks four buffers");
    for (int ci = 0; ci < nc; ci += kBuf) {
      step(ci, I0{});
      if (ci + 1 >= nc) break;
      step(ci + 1, I1{});
      if (ci + 2 >= nc) break;
      step(ci + 2, I2{});
      if (ci + 3 >= nc) break;
      step(ci + 3, I3{});
    }
    // Fetches past the part's end read no memory, but they still write
    // zeros into LDS: drain them, and the last body's K reads of a sub-tile
    // past the end, before the workgroup exits.
    wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  const float l = pair_sum(l_run);
  // The slot's row and head again, from a lane id the compiler cannot
  // match with the one above, so they are not kept (spilled) across the loop.
  const SlotRow sr = slot_row(fresh_lane_id(), wave, kvh, a.g, td.x, td.y, a.t);
  if (!sr.ok) return;
  const int ue = sr.u;
  if (a.n_splits > 1) {
    // Partial record: O unnormalised, then m and l; a row that saw no key
    // (l = 0) records the finite m of an empty part.
    write_record<T, D>(a, sr.row, sr.head, part, o, ue, l > 0.0f ? m_run : -1e30f, l);
    return;
  }
  store_output<T, D>(a, sr.row, sr.head, ue, o, l);
}

// --------------------------------------------------------------------------
// d = 256 and f32: one K/V chunk double-buffered in LDS, scored, then
// multiplied into O, one barrier per chunk.  O and Q take 192 VGPRs at
// d = 256 (Q alone 64 in f32), which leaves no room for a second score tile.
template <typename T, int D>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_kernel_seq(AttnArgs a) {
  using F = Frag<T, D>;
  constexpr int BN = F::BN;
  constexpr int NT = kAttnWaves * 64;
  constexpr int VEC = F::VEC;
  constexpr int RS = D + F::PAD;    // LDS row stride (elements) of the K tile
  constexpr int RSV = D + F::VPAD;  // LDS row stride of the V tile
  constexpr int TILE = BN * RS + BN * RSV;  // one K tile then one V tile
  constexpr int NKT = BN / 32;    // 32-key sub-tiles per key tile
  constexpr int NDT = D / 32;     // 32-wide slices of the head dim
  constexpr int NLD = BN * D / VEC / NT;  // 16-byte loads per thread per tensor
  static_assert(BN * D / VEC % NT == 0, "tile loads must split evenly");
  typedef typename F::Vec Vec;
  using P = typename F::P;
  __shared__ __align__(16) T smem[2 * TILE];

  cev_plan_header ph;
  if (!plan_ok(a, ph)) {
    poison_output<T, D>(a);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, u = lane >> 5;
  const int kvh = blockIdx.x % a.hkv;
  const int item = blockIdx.x / a.hkv;
  const int tile = item / a.n_splits, part = item % a.n_splits;
  const int4* tdp = (const int4*)(a.plan + ph.tiles_off) + 2 * tile;
  const int4 td = tdp[0];
  const int n_chunks = tdp[1].x;
  const int4* segs = (const int4*)(a.plan + ph.segs_off) + td.z;
  const int nseg = td.w;
  const int4* rows = (const int4*)(a.plan + ph.rows_off);
  // Query slot (wave, n) holds row slot / g of the tile, query head slot % g:
  // the valid rows of a short tile fill the first waves, and a wave with no
  // valid row skips the MFMA work (it still helps stage K/V).
  const int slot = wave * 32 + n;
  const int gi = slot % a.g;
  const int head = kvh * a.g + gi;
  const int rit = slot / a.g;
  const bool row_ok = rit < td.y && td.x + rit < a.t;
  const int row = row_ok ? td.x + rit : 0;
  const bool wave_active = (wave * 32) / a.g < td.y;
  const float c = a.scale_log2;

  F fr;
  fr.load_q((const T*)a.q + (int64_t)row * a.q_st + (int64_t)head * a.q_sh, row_ok, u);
  int4 rv = rows[row];
  if (!row_ok) rv = make_int4(0, 0, -1, 0);

  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
  float m_run = -1e30f, l_run = 0.0f;

  // ---- this part's slice of the tile's key stream: chunks [c0, c1)
  const int c0 = (int)((int64_t)part * n_chunks / a.n_splits);
  const int c1 = (int)((int64_t)(part + 1) * n_chunks / a.n_splits);
  ChunkCursor<BN> cursor{segs, nseg, a.s_cache, a.t, 0, 0, make_int4(0, 0, 0, 0)};
  cursor.seek(c0);
  KvSource<T> kvs;
  kvs.init(a, kvh);
  Vec kreg[NLD], vreg[NLD];
  auto load = [&](const Chunk& ch) { load_chunk<T, D, NLD, NT, Vec>(kvs, ch, tid, kreg, vreg); };
  auto store = [&](int buf) {
    T* sk = smem + buf * TILE;
    T* sv = sk + BN * RS;
#pragma unroll
    for (int r = 0; r < NLD; ++r) {
      const int v = tid + r * NT;
      const int key = v / (D / VEC), col = (v % (D / VEC)) * VEC;
      *(Vec*)&sk[key * RS + col] = kreg[r];
      *(Vec*)&sv[key * RSV + col] = vreg[r];
    }
  };

  const int my_chunks = c1 - c0;
  if (my_chunks > 0 && cursor.valid()) {
    Chunk ch = cursor.here();
    load(ch);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int ci = 0;; ++ci) {
      const bool more = ci + 1 < my_chunks;
      Chunk chn{0, 0, 0};
      if (more) {
        cursor.next();
        chn = cursor.here();
        load(chn);  // in flight while this chunk is scored
      }
      const T* sK = smem + buf * TILE;
      const T* sV = sK + BN * RS;
      const int key0 = ch.key0;
      const int nvalid = ch.nvalid;

      if (wave_active) {
        f32x16 s[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
          s[kt] = f32x16{};
#pragma unroll
          for (int st = 0; st < F::NQK; ++st) fr.template qk_step<RS>(sK, kt, st, n, u, s[kt]);
        }
        if (ch.local != 0 || nvalid < BN) {
          // Branch-free on purpose: a short-circuit && / || here gives every
          // element its own control flow, and hipcc 7.2 then reuses the
          // score register of element 0 for `key` and drops its select.
          const bool all_rows = ch.local == 0;
#pragma unroll
          for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int kk = kt * 32 + 8 * (i >> 2) + 4 * u + (i & 3);
              const int key = key0 + kk;
              const bool vis = (kk < nvalid) & (all_rows | ((key >= rv.x) & (key < rv.y)) | (key == rv.z));
              s[kt][i] = vis ? s[kt][i] : -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][i]);
        const float m_cand = pair_max(mx) * c;
        const bool grow = m_cand > m_run + kRescale;
        if (__ballot(grow)) {
          const float m_new = grow ? m_cand : m_run;
          const float alpha = fast_exp2(m_run - m_new);
          m_run = m_new;
          l_run *= alpha;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
        }
        float rs = 0.0f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
          for (int i = 0; i < 16; ++i) s[kt][i] = fast_exp2(__builtin_fmaf(s[kt][i], c, -m_run));
          P p;
          F::make_p(s[kt], p, rs);
#pragma unroll
          for (int j = 0; j < F::NPV; ++j) fr.template pv_step<RSV>(sV, kt, j, lane, u, p, o);
        }
        l_run += rs;
      }

      if (!more) break;
      store(buf ^ 1);  // that buffer was last read before the previous barrier
      __syncthreads();
      buf ^= 1;
      ch = chn;
    }
  }

  const float l = pair_sum(l_run);
  if (!row_ok) return;
  if (a.n_splits > 1) {
    // Partial record: O unnormalised, then m and l.
    write_record<T, D>(a, row, head, part, o, u, m_run, l);
    return;
  }
  store_output<T, D>(a, row, head, u, o, l);
}

// --------------------------------------------------------------------------
// bf16, d = 256: the sequential chunk body of attn_kernel_seq (score, softmax,
// then multiply into O) fed the way attn_kernel_pipe is fed.  32-key chunks
// go from HBM straight into a ring of kBuf LDS buffers (buffer_load ... lds),
// fetched kAhead chunks ahead of the one being scored, so no register holds
// staged K/V and a chunk has two chunk bodies to land (the body before its
// own reads its first K fragments) instead of none.  Rows are 512 bytes,
// unpadded, with the 16-byte column blocks permuted for conflict-free
// operand reads:
//   K: block c of row r at slot c ^ (r & 15)     (ds_read_b128, one key row
//      per lane: 16 rows cover every bank once)
//   V: block c of row r at slot c ^ 4(r & 3)     (ds_read_b64_tr_b16, four
//      rows x four blocks per 16 lanes)
// Bit 4 of a block index is never permuted, so the operand read addresses
// of the upper 128 head-dim values are the lower ones' plus 256 bytes.
namespace wide {
constexpr int kBuf = 4;
constexpr int kAhead = kBuf - 1;
constexpr int kKeys = 32;                      // keys per chunk
constexpr int kRowBytes = 512;                 // one bf16 row of d = 256
constexpr int kTileBytes = kKeys * kRowBytes;  // K (or V) of one chunk
constexpr int kVBase = kBuf * kTileBytes;      // the K tiles, then the V tiles
constexpr int kLoadsPerChunk = 4;              // buffer_load ... lds per wave per chunk
constexpr int kKPF = 3;                        // K fragments read ahead of their MFMA
constexpr int kVPF = 3;                        // V fragments read ahead of their MFMA
static_assert(kAttnWaves * 4 == kKeys, "each wave fetches four K rows and four V rows");

__device__ __forceinline__ int k_slot(int blk, int row) { return blk ^ (row & 15); }
__device__ __forceinline__ int v_slot(int blk, int row) { return blk ^ ((row & 3) << 2); }

// lgkmcnt of QK unit st (16 units, K reads kKPF ahead) and PV unit j (16
// units, two reads per V fragment, kVPF fragments ahead; the last kKPF units
// also issue the next chunk's first K reads): the LDS reads issued after
// the one the unit needs.  The PV counts replay one body's issue order.
constexpr int wait_k(int st) { return (15 - st) < kKPF - 1 ? 15 - st : kKPF - 1; }
struct PvWaits {
  int w[16];
};
constexpr PvWaits pv_waits() {
  PvWaits r{};
  int vhi[16] = {};
  int pos = 0;
  for (int j = 0; j < kVPF; ++j) {
    vhi[j] = pos + 1;
    pos += 2;
  }
  for (int j = 0; j < 16; ++j) {
    r.w[j] = pos - vhi[j] - 1;
    if (j + kVPF < 16) {
      vhi[j + kVPF] = pos + 1;
      pos += 2;
    }
    if (j >= 16 - kKPF) ++pos;
  }
  return r;
}
constexpr PvWaits kPvWaits = pv_waits();
constexpr int wait_v(int j) { return kPvWaits.w[j]; }
constexpr bool pv_waits_ok() {
  for (int j = 0; j < 16; ++j)
    if (kPvWaits.w[j] < 0 || kPvWaits.w[j] > 15) return false;
  return true;
}
static_assert(pv_waits_ok(), "lgkmcnt range");
static_assert(kVPF == 3 && kKPF == 3 ? (wait_v(0) == 4 && wait_v(12) == 4 && wait_v(13) == 4 && wait_v(14) == 3 && wait_v(15) == 2) : true,
              "wait counts at three fragments ahead");
}  // namespace wide

template <typename T, int D>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_kernel_wide(AttnArgs a) {
  using F = Frag<T, D>;
  using P = typename F::P;
  static_assert(sizeof(T) == 2 && D == 256 && F::BN == wide::kKeys && kAttnWaves == 8, "sized for bf16, d = 256");
  static_assert(F::NQK == 16 && F::NPV == 16, "unit layout below");
  using namespace wide;
  using pipe::i32x2;
  using pipe::KFrag;
  constexpr int NDT = D / 32;
  __shared__ __align__(16) char lds[2 * kBuf * kTileBytes];

  cev_plan_header ph;
  if (!plan_ok(a, ph)) {
    poison_output<T, D>(a);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform_i32(tid >> 6);
  const int n = lane & 31, u = lane >> 5;
  const int kvh = blockIdx.x % a.hkv;
  const int item = blockIdx.x / a.hkv;
  const int tile = item / a.n_splits, part = item % a.n_splits;
  const int4* tdp = (const int4*)(a.plan + ph.tiles_off) + 2 * tile;
  const int4 td = tdp[0];
  const int n_chunks = tdp[1].x;
  const int4* segs = (const int4*)(a.plan + ph.segs_off) + td.z;
  const int nseg = td.w;
  const int4* rows = (const int4*)(a.plan + ph.rows_off);
  // Query slot (wave, n) holds row slot / g of the tile, query head slot % g;
  // a wave with no valid row skips the MFMA work and still fetches its rows.
  const SlotRow sr0 = slot_row(lane, wave, kvh, a.g, td.x, td.y, a.t);
  const bool row_ok = sr0.ok;
  const int row = sr0.row, head = sr0.head;
  const bool wave_active = (wave * 32) / a.g < td.y;

  // Q arrives scaled by scale * log2 e (scores in base-2 units), and each
  // chunk's scores start from -m_run: exp2 is the whole softmax step per
  // score (the d = 128 loop's scheme, attn_kernel_pipe).
  F fr;
  fr.load_q((const T*)a.q + (int64_t)row * a.q_st + (int64_t)head * a.q_sh, row_ok, u);
  fr.scale_q(a.scale_log2);
  int4 rv = rows[row];
  if (!row_ok) rv = make_int4(0, 0, -1, 0);

  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
  // m_set: this row has seen a visible key, and m_run is a max it reached
  // (0 until then); rows that never see one keep l = 0.
  float m_run = 0.0f, l_run = 0.0f;
  bool m_set = false;

  const int c0 = (int)((int64_t)part * n_chunks / a.n_splits);
  const int c1 = (int)((int64_t)(part + 1) * n_chunks / a.n_splits);
  const int nc = c1 - c0;
  ChunkCursor<kKeys> cursor{segs, nseg, a.s_cache, a.t, 0, 0, make_int4(0, 0, 0, 0)};
  cursor.seek(c0);
  if (nc > 0 && cursor.valid()) {
    KvSource<T> kvs;
    kvs.init(a, kvh);

    // Per-lane byte offsets of the operand reads (V's include kVBase), for
    // head-dim blocks 0..15; the upper half adds 256 bytes as an immediate,
    // and so do the buffer and key row, so every offset field stays below
    // 64 KB.
    int koff[8], voff[4];
#pragma unroll
    for (int st = 0; st < 8; ++st) koff[st] = n * kRowBytes + (k_slot(2 * st + u, n) << 4);
    {
      const int i = lane & 15, g16 = (lane >> 4) & 1, rr = i >> 2;
      const int blk = 2 * g16 + ((i & 3) >> 1);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) voff[dt] = kVBase + (4 * u + rr) * kRowBytes + (v_slot(4 * dt + blk, rr) << 4) + 8 * (i & 1);
    }
    const int lds_base = (int)(size_t)(const __attribute__((address_space(3))) char*)lds;
    // K fragment st (head-dim values 16 st + 8u ..) of the chunk in buffer BUF.
    auto k_issue = [&](auto buf_c, auto st_c) {
      constexpr int BUF = decltype(buf_c)::value, ST = decltype(st_c)::value;
      return pipe::read_b128<BUF * kTileBytes + 256 * (ST >> 3)>(lds_base + koff[ST & 7]);
    };
    // V^T fragment j (keys 16 (j / 8) .., head-dim slice j % 8): the transpose
    // reads of rows r and r + 8.
    struct VFrag {
      i32x2 lo, hi;
    };
    auto v_issue = [&](auto buf_c, auto j_c) {
      constexpr int BUF = decltype(buf_c)::value, J = decltype(j_c)::value;
      constexpr int OFF = BUF * kTileBytes + 16 * (J / NDT) * kRowBytes + 256 * ((J % NDT) >> 2);
      const int va = lds_base + voff[(J % NDT) & 3];
      return VFrag{pipe::read_tr<OFF>(va), pipe::read_tr<OFF + 8 * kRowBytes>(va)};
    };

    // Chunk ch into buffer buf: wave w fetches K and V rows 4w .. 4w + 3, two
    // rows (1 KB) per instruction; rows past the chunk's last valid key read
    // as zero.
    auto fetch = [&](const Chunk& ch, int buf) {
      __amdgpu_buffer_rsrc_t rk, rvs;
      int kr, vr;
      kvs.rsrc(ch, rk, rvs, kr, vr);
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int krow = 4 * wave + 2 * r + (lane >> 5), blk = lane & 31;
        const int kdst = buf * kTileBytes + (4 * wave + 2 * r) * kRowBytes;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(lds + kdst), 16,
                                                 krow * kr + (k_slot(blk, krow) << 4), 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rvs, (__attribute__((address_space(3))) void*)(lds + kVBase + kdst), 16,
                                                 krow * vr + (v_slot(blk, krow) << 4), 0, 0, 0);
      }
    };

    // Stale LDS must hold finite values (a masked key's V row is multiplied
    // by p = 0): zero every buffer once, waiting for LDS writes only.
    for (int i = tid; i < 2 * kBuf * kTileBytes / 16; i += kAttnWaves * 64) *(f32x4*)(lds + 16 * i) = f32x4{};
    pipe::lds_barrier();

    int produced = 0;
    auto next_chunk = [&]() {
      Chunk ch{0, 0, 0};
      if (produced < nc) {
        if (produced > 0) cursor.next();
        ch = cursor.here();
      }
      ++produced;
      return ch;
    };
    Chunk chs[kAhead + 1];
#pragma unroll
    for (int k = 0; k < kAhead; ++k) {
      chs[k] = next_chunk();
      fetch(chs[k], k);
    }
    pipe::wait_vmcnt<kLoadsPerChunk * (kAhead - 2)>();  // chunks 0 and 1 landed
    __builtin_amdgcn_s_barrier();
    using I0 = std::integral_constant<int, 0>;
    // K reads in flight into the next body: the first body's are issued
    // here, every later body's in the previous body's last P.V units.
    KFrag kf[kKPF];
    if (wave_active) static_for<kKPF>([&](auto f_c) { kf[decltype(f_c)::value] = k_issue(I0{}, f_c); });

    // Iteration i scores the chunk in buffer B (chunk i of the part), after
    // fetching chunk i + kAhead into the buffer chunk i - 1 used; before its
    // barrier it waits for chunk i + 2 to land (the next iteration reads
    // chunk i + 2's first K fragments).
    auto step = [&](auto buf_tag) {
      constexpr int B = decltype(buf_tag)::value;
      using B_c = std::integral_constant<int, B>;
      chs[kAhead] = next_chunk();
      fetch(chs[kAhead], (B + kAhead) % kBuf);
      const Chunk ch = chs[0];
      if (wave_active) {
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = -m_run;
        static_for<F::NQK>([&](auto st_c) {
          constexpr int st = decltype(st_c)::value;
          pipe::wait_b128<wait_k(st)>(kf[st % kKPF]);
          fr.qk_mfma(__builtin_bit_cast(bf16x8, kf[st % kKPF]), st, s);
          if constexpr (st + kKPF < F::NQK) kf[st % kKPF] = k_issue(B_c{}, std::integral_constant<int, st + kKPF>{});
        });
        // the first V fragments load under the softmax
        VFrag vf[kVPF];
        static_for<kVPF>([&](auto j_c) { vf[decltype(j_c)::value] = v_issue(B_c{}, j_c); });
        if (ch.local != 0 || ch.nvalid < kKeys) {
          // Branch-free on purpose (see attn_kernel_seq).
          const bool all_rows = ch.local == 0;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = 8 * (i >> 2) + 4 * u + (i & 3);
            const int key = ch.key0 + kk;
            const bool vis = (kk < ch.nvalid) & (all_rows | ((key >= rv.x) & (key < rv.y)) | (key == rv.z));
            s[i] = vis ? s[i] : -INFINITY;
          }
        }
        // The max moves lazily (the d = 128 loop's scheme, checked on the
        // scores): P is made relative to m_run as long as no score of the
        // lane exceeds it by more than log2(kMaxP), so p < kMaxP.  Otherwise,
        // or for a row with no max yet, the row takes its max (a set row
        // only when it grew by more than kRescale) and the scores move by it
        // before P is made.  The check keeps no copy of the scores, so the
        // loop needs no more registers than with a per-chunk max.
        float ml = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) ml = fmaxf(ml, s[i]);
        if (__ballot((ml > kLog2MaxP) | !m_set)) {
          const float delta = pair_max(ml);
          const bool move = m_set ? delta > kRescale : delta > -INFINITY;
          const float dm = move ? delta : 0.0f;
          const float alpha = m_set ? fast_exp2(-dm) : 1.0f;
          m_set = m_set | move;
          m_run += dm;
          l_run *= alpha;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) s[i] -= dm;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = fast_exp2(s[i]);
        P p;
        float rs = 0.0f;
        F::make_p(s, p, rs);
        static_for<F::NPV>([&](auto j_c) {
          constexpr int j = decltype(j_c)::value;
          VFrag& f = vf[j % kVPF];
          pipe::wait_tr<wait_v(j)>(f.lo, f.hi);
          const bf16x4 lo = __builtin_bit_cast(bf16x4, f.lo), hi = __builtin_bit_cast(bf16x4, f.hi);
          F::pv_mfma(bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, j, p, o);
          if constexpr (j + kVPF < F::NPV) f = v_issue(B_c{}, std::integral_constant<int, j + kVPF>{});
          // the next body's first K reads (chunk i + 1, landed before the
          // previous barrier; past the part's end they read a stale buffer
          // and are never used)
          if constexpr (j >= F::NPV - kKPF)
            kf[j - (F::NPV - kKPF)] = k_issue(std::integral_constant<int, (B + 1) % kBuf>{}, std::integral_constant<int, j - (F::NPV - kKPF)>{});
        });
        l_run += rs;
      }
      pipe::wait_vmcnt<kLoadsPerChunk * (kAhead - 2)>();  // chunk i + 2 landed
      __builtin_amdgcn_s_barrier();
#pragma unroll
      for (int k = 0; k < kAhead; ++k) chs[k] = chs[k + 1];
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    static_assert(kBuf == 4, "the unrolled loop below walks four buffers");
    for (int ci = 0; ci < nc; ci += kBuf) {
      step(I0{});
      if (ci + 1 >= nc) break;
      step(I1{});
      if (ci + 2 >= nc) break;
      step(I2{});
      if (ci + 3 >= nc) break;
      step(I3{});
    }
    // Fetches past the part's end read no memory but still write zeros into
    // LDS: drain them before the workgroup exits.
    pipe::wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  const float l = pair_sum(l_run);
  // The slot's row and head again, from a lane id the compiler cannot
  // match with the one above, so they are not kept (spilled) across the loop.
  const SlotRow sr = slot_row(fresh_lane_id(), wave, kvh, a.g, td.x, td.y, a.t);
  if (!sr.ok) return;
  const int ue = sr.u;
  if (a.n_splits > 1) {
    // a row that saw no key (l = 0) records the finite m of an empty part
    write_record<T, D>(a, sr.row, sr.head, part, o, ue, l > 0.0f ? m_run : -1e30f, l);
    return;
  }
  store_output<T, D>(a, sr.row, sr.head, ue, o, l);
}

// Combines the parts of split tiles: for each (row, head),
//   M = max_s m_s,  L = sum_s 2^(m_s - M) l_s,  O = sum_s 2^(m_s - M) O_s / L.
// One wave per (row, head), kMergeWaves per workgroup.  Lane l reads the
// head-dim columns E (l % Q) .. +E-1 (E values per lane, Q = D / E lanes
// per record) of every (64 / Q)-th part starting at part l / Q; a batch of
// NB parts per lane is loaded before any of it is used, so a batch costs one
// memory latency, and batches combine with an online rescale.  The launcher
// picks NB from the part count (fewer registers, more waves per SIMD for
// few parts).
// When the plan's tiles cover every row once (rows_dense), workgroups map to
// rows directly and the record and gate loads go out beside the header load:
// they only touch the workspace and gate extents the launcher checked, and
// nothing is stored before the header has passed.  Otherwise a workgroup
// finds its rows through the tile table after the header check.
constexpr int kMergeWaves = 4;

// Values per lane access: 16 bytes (8 bf16) at d = 128, where a wave reads
// four parts side by side (the 32k-prefix x 16-token shape's 32 parts: 42.5
// / 42.9 us against 44.5 / 43.7 us with 8-byte lanes); 4 values otherwise.
// At d = 256 the 16-byte form put two parts in a wave, read each gate chunk
// twice and left half the wave idle at the end: c5a's K2 measured 148.0 /
// 148.3 against 142.5 / 142.9 us.
template <typename T, int D>
struct MergeShape {
  static constexpr int E = (sizeof(T) == 2 && D == 128) ? 8 : 4;
  static constexpr int Q = D / E;    // lanes per record
  static constexpr int PS = 64 / Q;  // parts read side by side
  static_assert(Q * PS == 64, "one wave covers the head dim");
};

// Max over the PS part phases of a wave (lanes Q = 64 / PS apart); the
// lanes of one phase hold the same parts, so they agree already.
template <int PS>
__device__ __forceinline__ float phase_max(float x) {
  static_assert(PS == 1 || PS == 2 || PS == 4, "part phases 16 or 32 lanes apart");
  if constexpr (PS == 4) x = pair16_max(x);
  if constexpr (PS >= 2) x = pair_max(x);
  return x;
}

template <typename T, int D, int NB>
__global__ __launch_bounds__(kMergeWaves * 64) void attn_merge_kernel(AttnArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  using MS = MergeShape<T, D>;
  constexpr int E = MS::E, Q = MS::Q, PS = MS::PS;
  using VE = VecN<T, E>;
  cev_plan_header ph;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int head = blockIdx.x % a.hq;
  int row;
  if (a.rows_dense) {
    // The header goes through vector loads (a lane offset the compiler
    // cannot fold), so no wait for a later kernel argument's scalar load
    // also waits for it.
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    const int4* hp = (const int4*)a.plan + zero;
    int4 hw[sizeof(cev_plan_header) / 16];
#pragma unroll
    for (int i = 0; i < (int)(sizeof(cev_plan_header) / 16); ++i) hw[i] = hp[i];
    __builtin_memcpy(&ph, hw, sizeof ph);
    // blockIdx -> (row group of kMergeWaves rows, head)
    row = (blockIdx.x / a.hq) * kMergeWaves + wave;
    if (row >= a.t) return;
  } else {
    ph = *(const cev_plan_header*)a.plan;
    if (!header_ok(a, ph)) return;
    // blockIdx -> (tile, row group of kMergeWaves rows, head)
    const int tile_rows = a.tile_rows;  // validated against the plan at launch
    const int groups = (tile_rows + kMergeWaves - 1) / kMergeWaves;
    const int grp = (blockIdx.x / a.hq) % groups;
    const int tile = blockIdx.x / (a.hq * groups);
    const int4 td = ((const int4*)(a.plan + ph.tiles_off))[2 * tile];
    const int r = grp * kMergeWaves + wave;
    if ((r >= td.y) | (td.x + r >= a.t)) return;
    row = td.x + r;
  }
  const int S = a.n_splits;
  const int col = lane % Q, phase = lane / Q;
  const int64_t i0 = record_index(a, row, head, 0);
  const T* rec = record_out<T, D>(a, i0);
  const float2* rml = record_ml<T, D>(a) + i0;
  // The gate chunk loads with the first records (from a record when there
  // is no gate, and is then unused), not after the merge.
  const int d = E * col;
  const T* gp = a.has_gate ? (const T*)a.gate + (int64_t)row * a.g_st + (int64_t)head * a.g_sh + d : rec;
  const VE graw = *(const VE*)gp;

  // Every record holds a finite m (a part with no visible key keeps its
  // initial -1e30 and l = 0), so M is finite after the first batch.
  float M = -INFINITY, L = 0.0f;
  float acc[E] = {};
  for (int s0 = 0; s0 < S; s0 += PS * NB) {
    // Every load of the batch is issued before any is used: parts past S
    // read part S - 1 again and are dropped by the selects below (no
    // per-part branch, so no wait between the loads).
    VE raw[NB];
    float2 ml[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int s = min(s0 + PS * i + phase, S - 1);
      raw[i] = *(const VE*)(rec + (int64_t)s * D + d);
      ml[i] = rml[s];
    }
    bool ok[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      ok[i] = s0 + PS * i + phase < S;
      if (!ok[i]) ml[i] = make_float2(-INFINITY, 0.0f);
    }
    float mb = -INFINITY;
#pragma unroll
    for (int i = 0; i < NB; ++i) mb = fmaxf(mb, ml[i].x);
    const float m_new = fmaxf(M, phase_max<PS>(mb));
    const float alpha = fast_exp2(M - m_new);
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] *= alpha;
    L *= alpha;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const float w = fast_exp2(ml[i].x - m_new);  // 0 for a dropped part
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] += w * (ok[i] ? (float)raw[i][e] : 0.0f);
      L += w * ml[i].y;
    }
    M = m_new;
  }
  if (a.rows_dense) {
    // The header is checked only now, so its loads and the record loads
    // are in flight together.  The empty asm keeps the loads and the
    // combine ahead of the check (a plain branch would let the compiler
    // sink them behind it).
    asm volatile("" ::"v"(L), "v"(acc[0]), "v"(acc[E - 1]), "v"(graw));
    if (!header_ok(a, ph)) return;
  }
  // The PS part phases of one column group sit Q lanes apart: sum them
  // with lane swaps on the VALU (lane ^ 16, then lane ^ 32).
  static_assert(PS == 1 || PS == 2 || PS == 4, "part phases 16 or 32 lanes apart");
  if constexpr (PS == 4) {
    L = pair16_sum(L);
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = pair16_sum(acc[e]);
  }
  if constexpr (PS >= 2) {
    L = pair_sum(L);
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = pair_sum(acc[e]);
  }
  if (phase != 0) return;
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  T* op = (T*)a.out + (int64_t)row * a.o_st + (int64_t)head * a.o_sh + d;
  VE v;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    float x = BF ? acc[e] * inv : (L > 0.0f ? acc[e] / L : 0.0f);
    if (a.has_gate) x = gate_value(x, (float)graw[e], BF);
    v[e] = (T)x;
  }
  *(VE*)op = v;
}

// stagger: the bf16 d = 128 loop's form (attn_kernel_pipe's STAG).
template <typename T, int D>
int32_t launch(const AttnArgs& a, bool stagger, hipStream_t stream) {
  const int64_t grid = (int64_t)a.n_tiles * a.n_splits * a.hkv;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid);
  if constexpr (sizeof(T) == 2 && D == 128)
    hipLaunchKernelGGL((stagger ? attn_kernel_pipe<T, D, true> : attn_kernel_pipe<T, D, false>), dim3((unsigned)grid),
                       dim3(kAttnWaves * 64), 0, stream, a);
  else if constexpr (sizeof(T) == 2 && D == 256)
    hipLaunchKernelGGL((attn_kernel_wide<T, D>), dim3((unsigned)grid), dim3(kAttnWaves * 64), 0, stream, a);
  else
    hipLaunchKernelGGL((attn_kernel_seq<T, D>), dim3((unsigned)grid), dim3(kAttnWaves * 64), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "packed attention launch: %s", hipGetErrorString(e));
  if (a.n_splits > 1) {
    const int groups = (a.tile_rows + kMergeWaves - 1) / kMergeWaves;
    const int64_t mgrid = a.rows_dense ? (int64_t)((a.t + kMergeWaves - 1) / kMergeWaves) * a.hq : (int64_t)a.n_tiles * groups * a.hq;
    if (mgrid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "merge grid too large");
    constexpr int PS = MergeShape<T, D>::PS;
    const int per_lane = (a.n_splits + PS - 1) / PS;  // parts each lane reads
    if (per_lane <= 1)
      hipLaunchKernelGGL((attn_merge_kernel<T, D, 1>), dim3((unsigned)mgrid), dim3(kMergeWaves * 64), 0, stream, a);
    else if (per_lane <= 2)
      hipLaunchKernelGGL((attn_merge_kernel<T, D, 2>), dim3((unsigned)mgrid), dim3(kMergeWaves * 64), 0, stream, a);
    else if (per_lane <= 4)
      hipLaunchKernelGGL((attn_merge_kernel<T, D, 4>), dim3((unsigned)mgrid), dim3(kMergeWaves * 64), 0, stream, a);
    else if (per_lane <= 8)
      hipLaunchKernelGGL((attn_merge_kernel<T, D, 8>), dim3((unsigned)mgrid), dim3(kMergeWaves * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_merge_kernel<T, D, 16>), dim3((unsigned)mgrid), dim3(kMergeWaves * 64), 0, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "attention merge launch: %s", hipGetErrorString(e));
  }
  return CEV_OK;
}

}  // namespace

// Scratch of the allocation-free entry point: the split-KV partial records
// (f32 O, m, l per row, head and part).  Every record a merge reads is
// written by the same call first, so nothing in it has to start at zero.
// Each GPU the library runs on holds its own copy until the process ends.
constexpr size_t kScratchBytes = CEV_ATTN_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

// Validation and launch shared by both entry points.
int32_t packed_attention_impl(const cev_attn_desc* d, const void* plan_host, const void* plan_dev, const void* q, const void* k_cache,
                              const void* v_cache, const void* k_new, const void* v_new, const void* gate, void* out, void* workspace,
                              size_t workspace_bytes, cev_stream stream) {
  CEV_CHECK_ARG(d != nullptr, "cev_packed_attention: null descriptor");
  // The strides, scale and gate flag of this launch are checked here, not
  // only when the plan was built: they may change between calls.
  int32_t drc = cev_check_attn_desc(d);
  if (drc) return drc;
  CEV_CHECK_ARG(plan_host != nullptr && plan_dev != nullptr, "cev_packed_attention: null plan");
  const cev_plan_header* h = (const cev_plan_header*)plan_host;
  CEV_CHECK_ARG(h->magic == CEV_PLAN_MAGIC && h->version == CEV_PLAN_VERSION, "cev_packed_attention: not a plan");
  CEV_CHECK_ARG(h->t == d->t && h->s_cache == d->s_cache && h->dtype == d->dtype && h->head_dim == d->head_dim &&
                    h->n_q_heads == d->n_q_heads && h->n_kv_heads == d->n_kv_heads,
                "cev_packed_attention: plan was built for another descriptor");
  if (h->n_tiles == 0) return CEV_OK;
  CEV_CHECK_ARG(q && k_new && v_new && out, "cev_packed_attention: null q, k_new, v_new or out");
  CEV_CHECK_ARG(d->s_cache == 0 || (k_cache && v_cache), "cev_packed_attention: null cache with s_cache %d", d->s_cache);
  CEV_CHECK_ARG(!d->has_gate || gate, "cev_packed_attention: has_gate without a gate");
  const int g = d->n_q_heads / d->n_kv_heads;
  CEV_CHECK_ARG(h->tile_rows == cev_attn_tile_rows(g) && h->block_n == cev_attn_block_n(d->dtype, d->head_dim) && h->n_splits >= 1,
                "cev_packed_attention: plan tiling does not match this library");
  size_t need = 0;
  int32_t rc = cev_attn_workspace_size(plan_host, &need);
  if (rc) return rc;
  if (need > 0) {
    CEV_CHECK_ARG(workspace != nullptr, "cev_packed_attention: the plan splits tiles and needs a %zu-byte workspace", need);
    if (workspace_bytes < need) return cev_fail(CEV_ERR_SPACE, "workspace of %zu bytes, plan needs %zu", workspace_bytes, need);
  }
  const uintptr_t al = 15;
  CEV_CHECK_ARG((((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)out |
                  (uintptr_t)gate | (uintptr_t)plan_dev | (uintptr_t)workspace) & al) == 0,
                "cev_packed_attention: device buffers must be 16-byte aligned");
  AttnArgs a;
  a.q = q;
  a.kc = k_cache;
  a.vc = v_cache;
  a.kn = k_new;
  a.vn = v_new;
  a.gate = gate;
  a.out = out;
  a.ws = (char*)workspace;
  a.plan = (const int32_t*)plan_dev;
  a.q_st = d->q_stride_t;
  a.q_sh = d->q_stride_h;
  a.kc_ss = d->kc_stride_s;
  a.kc_sh = d->kc_stride_h;
  a.vc_ss = d->vc_stride_s;
  a.vc_sh = d->vc_stride_h;
  a.kn_st = d->kn_stride_t;
  a.kn_sh = d->kn_stride_h;
  a.vn_st = d->vn_stride_t;
  a.vn_sh = d->vn_stride_h;
  a.g_st = d->g_stride_t;
  a.g_sh = d->g_stride_h;
  a.o_st = d->o_stride_t;
  a.o_sh = d->o_stride_h;
  a.n_tiles = h->n_tiles;
  a.t = d->t;
  a.s_cache = d->s_cache;
  a.hq = d->n_q_heads;
  a.hkv = d->n_kv_heads;
  a.g = g;
  a.has_gate = d->has_gate;
  a.n_splits = h->n_splits;
  a.tile_rows = h->tile_rows;
  a.scale_log2 = d->scale * 1.4426950408889634f;
  a.plan_sig = (uint32_t)h->sig;
  const int32_t* words = (const int32_t*)plan_host;
  CEV_CHECK_ARG(h->tiles_off >= (int32_t)(sizeof(cev_plan_header) / 4) &&
                    (int64_t)h->tiles_off + 8 * (int64_t)h->n_tiles <= (int64_t)h->bytes / 4,
                "cev_packed_attention: the plan's tile table lies outside the plan");
  // Tiles that cover rows [0, t) in order, each row once, let the merge map
  // its workgroups straight to rows.
  int64_t next_row = 0;
  for (int32_t i = 0; i < h->n_tiles && next_row >= 0; ++i) {
    const int32_t r0 = words[h->tiles_off + 8 * (int64_t)i], nr = words[h->tiles_off + 8 * (int64_t)i + 1];
    next_row = (r0 == next_row && nr >= 1 && nr <= h->tile_rows) ? next_row + nr : -1;
  }
  a.rows_dense = next_row == d->t ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  if (d->dtype == CEV_BF16) {
    if (d->head_dim == 128) {
      // Staggered loop when some tile keeps more than half of the
      // workgroup's waves busy (more than 4 x 32 query slots).
      bool stagger = false;
      for (int32_t i = 0; i < h->n_tiles && !stagger; ++i)
        stagger = (int64_t)words[h->tiles_off + 8 * (int64_t)i + 1] * g > 32 * kAttnWaves / 2;
      return launch<__bf16, 128>(a, stagger, s);
    }
    return launch<__bf16, 256>(a, false, s);
  }
  return launch<float, 128>(a, false, s);
}

// Device addresses of `scratch` (below), one per device, looked up once with that
// device current.  The array's name in host code is only a stand-in for
// the symbol and is never passed to a kernel.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;
// Host threads inside cev_packed_attention_noalloc per device: a second
// thread that enters while another is launching on the same device is
// refused, since their launches would share the buffer.
std::atomic<int> g_scratch_users[kMaxDevices];

int32_t current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (*dev < 0 || *dev >= kMaxDevices) return cev_fail(CEV_ERR_UNSUPPORTED, "device %d beyond the %d the library tracks", *dev, kMaxDevices);
  return CEV_OK;
}

int32_t scratch_ptr(int dev, void** out) {
  hipError_t e;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) return cev_fail(CEV_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return CEV_OK;
}

}  // namespace

extern "C" int32_t cev_packed_attention(const cev_attn_desc* d, const void* plan_host, const void* plan_dev, const void* q,
                                        const void* k_cache, const void* v_cache, const void* k_new, const void* v_new, const void* gate,
                                        void* out, void* workspace, size_t workspace_bytes, cev_stream stream) {
  return packed_attention_impl(d, plan_host, plan_dev, q, k_cache, v_cache, k_new, v_new, gate, out, workspace, workspace_bytes, stream);
}

extern "C" int32_t cev_packed_attention_noalloc(const cev_attn_desc* d, const void* plan_host, const void* plan_dev, const void* q,
                                                const void* k_cache, const void* v_cache, const void* k_new, const void* v_new,
                                                const void* gate, void* out, cev_stream stream) {
  CEV_CHECK_ARG(plan_host != nullptr, "cev_packed_attention_noalloc: null plan");
  const cev_plan_header* h = (const cev_plan_header*)plan_host;
  CEV_CHECK_ARG(h->magic == CEV_PLAN_MAGIC && h->version == CEV_PLAN_VERSION, "cev_packed_attention_noalloc: not a plan");
  size_t need = 0;
  int32_t rc = cev_attn_workspace_size(plan_host, &need);
  if (rc) return rc;
  if (need > kScratchBytes)
    return cev_fail(CEV_ERR_SPACE, "cev_packed_attention_noalloc: the plan needs %zu bytes of split records, the static scratch holds %zu",
                    need, kScratchBytes);
  if (need == 0)
    return packed_attention_impl(d, plan_host, plan_dev, q, k_cache, v_cache, k_new, v_new, gate, out, nullptr, 0, stream);
  int dev = 0;
  rc = current_device(&dev);
  if (rc) return rc;
  if (g_scratch_users[dev].fetch_add(1, std::memory_order_acq_rel) != 0) {
    g_scratch_users[dev].fetch_sub(1, std::memory_order_acq_rel);
    return cev_fail(CEV_ERR_SPACE,
                    "cev_packed_attention_noalloc: another thread is launching on device %d's static scratch; calls that "
                    "share it must be serialised",
                    dev);
  }
  void* ws = nullptr;
  rc = scratch_ptr(dev, &ws);
  if (!rc) rc = packed_attention_impl(d, plan_host, plan_dev, q, k_cache, v_cache, k_new, v_new, gate, out, ws, kScratchBytes, stream);
  g_scratch_users[dev].fetch_sub(1, std::memory_order_acq_rel);
  return rc;
}
