// Packed-prefill attention for gfx950: the replacement for Attention::attend
// (crates/cev-model/src/qwen3.rs:206-220, crates/cev-model/src/qwen35.rs:563-579)
// with the block-offset table in place of the dense mask.
//
// Design (one workgroup = one tile of query rows x one KV head):
//   - the waves of a workgroup own 32 query rows of one query head each and
//     together cover every query head of the KV head's GQA group, so a K/V
//     key tile staged in LDS once is scored by g x rows queries;
//   - scores are computed transposed, S^T = K . Q^T, on 32x32 MFMA tiles: a
//     lane then holds 16 keys of ONE query row, and the softmax row max and
//     row sum reduce inside the lane plus one exchange with the lane 32 away;
//   - online softmax in base 2 (exp2 of q.k * scale * log2 e), f32 state;
//   - O^T = V^T . P^T accumulates on MFMA: P stays in registers as the B
//     operand (its K slots follow the S^T register order) and V is staged
//     transposed in LDS so each lane reads 4-key runs;
//   - the key ranges a tile visits come from the plan: spans are unmasked,
//     local keys are masked per row from the row's [lo, hi) + diag;
//   - blockIdx -> (tile, kv head) with the kv head fastest, so consecutive
//     workgroups (spread round-robin over the 8 XCDs) of one XCD share a KV
//     head and its K/V stream stays in that XCD's L2.
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
  const int32_t* plan;
  int64_t q_st, q_sh, kc_ss, kc_sh, vc_ss, vc_sh, kn_st, kn_sh, vn_st, vn_sh, g_st, g_sh, o_st, o_sh;
  int32_t n_tiles, t, s_cache, hkv, g, has_gate;
  float scale_log2;
};

// The plan header on the device must describe the launch; anything else
// (a plan not copied from the host plan) makes every workgroup exit.
__device__ __forceinline__ bool plan_ok(const AttnArgs& a) {
  const cev_plan_header* h = (const cev_plan_header*)a.plan;
  return h->magic == CEV_PLAN_MAGIC && h->n_tiles == a.n_tiles && h->t == a.t && h->s_cache == a.s_cache;
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
    float sg = bf16_round(1.0f / den);
    return bf16_round(bf16_round(o) * sg);
  }
  return o * (1.0f / (expf(-g) + 1.0f));
}

// --------------------------------------------------------------------------
// bf16: QK^T and PV on v_mfma_f32_32x32x16_bf16.
//
// Per key tile of BN keys (double-buffered in LDS, the next tile's global
// loads in flight while this one is scored):
//   S^T = K . Q^T                  16 x (D/16) MFMAs per wave
//   row max on raw scores          lane-local + one permlane32 swap
//   lazy rescale                   O and l are rescaled only when a row's max
//                                  grows by more than 2^kRescale, so
//                                  exp2(s*c - m) <= 2^kRescale in between
//   P = exp2(fma(s, c, -m))        c = scale * log2(e)
//   O^T += V^T . P^T               V stays key-major in LDS; the A operand
//                                  (4 keys x 1 head-dim column per read) comes
//                                  from ds_read_b64_tr_b16, the gfx950 LDS
//                                  transpose load.
constexpr float kRescale = 8.0f;
constexpr int kPad = 8;  // bf16 elements of padding per LDS row

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 lds_read_tr(const __bf16* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A position in a tile's key stream: segment si, key offset k0 within it.
struct Cursor {
  int si, k0;
};

template <int D, int BN>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_bf16_kernel(AttnArgs a) {
  constexpr int NT = kAttnWaves * 64;
  constexpr int RS = D + kPad;    // LDS row stride (elements) of K and V tiles
  constexpr int TILE = BN * RS;   // one K or V tile
  constexpr int NKT = BN / 32;    // 32-key sub-tiles per key tile
  constexpr int NDT = D / 32;     // 32-wide slices of the head dim
  constexpr int NQS = D / 16;     // K=16 steps over the head dim
  constexpr int NLD = BN * D / 8 / NT;  // 16-byte loads per thread per tensor
  static_assert(BN * D / 8 % NT == 0, "tile loads must split evenly");
  __shared__ __align__(16) __bf16 smem[2 * 2 * TILE];

  if (!plan_ok(a)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, u = lane >> 5;
  const int kvh = blockIdx.x % a.hkv;
  const int tile = blockIdx.x / a.hkv;
  const cev_plan_header* ph = (const cev_plan_header*)a.plan;
  const int4 td = ((const int4*)(a.plan + ph->tiles_off))[tile];
  const int4* segs = (const int4*)(a.plan + ph->segs_off) + td.z;
  const int nseg = td.w;
  const int4* rows = (const int4*)(a.plan + ph->rows_off);
  const int gi = wave % a.g, rg = wave / a.g;
  const int head = kvh * a.g + gi;
  const int rit = rg * 32 + n;
  const bool row_ok = rit < td.y && td.x + rit < a.t;
  const int row = row_ok ? td.x + rit : 0;
  const float c = a.scale_log2;

  bf16x8 qf[NQS];
  {
    const __bf16* qp = (const __bf16*)a.q + (int64_t)row * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
    for (int s = 0; s < NQS; ++s) {
      bf16x8 z = {};
      qf[s] = row_ok ? *(const bf16x8*)(qp + 16 * s + 8 * u) : z;
    }
  }
  int4 rv = rows[row];
  if (!row_ok) rv = make_int4(0, 0, -1, 0);

  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
  float m_run = -1e30f, l_run = 0.0f;

  // ---- key stream
  auto seg_of = [&](int si) { return clamp_seg(segs[si], a.s_cache, a.t); };
  auto first = [&](Cursor& cu) {
    cu.si = 0;
    cu.k0 = 0;
    while (cu.si < nseg) {
      const int4 sg = seg_of(cu.si);
      if (sg.y > sg.x) return;
      ++cu.si;
    }
  };
  auto advance = [&](Cursor& cu) {
    const int4 sg = seg_of(cu.si);
    cu.k0 += BN;
    if (sg.x + cu.k0 < sg.y) return;
    cu.k0 = 0;
    for (++cu.si; cu.si < nseg; ++cu.si) {
      const int4 s2 = seg_of(cu.si);
      if (s2.y > s2.x) return;
    }
  };
  bf16x8 kreg[NLD], vreg[NLD];
  auto load = [&](const Cursor& cu) {
    const int4 sg = seg_of(cu.si);
    const int key0 = sg.x + cu.k0;
    const int nvalid = min(BN, sg.y - key0);
    const bool cached = key0 < a.s_cache;
    const __bf16* kb = cached ? (const __bf16*)a.kc + kvh * a.kc_sh + (int64_t)key0 * a.kc_ss
                              : (const __bf16*)a.kn + kvh * a.kn_sh + (int64_t)(key0 - a.s_cache) * a.kn_st;
    const __bf16* vb = cached ? (const __bf16*)a.vc + kvh * a.vc_sh + (int64_t)key0 * a.vc_ss
                              : (const __bf16*)a.vn + kvh * a.vn_sh + (int64_t)(key0 - a.s_cache) * a.vn_st;
    const int64_t ks = cached ? a.kc_ss : a.kn_st;
    const int64_t vs = cached ? a.vc_ss : a.vn_st;
#pragma unroll
    for (int r = 0; r < NLD; ++r) {
      const int v = tid + r * NT;
      const int key = v / (D / 8), col = (v % (D / 8)) * 8;
      bf16x8 x = {}, y = {};
      if (key < nvalid) {
        x = *(const bf16x8*)(kb + (int64_t)key * ks + col);
        y = *(const bf16x8*)(vb + (int64_t)key * vs + col);
      }
      kreg[r] = x;
      vreg[r] = y;
    }
  };
  auto store = [&](int buf) {
    __bf16* sk = smem + buf * 2 * TILE;
#pragma unroll
    for (int r = 0; r < NLD; ++r) {
      const int v = tid + r * NT;
      const int key = v / (D / 8), col = (v % (D / 8)) * 8;
      *(bf16x8*)&sk[key * RS + col] = kreg[r];
      *(bf16x8*)&sk[TILE + key * RS + col] = vreg[r];
    }
  };

  Cursor cur;
  first(cur);
  if (cur.si < nseg) {
    load(cur);
    store(0);
    __syncthreads();
    int buf = 0;
    for (;;) {
      Cursor nxt = cur;
      advance(nxt);
      const bool more = nxt.si < nseg;
      if (more) load(nxt);  // in flight while this tile is scored

      const __bf16* sK = smem + buf * 2 * TILE;
      const __bf16* sV = sK + TILE;
      const int4 sg = seg_of(cur.si);
      const int key0 = sg.x + cur.k0;
      const int nvalid = min(BN, sg.y - key0);

      f32x16 s[NKT];
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        s[kt] = f32x16{};
#pragma unroll
        for (int st = 0; st < NQS; ++st) {
          const bf16x8 af = *(const bf16x8*)&sK[(kt * 32 + n) * RS + 16 * st + 8 * u];
          s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[st], s[kt], 0, 0, 0);
        }
      }
      if (sg.z != 0 || nvalid < BN) {
        // Branch-free on purpose: a short-circuit && / || here gives every
        // element its own control flow, and hipcc 7.2 then reuses the score
        // register of element 0 for `key` and drops its select.
        const bool all_rows = sg.z == 0;
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
      // P as bf16 B operands: K slot 8u + j of half h holds S^T register
      // 8h + j, i.e. key 16h + 8(j/4) + 4u + j%4 of the sub-tile.
      bf16x8 pf[NKT][2];
      float rs = 0.0f;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float p = fast_exp2(__builtin_fmaf(s[kt][8 * h + j], c, -m_run));
            rs += p;
            pf[kt][h][j] = (__bf16)p;
          }
      l_run += rs;
      // O^T += V^T . P^T.  Lane (group g16 = lane/16, i = lane%16) reads row
      // key0' + (i/4), columns d0 + 4(i%4) .. +3; the transpose load hands it
      // 4 consecutive keys of head-dim column d0 + i.
      const int tr_row = (lane & 15) >> 2;
      const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const __bf16* vp = sV + (kt * 32 + 16 * h + 4 * u + tr_row) * RS + dt * 32 + tr_col;
            const bf16x4 lo = lds_read_tr(vp);
            const bf16x4 hi = lds_read_tr(vp + 8 * RS);
            const bf16x8 af = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, pf[kt][h], o[dt], 0, 0, 0);
          }

      if (!more) break;
      store(buf ^ 1);  // that buffer was last read before the previous barrier
      __syncthreads();
      buf ^= 1;
      cur = nxt;
    }
  }

  const float l = pair_sum(l_run);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (!row_ok) return;
  __bf16* op = (__bf16*)a.out + (int64_t)row * a.o_st + (int64_t)head * a.o_sh;
  const __bf16* gp = a.has_gate ? (const __bf16*)a.gate + (int64_t)row * a.g_st + (int64_t)head * a.g_sh : nullptr;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = dt * 32 + 8 * q4 + 4 * u;
      bf16x4 r;
      bf16x4 gv = {};
      if (gp) gv = *(const bf16x4*)(gp + d);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = o[dt][4 * q4 + e] * inv;
        if (gp) x = gate_value(x, (float)gv[e], true);
        r[e] = (__bf16)x;
      }
      *(bf16x4*)(op + d) = r;
    }
}

// --------------------------------------------------------------------------
// f32: QK^T and PV on v_mfma_f32_32x32x2_f32 (full f32 products).
// The head-dim order of the QK^T K slots is permuted (d = 8k + 4u + r) so a
// lane reads 4 consecutive floats for 4 steps; V stays key-major in LDS.
template <int D, int BN>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_f32_kernel(AttnArgs a) {
  constexpr int NT = kAttnWaves * 64;
  constexpr int KS = D + 4;
  constexpr int NKT = BN / 32;
  constexpr int NDT = D / 32;
  constexpr int NQ4 = D / 8;
  __shared__ __align__(16) float sK[BN * KS];
  __shared__ __align__(16) float sV[BN * KS];

  if (!plan_ok(a)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, u = lane >> 5;
  const int kvh = blockIdx.x % a.hkv;
  const int tile = blockIdx.x / a.hkv;
  const cev_plan_header* ph = (const cev_plan_header*)a.plan;
  const int4 td = ((const int4*)(a.plan + ph->tiles_off))[tile];
  const int4* segs = (const int4*)(a.plan + ph->segs_off);
  const int4* rows = (const int4*)(a.plan + ph->rows_off);
  const int gi = wave % a.g, rg = wave / a.g;
  const int head = kvh * a.g + gi;
  const int rit = rg * 32 + n;
  const bool row_ok = rit < td.y && td.x + rit < a.t;
  const int row = row_ok ? td.x + rit : 0;

  f32x4 qf[NQ4];
  {
    const float* qp = (const float*)a.q + (int64_t)row * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
    for (int k = 0; k < NQ4; ++k) qf[k] = row_ok ? *(const f32x4*)(qp + 8 * k + 4 * u) : f32x4{};
  }
  int4 rv = rows[row];
  if (!row_ok) rv = make_int4(0, 0, -1, 0);

  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
  float m_run = -INFINITY, l_run = 0.0f;

  for (int si = 0; si < td.w; ++si) {
    const int4 sg = clamp_seg(segs[td.z + si], a.s_cache, a.t);
    const bool cached = sg.x < a.s_cache;
    const float* kb = cached ? (const float*)a.kc + kvh * a.kc_sh + (int64_t)sg.x * a.kc_ss
                             : (const float*)a.kn + kvh * a.kn_sh + (int64_t)(sg.x - a.s_cache) * a.kn_st;
    const float* vb = cached ? (const float*)a.vc + kvh * a.vc_sh + (int64_t)sg.x * a.vc_ss
                             : (const float*)a.vn + kvh * a.vn_sh + (int64_t)(sg.x - a.s_cache) * a.vn_st;
    const int64_t ks = cached ? a.kc_ss : a.kn_st;
    const int64_t vs = cached ? a.vc_ss : a.vn_st;
    const int seg_len = sg.y - sg.x;
    for (int k0 = 0; k0 < seg_len; k0 += BN) {
      const int nvalid = min(BN, seg_len - k0);
      __syncthreads();
#pragma unroll
      for (int v = tid; v < BN * D / 4; v += NT) {
        const int key = v / (D / 4), c = (v % (D / 4)) * 4;
        f32x4 x = {}, y = {};
        if (key < nvalid) {
          x = *(const f32x4*)(kb + (int64_t)(k0 + key) * ks + c);
          y = *(const f32x4*)(vb + (int64_t)(k0 + key) * vs + c);
        }
        *(f32x4*)&sK[key * KS + c] = x;
        *(f32x4*)&sV[key * KS + c] = y;
      }
      __syncthreads();

      f32x16 s[NKT];
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        s[kt] = f32x16{};
#pragma unroll
        for (int k = 0; k < NQ4; ++k) {
          const f32x4 af = *(const f32x4*)&sK[(kt * 32 + n) * KS + 8 * k + 4 * u];
#pragma unroll
          for (int r = 0; r < 4; ++r) s[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[r], qf[k][r], s[kt], 0, 0, 0);
        }
      }
      const bool need_mask = sg.z != 0 || nvalid < BN;
      const int key0 = sg.x + k0;
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float x = s[kt][i] * a.scale_log2;
          if (need_mask) {
            const int kk = kt * 32 + 8 * (i >> 2) + 4 * u + (i & 3);
            const int key = key0 + kk;
            const bool vis = (kk < nvalid) & ((sg.z == 0) | ((key >= rv.x) & (key < rv.y)) | (key == rv.z));
            x = vis ? x : -INFINITY;
          }
          s[kt][i] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, swap_half(mx));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
      float rs = 0.0f;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = fast_exp2(s[kt][i] - m_use);
          s[kt][i] = p;
          rs += p;
        }
      l_run += rs;
      // O^T += V^T . P^T, one K=2 step per S^T register: K slot u is key
      // 8(i/4) + 4u + i%4 of the sub-tile.
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kt * 32 + 8 * (i >> 2) + 4 * u + (i & 3);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(sV[key * KS + dt * 32 + n], s[kt][i], o[dt], 0, 0, 0);
        }
    }
  }

  const float l = l_run + swap_half(l_run);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (!row_ok) return;
  float* op = (float*)a.out + (int64_t)row * a.o_st + (int64_t)head * a.o_sh;
  const float* gp = a.has_gate ? (const float*)a.gate + (int64_t)row * a.g_st + (int64_t)head * a.g_sh : nullptr;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = dt * 32 + 8 * q4 + 4 * u;
      f32x4 r;
      f32x4 gv = {};
      if (gp) gv = *(const f32x4*)(gp + d);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = o[dt][4 * q4 + e] / l;
        if (!(l > 0.0f)) x = 0.0f;
        if (gp) x = gate_value(x, gv[e], false);
        r[e] = x;
      }
      *(f32x4*)(op + d) = r;
    }
  (void)inv;
}

template <typename Kernel>
int32_t launch(Kernel k, const AttnArgs& a, hipStream_t stream) {
  const int64_t grid = (int64_t)a.n_tiles * a.hkv;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "grid of %lld workgroups is too large", (long long)grid);
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kAttnWaves * 64), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "packed attention launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

}  // namespace

extern "C" int32_t cev_packed_attention(const cev_attn_desc* d, const void* plan_host, const void* plan_dev, const void* q,
                                        const void* k_cache, const void* v_cache, const void* k_new, const void* v_new, const void* gate,
                                        void* out, cev_stream stream) {
  CEV_CHECK_ARG(d != nullptr, "cev_packed_attention: null descriptor");
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
  CEV_CHECK_ARG(h->tile_rows == cev_attn_tile_rows(g), "cev_packed_attention: plan tile size mismatch");
  const uintptr_t al = 15;
  CEV_CHECK_ARG((((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)out |
                  (uintptr_t)gate | (uintptr_t)plan_dev) & al) == 0,
                "cev_packed_attention: device buffers must be 16-byte aligned");
  AttnArgs a;
  a.q = q;
  a.kc = k_cache;
  a.vc = v_cache;
  a.kn = k_new;
  a.vn = v_new;
  a.gate = gate;
  a.out = out;
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
  a.hkv = d->n_kv_heads;
  a.g = g;
  a.has_gate = d->has_gate;
  a.scale_log2 = d->scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  if (d->dtype == CEV_BF16) {
    if (d->head_dim == 128) return launch(attn_bf16_kernel<128, 64>, a, s);
    return launch(attn_bf16_kernel<256, 32>, a, s);
  }
  return launch(attn_f32_kernel<128, 32>, a, s);
}
