// Gated DeltaNet layer core for gfx950: the replacement for the part of
// GatedDeltaNet::forward (crates/cev-model/src/qwen35.rs:414-453) between the
// input projections and out_proj.
//
//   conv:  depthwise causal conv over [conv state || x] + SiLU, new state
//          (qwen35.rs:428-430, decoder.rs:137-151), model dtype ops;
//   prep:  per (row, value head, 64-token chunk), in f32: q, k l2norm
//          (q * dk^-0.5), beta = sigmoid(b), g = softplus(a + dt_bias) * -e^A,
//          cum = prefix sum of g, ut = (k beta) k^T * pair, intra = q k^T * pair,
//          inv = (I + strict_lower(ut))^-1, new_values = inv (v beta),
//          k_cumdecay = inv (k beta e^cum) (qwen35.rs:301-345);
//   scan:  the sequential chunk recurrence (qwen35.rs:346-365) with the
//          state split into 16-column slices (columns of S evolve
//          independently), one workgroup per (row, head, slice);
//   norm:  gated RMSNorm * SiLU(z) and the cast to the model dtype
//          (qwen35.rs:447-451).
//
// All chunk-rule products run on v_mfma_f32_16x16x4_f32 (full f32 like the
// reference).  Lane layout (16x16x4): A lane l holds A[l%16][l/16], B lane l
// holds B[l/16][l%16], D lane l register r holds D[4(l/16)+r][l%16].
#include <cstring>

#include <type_traits>

#include "cev_device.h"
#include "cev_internal.h"

namespace {

constexpr int kC = 64;     // chunk length (qwen35.rs:302)
constexpr int kD = 128;    // head_k_dim = head_v_dim supported here
constexpr int kW = 16;     // state columns per scan workgroup
constexpr int kSX = 132;   // LDS row stride (floats) of 128-wide f32 tiles
constexpr int kSC = 68;    // LDS row stride of 64-wide f32 tiles
// Per (row, head, chunk) record in the workspace, in floats, stored in the
// order the scan's MFMAs consume it: lane l of a wave reads 4 consecutive
// floats (4 k-steps, or the 4 accumulator rows) with one 16-byte load.
//   Qd  q e^cum           A operand, row tile w:   [w 4][j 8][lane][4] = Qd[16w + l%16][4(4j+e) + l/16]
//   Kc  k_cumdecay        same layout as Qd
//   Kd  k e^(last - cum)  A = Kd^T, dk tile ti:    [ti 8][j 4][lane][4] = Kd[4(4j+e) + l/16][16ti + l%16]
//   In  intra             A operand, row tile w:   [w 4][j 4][lane][4] = In[16w + l%16][4(4j+e) + l/16]
//   Nv  new_values        accumulator, slice sl:   [sl 8][w 4][lane][4] = Nv[16w + 4(l/16) + e][16sl + l%16]
//   decay                 e^last
// bf16 models keep q and k as the raw bf16 conv output instead of Qd and Kd,
// 16 values per lane in 32 bytes, plus the factors prep multiplies them by:
//   Qb  [w 4][K half 2][lane][j' 4][e 4] = q[16w + l%16][4(4(4 half + j') + e) + l/16]
//   Kb  [ti 8][lane][j 4][e 4]            = k[4(4j+e) + l/16][16ti + l%16]
//   Qf  [row][2] = (dk^-0.5 / |q_row|, e^cum_row)
//   Kf  [2][l/16][m 16] = 1 / |k_t| and e^(last - cum_t) of token t = 4m + l/16
// The scan rebuilds Qd = (q * Qf0) * Qf1 and Kd = (k * 1/|k|) * e^(last - cum)
// with prep's own two roundings, so both layouts give the same bits; the bf16
// record is 113 KB instead of 144 KB.  Qb and Kb depend on the key head only:
// for the many-chunk scan the first value head of each key head's group writes
// them, and the scans of the group's other value heads read them from that
// head's record.
// In's six tiles above the diagonal are zero.  The scan skips their MFMAs,
// and the many-chunk scan never loads them either, so prep stores them only
// for the one-chunk scan, which loads every tile at a fixed offset (it is
// held to 128 registers, and the clamped addresses cost it spills).
template <bool BF>
struct RecLayout;
template <>
struct RecLayout<false> {
  static constexpr int Qd = 0, Kc = kC * kD, Kd = 2 * kC * kD, Nv = 3 * kC * kD, In = 4 * kC * kD;
  static constexpr int Decay = In + kC * kC, Qf = Decay, Kf = Decay;  // no factors
  static constexpr int Floats = Decay + 16;
};
template <>
struct RecLayout<true> {
  static constexpr int Qd = 0, Kc = kC * kD / 2, Kd = Kc + kC * kD, Nv = Kd + kC * kD / 2, In = Nv + kC * kD;
  static constexpr int Decay = In + kC * kC, Qf = Decay + 16, Kf = Qf + 2 * kC;
  static constexpr int Floats = Kf + 2 * kC;
};
constexpr int kRecFloats = RecLayout<false>::Floats;  // the workspace's record size (the larger one)
static_assert(RecLayout<true>::Floats % 16 == 0 && RecLayout<false>::Floats % 16 == 0, "64-byte aligned records");

typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4v mma16(float a, float b, f32x4v c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

template <typename T>
__device__ __forceinline__ float to_f(T x) {
  return (float)x;
}
template <typename T>
__device__ __forceinline__ T from_f(float x);
template <>
__device__ __forceinline__ float from_f<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ __bf16 from_f<__bf16>(float x) {
  return (__bf16)x;
}
template <typename T>
__device__ __forceinline__ float rnd(float x) {  // one model-dtype op result
  return sizeof(T) == 2 ? bf16_round(x) : x;
}

struct GdnArgs {
  const void* mixed;
  const void* z;
  const void* b;
  const void* a;
  const void* conv_w;
  const float* neg_a;
  const float* dt_bias;
  const float* norm_w;
  const void* conv_in;
  const float* s_in;
  void* y;
  void* conv_out;
  float* s_out;
  void* conved;  // workspace: (B, T, conv_dim) model dtype
  float* rec;    // workspace: (B, nv, n_chunks) records
  float* core;   // workspace: (B, T, nv, dv) f32
  int64_t mixed_sb, mixed_st, z_sb, z_st, ab_sb, ab_st, conv_in_sb, s_in_sb, y_sb, y_st;
  int32_t batch, t, nk, nv, kernel, conv_dim, n_chunks, conv_run;
  float eps;
};

// ---------------------------------------------------------------------------
// conv + SiLU.  Thread = (row, 8 channels, run of conv_run tokens): the 8 x K
// weights stay in registers and the last K-1 input rows slide through a
// register window, so every input row is read once as one 16-byte vector.
// Each product and partial sum is one model-dtype op (decoder.rs:143-150);
// SiLU is candle's v / (1 + exp(-v)) with each op in the model dtype.  The
// thread of a row's last run also writes the new conv state: its window then
// holds the last K-1 columns of [state || x] (qwen35.rs:429).
// Run length: 16 tokens, or 8 / 4 when that leaves fewer workgroups than
// CUs (short rows, e.g. 32 rows of 64 tokens).
constexpr int kConvRunMax = 16;
constexpr int kConvCus = 256;
// 16 waves per workgroup share one table; widths 7 and 8 need more than the
// 128 registers that leaves each lane, so they run 8 waves
constexpr int conv_threads(int K) { return K <= 6 ? 1024 : 512; }

// Each conv workgroup first tabulates the bf16 SiLU in LDS (silu_fill), and
// a token whose 8 x 64 values are not all in the table's range takes
// silu_bf16 itself (wave-uniform branch).

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
// two values rounded to bf16 by one conversion
__device__ __forceinline__ f32x2v bf16_round2(f32x2v x) {
  return __builtin_convertvector(__builtin_convertvector(x, bf16x2v), f32x2v);
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v);
template <>
__device__ __forceinline__ void load8<__bf16>(const __bf16* p, float* v) {
  const bf16x8 x = *(const bf16x8*)p;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)x[e];
}
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* v) {
  const f32x4 x = *(const f32x4*)p, y = *(const f32x4*)(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = x[e];
    v[e + 4] = y[e];
  }
}
// 8 channels of one input row as loaded (converted to f32 where used, so a
// row loaded one iteration ahead is not waited for early)
template <typename T>
struct Raw8;
template <>
struct Raw8<__bf16> {
  bf16x8 x;
  __device__ __forceinline__ void load(const __bf16* p) { x = *(const bf16x8*)p; }
  __device__ __forceinline__ float operator[](int e) const { return (float)x[e]; }
};
template <>
struct Raw8<float> {
  f32x4 x, y;
  __device__ __forceinline__ void load(const float* p) {
    x = *(const f32x4*)p;
    y = *(const f32x4*)(p + 4);
  }
  __device__ __forceinline__ float operator[](int e) const { return e < 4 ? x[e] : y[e - 4]; }
};

template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v);
template <>
__device__ __forceinline__ void store8<__bf16>(__bf16* p, const float* v) {
  bf16x8 x;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (__bf16)v[e];
  *(bf16x8*)p = x;
}
template <>
__device__ __forceinline__ void store8<float>(float* p, const float* v) {
  *(f32x4*)p = f32x4{v[0], v[1], v[2], v[3]};
  *(f32x4*)(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

template <typename T, int K>
__device__ __forceinline__ void conv_run(const GdnArgs& g, const float* silu_tab, int r, int t0, int c0) {
  const T* x = (const T*)g.mixed + r * g.mixed_sb;
  const T* tail = g.conv_in ? (const T*)g.conv_in + r * g.conv_in_sb : nullptr;
  float w[8][K];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int u = 0; u < K; ++u) w[e][u] = to_f(((const T*)g.conv_w)[(int64_t)(c0 + e) * K + u]);
  // window[j] = input row t - (K-1) + j for the token t being produced
  float win[K][8];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int p = t0 - (K - 1) + j;
    if (p >= 0) {
      load8<T>(x + (int64_t)p * g.mixed_st + c0, win[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[j][e] = tail ? to_f(tail[(int64_t)(c0 + e) * (K - 1) + (K - 1 + p)]) : 0.0f;
    }
  }
  T* out = (T*)g.conved + ((int64_t)r * g.t + t0) * g.conv_dim + c0;
  const int n = min(g.conv_run, g.t - t0);
  // the next row loads while this one is computed (the last load repeats
  // the last row, so it stays unconditional and in bounds)
  Raw8<T> next;
  const T* xp = x + (int64_t)t0 * g.mixed_st + c0;
  next.load(xp);
  // s_waitcnt vmcnt(0): with nothing pending at the loop entry, the wait at
  // the loop head covers only the prefetch, not the previous row's store
  __builtin_amdgcn_s_waitcnt(0x0F70);
  for (int i = 0; i < n; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) win[K - 1][e] = next[e];
    xp += i + 1 < n ? g.mixed_st : 0;
    next.load(xp);
    float y[8];
    if constexpr (sizeof(T) == 2) {
      // products and partial sums, each rounded to bf16, two channels per
      // conversion
      f32x2v acc[4];
#pragma unroll
      for (int u = 0; u < K; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x2v term = bf16_round2(f32x2v{win[u][2 * q] * w[2 * q][u], win[u][2 * q + 1] * w[2 * q + 1][u]});
          acc[q] = u == 0 ? term : bf16_round2(acc[q] + term);
        }
      uint32_t slot[8];
      bool hit = true;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        slot[e] = silu_slot(acc[e / 2][e % 2]);
        hit = hit && slot[e] < (uint32_t)kSiluEntries;
      }
      if (__all(hit)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = silu_tab[slot[e]];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = silu_bf16(acc[e / 2][e % 2]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < K; ++u) acc = u == 0 ? win[u][e] * w[e][u] : acc + win[u][e] * w[e][u];
        y[e] = acc / (1.0f + expf(-acc));
      }
    }
    store8<T>(out + (int64_t)i * g.conv_dim, y);
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[j][e] = win[j + 1][e];
  }
  if (t0 + n == g.t) {
    // new conv state (conv_dim, K-1) of this row: the window's last K-1 columns
    T* st = (T*)g.conv_out + ((int64_t)r * g.conv_dim + c0) * (K - 1);
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int j = 0; j < K - 1; ++j) st[e * (K - 1) + j] = from_f<T>(win[j][e]);
  }
}

// One kernel per conv width, so each gets its own register allocation (the
// window and weights take 16 K registers).
template <typename T, int K>
__global__ __launch_bounds__(conv_threads(K)) void gdn_conv_kernel(GdnArgs g) {
  constexpr int kConvThreads = conv_threads(K);
  __shared__ float silu_tab[sizeof(T) == 2 ? kSiluEntries : 1];
  if constexpr (sizeof(T) == 2) {
    silu_fill(silu_tab, kConvThreads);
    __syncthreads();
  }
  const int64_t cg = g.conv_dim / 8;
  const int64_t runs = (g.t + g.conv_run - 1) / g.conv_run;
  const int64_t idx = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
  if (idx >= (int64_t)g.batch * runs * cg) return;
  const int c0 = (int)(idx % cg) * 8;
  const int64_t rr = idx / cg;
  const int t0 = (int)(rr % runs) * g.conv_run, r = (int)(rr / runs);
  conv_run<T, K>(g, silu_tab, r, t0, c0);
}

template <typename T, int K>
void launch_conv_k(const GdnArgs& g, int64_t items, hipStream_t s) {
  constexpr int n = conv_threads(K);
  hipLaunchKernelGGL((gdn_conv_kernel<T, K>), dim3((unsigned)((items + n - 1) / n)), dim3(n), 0, s, g);
}

template <typename T>
void launch_conv(const GdnArgs& g, int64_t items, hipStream_t s) {
  switch (g.kernel) {
    case 2: launch_conv_k<T, 2>(g, items, s); break;
    case 3: launch_conv_k<T, 3>(g, items, s); break;
    case 4: launch_conv_k<T, 4>(g, items, s); break;
    case 5: launch_conv_k<T, 5>(g, items, s); break;
    case 6: launch_conv_k<T, 6>(g, items, s); break;
    case 7: launch_conv_k<T, 7>(g, items, s); break;
    default: launch_conv_k<T, 8>(g, items, s); break;
  }
}

// ---------------------------------------------------------------------------
// prep: one workgroup (8 waves) per (row, value head, chunk).
constexpr int kPrepThreads = 512;
constexpr int kPrepWaves = kPrepThreads / 64;
static_assert(kPrepWaves == 8, "the prep kernel's work split assumes 8 waves");

// Sum over the 16 lanes of a DPP row.  Every lane ends with the same bits:
// each step adds two values that the partner lane adds in the other order.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<0xB1>(x);   // lane ^ 1
  x += dpp_f<0x4E>(x);   // lane ^ 2
  x += dpp_f<0x141>(x);  // half-row mirror: quad 0 <-> 1, 2 <-> 3
  x += dpp_f<0x140>(x);  // row mirror: quads {0,1} <-> {3,2}
  return x;
}

constexpr int kSB = 136;  // LDS row stride (bf16 elements) of the raw 128-wide q / k rows
constexpr int kST = 20;   // row stride (floats) of a packed 16x16 tile

// Every access to ut and the inverse falls in a 16x16 tile at or below the
// diagonal.  us(i, j) / iv(i, j) name element (i, j) of ut / inv.
struct PrepGates {
  float betas[kC], cums[kC], ecum[kC], ekd[kC];
};
template <bool BF>
struct PrepLds;
// f32 models: normalised f32 q / k rows, full 64 x 64 ut and inverse.
template <>
struct __attribute__((aligned(16))) PrepLds<false> : PrepGates {
  float Qs[kC * kSX];  // q normalised * dk^-0.5; later k_cumdecay staging
  float Ks[kC * kSX];  // k normalised
  float Us[kC * kSC];  // ut, strict lower (tiles at and below the diagonal)
  float Iv[kC * kSC];  // (I + ut)^-1 (tiles at and below the diagonal)
  // Products of the block inversion.  Before the inversion (the tile phase)
  // the same space holds the intra tiles on their way to record order.
  float Tm[kC * kSC];
  __device__ float& us(int i, int j) { return Us[i * kSC + j]; }
  __device__ float& iv(int i, int j) { return Iv[i * kSC + j]; }
  __device__ float* kc_stage() { return Qs; }
};
// bf16 models: the raw q / k rows (the conv output, exact in bf16) with each
// row's l2norm factor, ut and the inverse packed as their ten lower 16x16
// tiles; 78 KB, so two workgroups share a CU.
constexpr int lower_tile(int ti, int tj) { return ti * (ti + 1) / 2 + tj; }
template <>
struct __attribute__((aligned(16))) PrepLds<true> : PrepGates {
  // Qb then Kb; after the inversion both hold the k_cumdecay staging
  // (64 x kSX floats fit in their 64 x 2 kSB bf16).
  __bf16 Qb[kC * kSB];
  __bf16 Kb[kC * kSB];
  float Us[10 * 16 * kST];
  float Iv[10 * 16 * kST];
  float Tm[kC * kSC];
  float qf[kC];  // dk^-0.5 / |q_i|
  float kf[kC];  // 1 / |k_i|
  __device__ static int at(int i, int j) { return lower_tile(i >> 4, j >> 4) * (16 * kST) + (i & 15) * kST + (j & 15); }
  __device__ float& us(int i, int j) { return Us[at(i, j)]; }
  __device__ float& iv(int i, int j) { return Iv[at(i, j)]; }
  __device__ float* kc_stage() { return (float*)Qb; }
};
static_assert(sizeof(PrepLds<true>) <= 80 * 1024, "two bf16 prep workgroups per CU");
static_assert(kC * kSX * sizeof(float) <= 2 * kC * kSB * sizeof(__bf16), "k_cumdecay staging fits in Qb / Kb");

// Epilogue of one 16x16 tile (ti, tj), tj <= ti, in the MFMA accumulator
// layout (lane: column 16 tj + fm, rows 16 ti + 4 fq + e):
//   ut[i][j] = G[i][j] pair[i][j] for j < i,   pair = e^(cum_i - cum_j),
//   intra[i][j] = QK[i][j] pair[i][j] for j <= i  (qwen35.rs:318-330),
// ut into Us; intra through the wave's own tile of Tm into its record order.
template <bool DG, bool DQ, typename LT>
__device__ __forceinline__ void prep_tile_store(LT& L, float* rec_in, int ti, int tj, int lane, const f32x4v& gacc, const f32x4v& qacc) {
  const int fm = lane & 15, fq = lane >> 4;
  const int j = 16 * tj + fm;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = 16 * ti + 4 * fq + e;
    const float pair = j <= i ? expf(L.cums[i] - L.cums[j]) : 0.0f;
    if (DG) L.us(i, j) = j < i ? gacc[e] * pair : 0.0f;
    if (DQ) L.Tm[i * kSC + j] = qacc[e] * pair;
  }
  if (DQ) {
    wave_lds_sync();
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = L.Tm[(16 * ti + fm) * kSC + 16 * tj + 4 * e + fq];
    *(f32x4*)(rec_in + 4 * ((ti * 4 + tj) * 64 + lane)) = v;
  }
}

// The tile products for bf16 models: G = (k beta) k^T and QK = q k^T on
// v_mfma_f32_16x16x32_bf16 over the raw bf16 rows (every product of two
// bf16 values is exact in f32 and the sums are f32, as with the normalised
// f32 operands), then the l2norm factors and beta:
//   G[i][j] = (k_i . k_j) (beta_i / |k_i|) / |k_j|,  QK[i][j] = (q_i . k_j) (dk^-0.5 / |q_i|) / |k_j|.
// Lane (fm, fq) reads row 16 t + fm, columns 32 s + 8 fq .. + 7 (16 bytes)
// of A and B, so both operands pair up over the same k.
template <bool DG, bool DQ>
__device__ __forceinline__ void prep_tile_bf16(PrepLds<true>& L, float* rec_in, int ti, int tj, int lane) {
  const int fm = lane & 15, fq = lane >> 4;
  const __bf16* ka = L.Kb + (16 * ti + fm) * kSB + 8 * fq;
  const __bf16* qa = L.Qb + (16 * ti + fm) * kSB + 8 * fq;
  const __bf16* kb = L.Kb + (16 * tj + fm) * kSB + 8 * fq;
  f32x4v gacc = {0, 0, 0, 0}, qacc = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < kD / 32; ++s) {
    const bf16x8 b8 = *(const bf16x8*)(kb + 32 * s);
    if (DG) gacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8*)(ka + 32 * s), b8, gacc, 0, 0, 0);
    if (DQ) qacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8*)(qa + 32 * s), b8, qacc, 0, 0, 0);
  }
  const float kfj = L.kf[16 * tj + fm];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = 16 * ti + 4 * fq + e;
    if (DG) gacc[e] = gacc[e] * (L.betas[i] * L.kf[i]) * kfj;
    if (DQ) qacc[e] = qacc[e] * L.qf[i] * kfj;
  }
  prep_tile_store<DG, DQ>(L, rec_in, ti, tj, lane, gacc, qacc);
}

// One 16x16 tile (ti, tj), tj <= ti, of G = (k beta) k^T (DG) and / or
// QK = q k^T (DQ) on the normalised f32 rows.  The k-sum runs in the order
// 16j + 4fq + e, so each lane reads its A and B operands as 16-byte vectors.
template <bool DG, bool DQ, typename LT>
__device__ __forceinline__ void prep_tile(LT& L, float* rec_in, int ti, int tj, int lane) {
  const int fm = lane & 15, fq = lane >> 4;
  const float* ka = L.Ks + (16 * ti + fm) * kSX + 4 * fq;
  const float* qa = L.Qs + (16 * ti + fm) * kSX + 4 * fq;
  const float* kb = L.Ks + (16 * tj + fm) * kSX + 4 * fq;
  const float bi = DG ? L.betas[16 * ti + fm] : 0.0f;
  f32x4v gacc = {0, 0, 0, 0}, qacc = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < kD / 16; ++j) {
    const f32x4 b4 = *(const f32x4*)(kb + 16 * j);
    f32x4 a4 = {0, 0, 0, 0}, q4 = {0, 0, 0, 0};
    if (DG) a4 = *(const f32x4*)(ka + 16 * j);
    if (DQ) q4 = *(const f32x4*)(qa + 16 * j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (DG) gacc = mma16(a4[e] * bi, b4[e], gacc);
      if (DQ) qacc = mma16(q4[e], b4[e], qacc);
    }
  }
  prep_tile_store<DG, DQ>(L, rec_in, ti, tj, lane, gacc, qacc);
}

// 16x16 diagonal block b of inv = (I + L)^-1, L = Us strict lower, by
// forward substitution: lane j (of each 16-lane group) owns column j,
//   inv[i][j] = -sum_{k<i} L[i][k] inv[k][j]  (inv[k][j] = 0 for k < j,
//   1 for k == j); the L[i][k] reads are broadcasts.  Lanes with fq == 0 write.
template <typename LT>
__device__ __forceinline__ void prep_inv16(LT& L, int b, int lane) {
  const int b0 = 16 * b, j = lane & 15;
  float col[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) col[k] = k == j ? 1.0f : 0.0f;
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < i; ++k) acc += L.us(b0 + i, b0 + k) * col[k];
    col[i] = i > j ? -acc : col[i];
  }
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) L.iv(b0 + i, b0 + j) = col[i];
  }
}

// Work split (8 waves, wave w on SIMD w % 4; every SIMD gets 5 tile products):
//   load   all:  v column slice 16w.. into registers, q / k rows l2-normed
//                into LDS; wave 0: gates, cum (sequential, as the reference)
//   tiles  w 0-2: two off-diagonal tiles, both products; w 3: the four
//                diagonal QK products; w 4 + b: the diagonal G product of
//                block b and its 16x16 inverse
//   inv    32-level (w 0, 1; w 2-7 write the Qd records), 64-level (w 0-3;
//                w 4-7 write the Kd records and intra's zero tiles); every
//                wave scales its nv / kc operands after the 32-level
//   nv/kc  wave w: column tile w of new_values and k_cumdecay, row tiles 0-3
template <typename T>
__global__ __launch_bounds__(kPrepThreads) void gdn_prep_kernel(GdnArgs g) {
  constexpr bool BF = std::is_same<T, __bf16>::value;
  using R = RecLayout<BF>;
  __shared__ PrepLds<BF> L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fm = lane & 15, fq = lane >> 4;  // fragment row / k-slot of this lane
  const int c = blockIdx.x % g.n_chunks;
  const int hr = blockIdx.x / g.n_chunks;
  const int h = hr % g.nv, r = hr / g.nv;
  const int kh = h / (g.nv / g.nk);  // value head h reads key head h / (nv/nk) (qwen35.rs:436-442)
  // bf16 records for the many-chunk scan: only the group's first value head
  // stores the raw q / k rows (the one-chunk scan reads its own record's)
  const bool qk_rows = !BF || g.n_chunks == 1 || h % (g.nv / g.nk) == 0;
  // intra's zero tiles: read only by the one-chunk scan
  const bool zero_tiles = g.n_chunks == 1;
  const int key_dim = g.nk * kD;
  const int t0 = c * kC;
  const T* cv = (const T*)g.conved + (int64_t)r * g.t * g.conv_dim;
  float* rec = g.rec + (int64_t)blockIdx.x * R::Floats;

  // All loads below read a valid row (clamped to the last token) and the
  // rows past t are zeroed afterwards, so no load sits behind a branch and
  // all of them are in flight together.
  const int t_last = g.t - 1;
  // ---- v column slice of this wave, in the nv k order:
  // vreg[4jg + e] = v[16jg + 4fq + e][16 wave + fm] (rows past t are zero)
  float vreg[16], kreg[16];
  {
    const T* vcol = cv + 2 * key_dim + h * kD + 16 * wave + fm;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int t = t0 + 16 * (x >> 2) + 4 * fq + (x & 3);
      const float v = to_f(vcol[(int64_t)min(t, t_last) * g.conv_dim]);
      vreg[x] = t < g.t ? v : 0.0f;
    }
  }
  // ---- q, k rows i and i + 32, 16 lanes per row, 8 columns each; l2norm
  // x / sqrt(sum x^2 + 1e-6), q then * dk^-0.5 (qwen35.rs:250-254, :305-306)
  {
    const int i0 = tid >> 4, col = (tid & 15) * 8;
    float qv[2][8], kv[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + i0 + 32 * u;
      const T* row = cv + (int64_t)min(t, t_last) * g.conv_dim;
      load8<T>(row + kh * kD + col, qv[u]);
      load8<T>(row + key_dim + kh * kD + col, kv[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qv[u][e] = t < g.t ? qv[u][e] : 0.0f;
        kv[u][e] = t < g.t ? kv[u][e] : 0.0f;
      }
    }
    const float qscale = 0.08838834764831845f;  // 128^-0.5
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float sq = 0.0f, sk = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sq += qv[u][e] * qv[u][e];
        sk += kv[u][e] * kv[u][e];
      }
      const float nq = sqrtf(row16_sum(sq) + 1e-6f), nk = sqrtf(row16_sum(sk) + 1e-6f);
      if constexpr (!BF) {
        float* qrow = L.Qs + (i0 + 32 * u) * kSX + col;
        float* krow = L.Ks + (i0 + 32 * u) * kSX + col;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          f32x4 a, b;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[e] = qv[u][4 * hf + e] / nq * qscale;
            b[e] = kv[u][4 * hf + e] / nk;
          }
          *(f32x4*)(qrow + 4 * hf) = a;
          *(f32x4*)(krow + 4 * hf) = b;
        }
      } else {
        bf16x8 qb, kb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qb[e] = (__bf16)qv[u][e];  // exact: the values came from bf16
          kb[e] = (__bf16)kv[u][e];
        }
        *(bf16x8*)(L.Qb + (i0 + 32 * u) * kSB + col) = qb;
        *(bf16x8*)(L.Kb + (i0 + 32 * u) * kSB + col) = kb;
        if ((tid & 15) == 0) {
          L.qf[i0 + 32 * u] = qscale / nq;
          L.kf[i0 + 32 * u] = 1.0f / nk;
        }
      }
    }
  }
  // ---- gates (lane = chunk row): beta = sigmoid(b), g = softplus(a +
  // dt_bias) * -e^A (qwen35.rs:243-248, :436-440); cum = running sum of g in
  // row order (lane i adds g_0 .. g_i one by one, like the reference)
  if (wave == 0) {
    const int t = t0 + lane;
    const int64_t ab = r * g.ab_sb + (int64_t)min(t, t_last) * g.ab_st + h;
    const float av = to_f(((const T*)g.a)[ab]);
    const float bb = to_f(((const T*)g.b)[ab]);
    const float x = av + g.dt_bias[h];
    const float sp = fmaxf(x, 0.0f) + logf(expf(-fabsf(x)) + 1.0f);
    const float gv = t < g.t ? sp * g.neg_a[h] : 0.0f;
    const float bv = t < g.t ? 1.0f / (1.0f + expf(-bb)) : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < kC; ++k) {
      const float gk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gv), k));
      const float s = acc + gk;
      acc = k <= lane ? s : acc;
    }
    const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), kC - 1));
    L.betas[lane] = bv;
    L.cums[lane] = acc;
    L.ecum[lane] = expf(acc);
    L.ekd[lane] = expf(last - acc);
    if (lane == 0) rec[R::Decay] = expf(last);
  }
  __syncthreads();

  // v beta for the nv operands: done before this wave issues any store, so
  // the wait for the v loads waits for nothing else
#pragma unroll
  for (int jg = 0; jg < 4; ++jg) {
    const f32x4 b4 = *(const f32x4*)(L.betas + 16 * jg + 4 * fq);
#pragma unroll
    for (int e = 0; e < 4; ++e) vreg[4 * jg + e] = vreg[4 * jg + e] * b4[e];
  }
#pragma unroll
  for (int x = 0; x < 16; ++x) asm volatile("" : "+v"(vreg[x]));  // keeps the compiler from sinking it

  // ---- G / QK tiles and the 16x16 diagonal inverses
  // (Tile indices by arithmetic: a table indexed by wave would be a global
  // load, and its wait would also wait for this wave's record stores.)
  auto tile = [&](auto dg_c, auto dq_c, int ti, int tj) {
    constexpr bool DG = decltype(dg_c)::value, DQ = decltype(dq_c)::value;
    if constexpr (BF)
      prep_tile_bf16<DG, DQ>(L, rec + R::In, ti, tj, lane);
    else
      prep_tile<DG, DQ>(L, rec + R::In, ti, tj, lane);
  };
  using Yes = std::true_type;
  using No = std::false_type;
  if (wave < 3) {
    // wave 0: (1,0) (2,0); wave 1: (2,1) (3,0); wave 2: (3,1) (3,2)
    tile(Yes{}, Yes{}, wave == 0 ? 1 : wave + 1, wave == 0 ? 0 : 1);
    tile(Yes{}, Yes{}, wave == 0 ? 2 : 3, wave == 2 ? 2 : 0);
  } else if (wave == 3) {
#pragma unroll
    for (int b = 0; b < 4; ++b) tile(No{}, Yes{}, b, b);
  } else {
    const int b = wave - 4;
    tile(Yes{}, No{}, b, b);
    wave_lds_sync();
    prep_inv16(L, b, lane);
  }
  __syncthreads();

  // Normalised q (times dk^-0.5) and k: stored in f32 for f32 models, the
  // raw bf16 value times the row's factor for bf16 models.
  auto q_hat = [&](int i, int c) {
    if constexpr (BF)
      return (float)L.Qb[i * kSB + c] * L.qf[i];
    else
      return L.Qs[i * kSX + c];
  };
  auto k_hat = [&](int i, int c) {
    if constexpr (BF)
      return (float)L.Kb[i * kSB + c] * L.kf[i];
    else
      return L.Ks[i * kSX + c];
  };
  // Records the inversion's idle waves write: q e^cum (Qd) and k e^(last -
  // cum) (Kd) in their fragment orders (bf16 models: the raw rows, from the
  // group's first value head only, and every head's factors), and for the
  // one-chunk scan intra's six zero tiles.
  constexpr int kQdStores = BF ? kC * kD / 8 : kC * kD / 4;  // 16-byte stores per record part
  auto qd_records = [&](int p0, int step) {
    for (int p = p0; p < kQdStores; p += step) {
      if constexpr (BF) {
        const int hf = p & 1, l = (p >> 1) & 63, half = (p >> 7) & 1, w = p >> 8;  // [w 4][half 2][lane][hf 2]
        bf16x8 v;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const int j = 4 * half + 2 * hf + (x >> 2), e = x & 3;
          v[x] = L.Qb[(16 * w + (l & 15)) * kSB + 4 * (4 * j + e) + (l >> 4)];
        }
        *(bf16x8*)(rec + R::Qd + 4 * p) = v;
      } else {
        const int l = p & 63, j = (p >> 6) & 7, w = p >> 9;  // [w 4][j 8][lane]
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 16 * w + (l & 15), k = 4 * (4 * j + e) + (l >> 4);
          v[e] = q_hat(i, k) * L.ecum[i];
        }
        *(f32x4*)(rec + R::Qd + 4 * p) = v;
      }
    }
  };
  auto kd_records = [&](int p0, int p_end, int step) {
    for (int p = p0; p < p_end; p += step) {
      if constexpr (BF) {
        const int hf = p & 1, l = (p >> 1) & 63, ti = p >> 7;  // [ti 8][lane][hf 2]
        bf16x8 v;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const int j = 2 * hf + (x >> 2), e = x & 3;
          v[x] = L.Kb[(4 * (4 * j + e) + (l >> 4)) * kSB + 16 * ti + (l & 15)];
        }
        *(bf16x8*)(rec + R::Kd + 4 * p) = v;
      } else {
        const int l = p & 63, jj = (p >> 6) & 3, ti = p >> 8;  // [ti 8][j 4][lane]
        f32x4 u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * (4 * jj + e) + (l >> 4), col = 16 * ti + (l & 15);
          u[e] = k_hat(i, col) * L.ekd[i];
        }
        *(f32x4*)(rec + R::Kd + 4 * p) = u;
      }
    }
  };
  // bf16 models: the row factors of q and the token factors of k
  auto factor_records = [&](int i) {
    if constexpr (BF) {
      if (i < kC) {
        *(f32x2v*)(rec + R::Qf + 2 * i) = f32x2v{L.qf[i], L.ecum[i]};
        rec[R::Kf + (i & 3) * 16 + (i >> 2)] = L.kf[i];
        rec[R::Kf + kC + (i & 3) * 16 + (i >> 2)] = L.ekd[i];
      }
    }
  };

  auto zero_intra = [&](int p0, int step) {
    for (int p = p0; p < 6 * 64; p += step) {
      const int q = p >> 6;  // (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
      const int ti = q < 3 ? 0 : (q < 5 ? 1 : 2), tj = q < 3 ? q + 1 : (q < 5 ? q - 1 : 3);
      *(f32x4*)(rec + R::In + 4 * ((ti * 4 + tj) * 64 + (p & 63))) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };

  // kc operands of this wave's column tile: (k beta) e^cum
  // (qwen35.rs:309-312, :336-340), in the same k order as vreg
  auto operands = [&]() {
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      const f32x4 b4 = *(const f32x4*)(L.betas + 16 * jg + 4 * fq);
      const f32x4 e4 = *(const f32x4*)(L.ecum + 16 * jg + 4 * fq);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * jg + 4 * fq + e;
        kreg[4 * jg + e] = (k_hat(i, 16 * wave + fm) * b4[e]) * e4[e];
      }
    }
  };

  // ---- inverse, 32x32 level: blocks [0,32) (wave 0) and [32,64) (wave 1),
  // off-diagonal 16x16 block = -(B^-1 C) A^-1 (the split of
  // inv_unit_lower, qwen35.rs:277-296)
  if (wave < 2) {
    const int o = 32 * wave;
    f32x4v bc = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; k += 4) bc = mma16(L.iv(o + 16 + fm, o + 16 + k + fq), L.us(o + 16 + k + fq, o + fm), bc);
#pragma unroll
    for (int e = 0; e < 4; ++e) L.Tm[(o + 4 * fq + e) * kSC + fm] = bc[e];
    wave_lds_sync();
    f32x4v x = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; k += 4) x = mma16(L.Tm[(o + fm) * kSC + k + fq], L.iv(o + k + fq, o + fm), x);
#pragma unroll
    for (int e = 0; e < 4; ++e) L.iv(o + 16 + 4 * fq + e, o + fm) = -x[e];
  } else if (qk_rows) {
    qd_records(tid - 128, 384);
  }
  operands();
  __syncthreads();
  // ---- 64x64 level: off block (rows 32..63, cols 0..31) = -(B^-1 C) A^-1
  // with A^-1 = Iv[0:32, 0:32], B^-1 = Iv[32:64, 32:64], C = Us[32:64, 0:32];
  // wave w < 4 takes the 16x16 tile (w / 2, w % 2) of each product.  Both
  // inverses are lower triangular, so the k range of tile row ti stops at
  // 16 (ti + 1) in B^-1 C and starts at 16 tj in the product with A^-1.
  const int ti2 = (wave >> 1) & 1, tj2 = wave & 1;
  if (wave < 4) {
    f32x4v bc = {0, 0, 0, 0};
    for (int k = 0; k < 16 * (ti2 + 1); k += 4)
      bc = mma16(L.iv(32 + 16 * ti2 + fm, 32 + k + fq), L.us(32 + k + fq, 16 * tj2 + fm), bc);
#pragma unroll
    for (int e = 0; e < 4; ++e) L.Tm[(16 * ti2 + 4 * fq + e) * kSC + 16 * tj2 + fm] = bc[e];
  } else {
    if (qk_rows) kd_records(tid - 256, kQdStores / 2, 256);
    if (zero_tiles) zero_intra(tid - 256, 256);
    factor_records(tid - 256);
  }
  __syncthreads();
  if (wave < 4) {
    f32x4v x = {0, 0, 0, 0};
    for (int k = 16 * tj2; k < 32; k += 4)
      x = mma16(L.Tm[(16 * ti2 + fm) * kSC + k + fq], L.iv(k + fq, 16 * tj2 + fm), x);
#pragma unroll
    for (int e = 0; e < 4; ++e) L.iv(32 + 16 * ti2 + 4 * fq + e, 16 * tj2 + fm) = -x[e];
  } else if (qk_rows) {
    kd_records(kQdStores / 2 + tid - 256, kQdStores, 256);
  }
  __syncthreads();

  // ---- new_values = inv (v beta), k_cumdecay = inv (k beta e^cum) for the
  // row tiles ti of this wave's column tile; inv is lower triangular, so
  // row tile ti sums over k < 16 (ti + 1).  new_values goes out in the
  // scan's accumulator order; k_cumdecay through this wave's columns of the
  // staging area (Qs, or Qb / Kb for bf16; free now) into A-fragment order.
  float* stage = L.kc_stage();
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    f32x4v nv = {0, 0, 0, 0}, kc = {0, 0, 0, 0};
    f32x4 a4[4];  // the row tile's inv operands, read before its MFMAs
#pragma unroll
    for (int jg = 0; jg <= ti; ++jg) a4[jg] = *(const f32x4*)&L.iv(16 * ti + fm, 16 * jg + 4 * fq);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jg = 0; jg <= ti; ++jg) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nv = mma16(a4[jg][e], vreg[4 * jg + e], nv);
        kc = mma16(a4[jg][e], kreg[4 * jg + e], kc);
      }
    }
    *(f32x4*)(rec + R::Nv + ((wave * 4 + ti) * 64 + lane) * 4) = f32x4{nv[0], nv[1], nv[2], nv[3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) stage[(16 * ti + 4 * fq + e) * kSX + 16 * wave + fm] = kc[e];
  }
  wave_lds_sync();
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = stage[(16 * ti + fm) * kSX + 16 * wave + 4 * e + fq];
    *(f32x4*)(rec + R::Kc + 4 * ((ti * 8 + wave) * 64 + lane)) = v;
  }
}

// ---------------------------------------------------------------------------
// scan: one workgroup (8 waves) per (row, value head, 16-column slice of the
// state).  Per chunk (qwen35.rs:353-364):
//   v_new = new_values - k_cumdecay . S;   out = (q e^cum) . S + intra . v_new;
//   S = S e^last + (k e^(last-cum))^T . v_new.
// Only v_new and the state update carry the recurrence; the output terms do
// not, so they are spread to fill the second phase:
//   phase A (all 8 waves): wave (row tile rt = w % 4, K half kh = w / 4)
//     forms rows 16rt.. of k_cumdecay . S over its half of dk (16 MFMAs);
//     kh = 0 writes new_values - that, kh = 1 writes its partial;
//   phase B: every wave updates state rows 16w.. in place ((k e^(last-cum))^T
//     . v_new, 16 MFMAs), forms its half of (q e^cum) . S from the state
//     operands it read in phase A (16 MFMAs) and its blocks of intra . v_new
//     (rows 16rt.., blocks kh and kh + 2 up to the diagonal); kh = 0 keeps
//     its sum, kh = 1 hands its sum over through LDS, and kh = 0 stores the
//     chunk's output at the start of the next chunk.
// The A operands come straight from the fragment-ordered record (L2), the
// B operands (S, v_new) from LDS.  blockIdx -> (item, slice) keeps the 8
// slices of one head, and in the bf16 many-chunk scan the value heads of one
// key head, on one XCD (workgroups go round-robin over the 8 XCDs), so each
// head's records, and the raw q / k rows the group shares, are fetched into
// one L2 only.
constexpr int kXcds = 8;
constexpr int kScanThreads = 512;

// A operands of one chunk for one wave; every field is written on every path
// (a struct written on one branch only is kept in scratch memory).  bf16
// records hold raw q / k rows and their factors instead of Qd / Kd.
template <bool BF>
struct ScanOps;
template <>
struct ScanOps<false> {
  f32x4 kc[4], qd[4], kd[4], in[2], nvv;
  float decay;
};
template <>
struct ScanOps<true> {
  f32x4 kc[4], in[2], nvv;
  bf16x8 qb[2], kb[2];
  f32x2v qf, kf;  // this lane's (dk^-0.5/|q|, e^cum) row factors; its part of the Kf array
  float decay;
};

template <bool kPrefetch, bool BF>
__device__ __forceinline__ void gdn_scan(const GdnArgs& g) {
  using R = RecLayout<BF>;
  using Ops = ScanOps<BF>;
  // 16-column tiles.  The prefetching loop stores row r at row
  // r ^ ((r >> 2) & 3) of a 16-float stride: the B-operand reads (rows
  // 4i .. 4i+3 across a wave) and the accumulator writes (rows 4fq + e) then
  // both touch 64 distinct banks.  The one-chunk kernel keeps a 20-float
  // stride (2-way conflicts on the reads): the swizzle's extra address
  // registers would not fit its 128.
  constexpr int kRow = kPrefetch ? 16 : 20;
  __shared__ float S[kD * kRow];     // state slice (dk x 16), updated in place
  __shared__ float Vn0[kC * kRow];   // new_values - k_cumdecay . S, first half of dk
  __shared__ float Vn1[kC * kRow];   // k_cumdecay . S, second half of dk
  __shared__ float Opart[kC * kRow]; // (q e^cum) . S, second half of dk
  __shared__ float KF[BF ? 2 * kC : 1];  // bf16: the chunk's Kf array
  auto sx = [](int row, int col) { return kPrefetch ? (row ^ ((row >> 2) & 3)) * 16 + col : row * 20 + col; };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rt = wave & 3, kh = wave >> 2;
  constexpr int nslice = kD / kW;
  // value heads that share one key head's q / k rows (bf16 records, many-chunk scan)
  const int grp = BF && kPrefetch ? g.nv / g.nk : 1;
  // workgroup b runs on XCD b % 8; the groups G = item / grp with G % 8 ==
  // that XCD take its workgroups, slice fastest, then group member m
  const int b = blockIdx.x, y = b / kXcds;
  const int sl = y % nslice, m = (y / nslice) % grp;
  const int item = ((y / nslice / grp) * kXcds + b % kXcds) * grp + m;  // (row, head) index
  if (item >= g.batch * g.nv) return;
  const int h = item % g.nv, r = item / g.nv;
  // float offset from this head's record to its group's first head's, which
  // holds the raw q / k rows for the many-chunk scan.  The one-chunk scan,
  // held to 128 registers, reads its own record's copy: the second base
  // address took it from 124 registers to its cap of 128.
  const int64_t lead_off = kPrefetch ? -(int64_t)m * g.n_chunks * R::Floats : 0;
  const int col0 = sl * kW;
  const int fm = lane & 15, fq = lane >> 4;

  // this lane's float offsets inside a record: kc / qd operand j at + 256 j,
  // kd operand j at + 256 j, intra blocks kh and kh + 2 at + 0 and + 512;
  // bf16 q and k rows at + 0 and + 4 (two 16-byte halves)
  const int kc_off = R::Kc + 4 * (rt * 8 * 64 + 4 * kh * 64 + lane);
  const int qd_off = BF ? R::Qd + 8 * ((rt * 2 + kh) * 64 + lane) : R::Qd + 4 * (rt * 8 * 64 + 4 * kh * 64 + lane);
  const int kd_off = BF ? R::Kd + 8 * (wave * 64 + lane) : R::Kd + 4 * (wave * 4 * 64 + lane);
  // intra blocks kh and kh + 2 of row tile rt.  Blocks above the diagonal
  // are zero and their MFMAs are skipped; the many-chunk loop reads the
  // diagonal block in their place (a line the wave pair reads anyway), so
  // prep need not store them
  const int in_off = R::In + 4 * (rt * 4 * 64 + kh * 64 + lane);
  // the second block's distance from the first, wave-uniform (kept in an
  // SGPR, so the per-lane offset stays one register)
  const int in_d1 = __builtin_amdgcn_readfirstlane(4 * 64 * (min(kh + 2, rt) - kh));
  const int in_d0 = __builtin_amdgcn_readfirstlane(4 * 64 * (min(kh, rt) - kh));
  const int nv_off = R::Nv + 4 * ((sl * 4 + rt) * 64 + lane);  // read by kh = 0 only
  const int qf_off = R::Qf + 2 * (16 * rt + fm);
  const int kf_off = R::Kf + 2 * lane;
  auto rec_at = [&](int c) { return g.rec + ((int64_t)item * g.n_chunks + c) * R::Floats; };
  auto ld4 = [](const float* p) { return *(const f32x4*)p; };
  auto ldb = [](const float* p) { return *(const bf16x8*)p; };
  auto ld2 = [](const float* p) { return *(const f32x2v*)p; };
  // the phase-A operands (k_cumdecay, new_values, decay; the Kf array), the
  // phase-B ones (q e^cum or q, k e^(last - cum) or k, intra; the q factors)
  auto fetch_a = [&](const float* rec, Ops& o, int j) {
    o.kc[j] = ld4(rec + kc_off + 256 * j);
    if (j == 3) {
      // kh = 1 waves do not use new_values; the prefetching loop loads it
      // anyway (loads under a branch defeat the compiler's wait tracking there)
      o.nvv = (kPrefetch || kh == 0) ? ld4(rec + nv_off) : f32x4{};
      o.decay = rec[R::Decay];
      if constexpr (BF) o.kf = ld2(rec + kf_off);
    }
  };
  auto fetch_b = [&](const float* rec, Ops& o, int j) {
    if constexpr (BF) {
      if (j < 2) {
        o.qb[j] = ldb(rec + lead_off + qd_off + 4 * j);
        o.kb[j] = ldb(rec + lead_off + kd_off + 4 * j);
      }
      if (j == 2) o.qf = ld2(rec + qf_off);
    } else {
      o.qd[j] = ld4(rec + qd_off + 256 * j);
      o.kd[j] = ld4(rec + kd_off + 256 * j);
    }
    if (j < 2) o.in[j] = kPrefetch ? ld4(rec + in_off + (j == 0 ? in_d0 : in_d1)) : ld4(rec + in_off + 512 * j);
  };
  auto fetch = [&](const float* rec, Ops& o) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      fetch_a(rec, o, j);
      fetch_b(rec, o, j);
    }
  };
  // the output of the previous chunk (kh = 0 waves): its first half and intra
  // term in registers, the second half in Opart
  f32x4v out_prev = {0, 0, 0, 0};
  auto store_out = [&](int c) {
    if (kh == 0 && c >= 0) {
      // the four Opart reads go out together, ahead of the stores' branches
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = out_prev[e] + Opart[sx(16 * rt + 4 * fq + e, fm)];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = c * kC + 16 * rt + 4 * fq + e;
        if (t < g.t) g.core[(((int64_t)r * g.t + t) * g.nv + h) * kD + col0 + fm] = o[e];
      }
    }
  };
  // One chunk.  With kPrefetch the next chunk's operands (nrec) load into
  // nxt one phase ahead of their use, a few loads after each group of four
  // MFMAs: phase A loads the next phase A's k_cumdecay, new_values and decay,
  // phase B the next phase B's operands.  Each wave issues 15 16-byte loads
  // per chunk and the CU's load path takes 64 B/clk, so a burst of them
  // would hold every wave's next instruction (and the barrier after it) for
  // about 1.8k cycles; spread out, they issue while the MFMAs run and each
  // has a whole chunk to land.
  auto chunk = [&](int c, Ops& cur, Ops& nxt, const float* nrec) {
    store_out(c - 1);
    // phase A: this wave's half of dk against the state slice; the 16 state
    // operands are read before the first MFMA and reused by (q e^cum) . S
    float sb[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sb[i] = S[sx(4 * (16 * kh + i) + fq, fm)];
    // bf16: q e^cum and k e^(last - cum) are rebuilt here, one k-step group
    // per MFMA group, so the VALU work runs beside the chain and phase B's
    // MFMAs read finished operands; the k factors of this lane's tokens
    // 4m + fq come from the chunk's Kf array in LDS
    // (read ahead of the MFMAs in the prefetching loop; the one-chunk
    // kernel, held to 128 registers, reads each group's just before use)
    f32x4 kf4[BF ? 4 : 1], ek4[BF ? 4 : 1];
    float qdf[BF ? 16 : 1], kdf[BF ? 16 : 1];
    auto k_factors = [&](int j) {
      kf4[j] = *(const f32x4*)(KF + 16 * fq + 4 * j);
      ek4[j] = *(const f32x4*)(KF + kC + 16 * fq + 4 * j);
    };
    if constexpr (BF && kPrefetch) {
#pragma unroll
      for (int j = 0; j < 4; ++j) k_factors(j);
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4v acc = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mma16(cur.kc[j][e], sb[4 * j + e], acc);
      if constexpr (BF) {
        if constexpr (!kPrefetch) k_factors(j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qdf[4 * j + e] = ((float)cur.qb[j >> 1][(j & 1) * 4 + e] * cur.qf[0]) * cur.qf[1];
          kdf[4 * j + e] = ((float)cur.kb[j >> 1][(j & 1) * 4 + e] * kf4[j][e]) * ek4[j][e];
        }
      }
      if (kPrefetch) {
        __builtin_amdgcn_sched_barrier(0);
        fetch_a(nrec, nxt, j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * rt + 4 * fq + e;
      if (kh == 0)
        Vn0[sx(row, fm)] = cur.nvv[e] - acc[e];
      else
        Vn1[sx(row, fm)] = acc[e];
    }
    __syncthreads();
    // phase B
    float vb[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) vb[i] = Vn0[sx(4 * i + fq, fm)] - Vn1[sx(4 * i + fq, fm)];
    __builtin_amdgcn_sched_barrier(0);
    f32x4v su = {0, 0, 0, 0}, ob = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float kd, qd;
        if constexpr (BF) {
          kd = kdf[4 * j + e];
          qd = qdf[4 * j + e];
        } else {
          kd = cur.kd[j][e];
          qd = cur.qd[j][e];
        }
        su = mma16(kd, vb[4 * j + e], su);
        ob = mma16(qd, sb[4 * j + e], ob);
      }
      if (kPrefetch) {
        __builtin_amdgcn_sched_barrier(0);
        fetch_b(nrec, nxt, j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // intra . v_new: intra is lower triangular (K stops at the diagonal
    // block); blocks j = kh, kh + 2 go to this wave so the two halves share it
    // (kh picks the path: a register array indexed by it would live in scratch)
    auto intra = [&](auto kh_c) {
      constexpr int KH = decltype(kh_c)::value;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * jj + KH;
        if (j <= rt) {
#pragma unroll
          for (int e = 0; e < 4; ++e) ob = mma16(cur.in[jj][e], vb[4 * (2 * jj + KH) + e], ob);
        }
      }
    };
    if (kh == 0)
      intra(std::integral_constant<int, 0>{});
    else
      intra(std::integral_constant<int, 1>{});
    if (kh == 0) {
      out_prev = ob;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) Opart[sx(16 * rt + 4 * fq + e, fm)] = ob[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r0 = 16 * wave + 4 * fq + e;
      S[sx(r0, fm)] = S[sx(r0, fm)] * cur.decay + su[e];
    }
    // the next chunk's Kf array, read in its phase A; every wave writes the
    // same values (keeps the load unconditional).  Only the prefetching loop
    // has a next chunk: the one-chunk kernel runs a single chunk.
    if constexpr (BF && kPrefetch) *(f32x2v*)(KF + 2 * lane) = nxt.kf;
    __syncthreads();
  };
  Ops ops_a, ops_b;
  fetch(rec_at(0), ops_a);
  for (int p = tid; p < kD * kW; p += kScanThreads) {
    const int i = p / kW, j = p % kW;
    S[sx(i, j)] = g.s_in ? g.s_in[r * g.s_in_sb + ((int64_t)h * kD + i) * kD + col0 + j] : 0.0f;
  }
  if constexpr (BF) *(f32x2v*)(KF + 2 * lane) = ops_a.kf;  // chunk 0's
  __syncthreads();
  if constexpr (kPrefetch) {
    // Two chunks per iteration so the operand sets alternate without a copy
    // (a copy would wait for every prefetch to land).  The prefetch address
    // is clamped to the last chunk: the loads stay unconditional, because a
    // branch around them made the compiler's wait tracking give up.
    const int last = g.n_chunks - 1;
    int c = 0;
    for (; c + 1 < g.n_chunks; c += 2) {
      chunk(c, ops_a, ops_b, rec_at(c + 1));
      chunk(c + 1, ops_b, ops_a, rec_at(min(c + 2, last)));
    }
    if (c < g.n_chunks) chunk(c, ops_a, ops_b, rec_at(last));
  } else {
    for (int c = 0; c < g.n_chunks; ++c) {
      if (c > 0) fetch(rec_at(c), ops_a);
      chunk(c, ops_a, ops_a, nullptr);
    }
  }
  store_out(g.n_chunks - 1);
  for (int p = tid; p < kD * kW; p += kScanThreads) {
    const int i = p / kW, j = p % kW;
    g.s_out[((int64_t)r * g.nv + h) * kD * kD + (int64_t)i * kD + col0 + j] = S[sx(i, j)];
  }
}

// Many chunks: the prefetching loop (up to 256 VGPRs, one workgroup per CU).
template <bool BF>
__global__ __launch_bounds__(kScanThreads) void gdn_scan_kernel(GdnArgs g) {
  gdn_scan<true, BF>(g);
}
// One chunk per (row, head): no loop to prefetch across, so the registers
// are held to 128 and two workgroups share a CU, one loading while the
// other computes.
template <bool BF>
__global__ __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(4))) void gdn_scan_one_chunk_kernel(GdnArgs g) {
  gdn_scan<false, BF>(g);
}

// ---------------------------------------------------------------------------
// norm: y = core / sqrt(mean core^2 + eps) * w * silu(z), cast to the model
// dtype (qwen35.rs:447-451), all in f32.  The division by the row's norm is
// one reciprocal per row and silu(z) = z / (1 + e^-z) takes the hardware
// exp2 and reciprocal: a few f32 ulps from the reference's op sequence,
// which the output's tolerance covers, for a third of the VALU work (the
// kernel is otherwise bound by it, not by its 134 MB of traffic on a
// 4096-token row).
__device__ __forceinline__ float gated_norm(float c, float inv, float w, float z) {
  const float ez = __builtin_amdgcn_exp2f(z * -1.4426950408889634f);
  return c * inv * w * (z * __builtin_amdgcn_rcpf(1.0f + ez));
}

// One wave per (row, token, value head).
template <typename T>
__global__ __launch_bounds__(256) void gdn_norm_kernel(GdnArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)g.batch * g.t * g.nv) return;
  const int h = (int)(item % g.nv);
  const int64_t rt = item / g.nv;
  const int t = (int)(rt % g.t), r = (int)(rt / g.t);
  // lane holds head-dim elements 2 lane, 2 lane + 1
  const float2 cv = *(const float2*)(g.core + item * kD + 2 * lane);
  float s = cv.x * cv.x + cv.y * cv.y;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float inv = 1.0f / sqrtf(s / (float)kD + g.eps);
  const T* zr = (const T*)g.z + r * g.z_sb + (int64_t)t * g.z_st + h * kD + 2 * lane;
  T* yr = (T*)g.y + r * g.y_sb + (int64_t)t * g.y_st + h * kD + 2 * lane;
  const float2 wv = *(const float2*)(g.norm_w + 2 * lane);
  const float c2[2] = {cv.x, cv.y}, w2[2] = {wv.x, wv.y};
#pragma unroll
  for (int e = 0; e < 2; ++e) yr[e] = from_f<T>(gated_norm(c2[e], inv, w2[e], to_f(zr[e])));
}

// The same with 16 lanes per (row, token, value head), 8 elements each:
// 16-byte loads and stores, the sum of squares over the row by DPP.  Each
// 16-lane group takes kNormRows rows, 16 rows apart so that every load
// instruction of the workgroup covers 16 consecutive rows, and issues all
// their core and z loads before the first sum.  Needs z and y rows 16-byte
// aligned (checked by the launcher).
constexpr int kNormRows = 2;

template <typename T>
__global__ __launch_bounds__(256) void gdn_norm_vec_kernel(GdnArgs g) {
  const int sub = threadIdx.x & 15;
  const int64_t n_items = (int64_t)g.batch * g.t * g.nv;
  const int64_t first = (int64_t)blockIdx.x * (16 * kNormRows) + (threadIdx.x >> 4);
  f32x4 c0[kNormRows], c1[kNormRows];
  float zv[kNormRows][8];
  int64_t yoff[kNormRows];
#pragma unroll
  for (int k = 0; k < kNormRows; ++k) {
    // rows past the end recompute the last row (the DPP sum needs all 16
    // lanes of a row) and store nothing
    const int64_t item = first + 16 * k;
    const int64_t it = item < n_items ? item : n_items - 1;
    const int h = (int)(it % g.nv);
    const int64_t rt = it / g.nv;
    const int t = (int)(rt % g.t), r = (int)(rt / g.t);
    const float* cp = g.core + it * kD + 8 * sub;
    c0[k] = *(const f32x4*)cp;
    c1[k] = *(const f32x4*)(cp + 4);
    load8<T>((const T*)g.z + r * g.z_sb + (int64_t)t * g.z_st + h * kD + 8 * sub, zv[k]);
    yoff[k] = r * g.y_sb + (int64_t)t * g.y_st + h * kD + 8 * sub;
  }
  const f32x4 w0 = *(const f32x4*)(g.norm_w + 8 * sub), w1 = *(const f32x4*)(g.norm_w + 8 * sub + 4);
  const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
  for (int k = 0; k < kNormRows; ++k) {
    const float cv[8] = {c0[k][0], c0[k][1], c0[k][2], c0[k][3], c1[k][0], c1[k][1], c1[k][2], c1[k][3]};
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += cv[e] * cv[e];
    const float inv = 1.0f / sqrtf(row16_sum(s) / (float)kD + g.eps);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = gated_norm(cv[e], inv, wv[e], zv[k][e]);
    if (first + 16 * k < n_items) store8<T>((T*)g.y + yoff[k], y);
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct GdnLayout {
  size_t conved, rec, core, total;
};

GdnLayout gdn_layout(const cev_gdn_desc* d) {
  const size_t esz = d->dtype == CEV_BF16 ? 2 : 4;
  const int64_t conv_dim = 2LL * d->n_k_heads * d->head_k_dim + (int64_t)d->n_v_heads * d->head_v_dim;
  const int64_t n_chunks = (d->t + kC - 1) / kC;
  GdnLayout L;
  L.conved = 0;
  L.rec = align256((size_t)d->batch * d->t * conv_dim * esz);
  L.core = L.rec + align256((size_t)d->batch * d->n_v_heads * n_chunks * kRecFloats * sizeof(float));
  L.total = L.core + align256((size_t)d->batch * d->t * d->n_v_heads * d->head_v_dim * sizeof(float));
  return L;
}

int32_t check_gdn(const cev_gdn_desc* d) {
  CEV_CHECK_ARG(d != nullptr, "null GDN descriptor");
  if (d->dtype != CEV_F32 && d->dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "dtype %d not supported", d->dtype);
  CEV_CHECK_ARG(d->batch >= 1 && d->t >= 1, "batch %d and t %d must be positive", d->batch, d->t);
  CEV_CHECK_ARG(d->n_k_heads >= 1 && d->n_v_heads >= 1 && d->n_v_heads % d->n_k_heads == 0,
                "n_v_heads %d must be a positive multiple of n_k_heads %d", d->n_v_heads, d->n_k_heads);
  if (d->head_k_dim != kD || d->head_v_dim != kD)
    return cev_fail(CEV_ERR_UNSUPPORTED, "head dims %d x %d not supported (128 x 128)", d->head_k_dim, d->head_v_dim);
  CEV_CHECK_ARG(d->conv_kernel >= 2 && d->conv_kernel <= 8, "conv_kernel %d outside [2, 8]", d->conv_kernel);
  CEV_CHECK_ARG(d->eps >= 0.0f && d->eps <= 3.4e38f, "eps must be finite and non-negative");
  const int64_t* st[] = {&d->mixed_stride_b, &d->mixed_stride_t, &d->z_stride_b, &d->z_stride_t, &d->ab_stride_b,
                         &d->ab_stride_t, &d->conv_in_stride_b, &d->s_in_stride_b, &d->y_stride_b, &d->y_stride_t};
  for (const int64_t* s : st) CEV_CHECK_ARG(*s >= 0, "negative stride");
  const int64_t conv_dim = 2LL * d->n_k_heads * kD + (int64_t)d->n_v_heads * kD;
  CEV_CHECK_ARG(d->mixed_stride_t >= conv_dim && d->z_stride_t >= (int64_t)d->n_v_heads * kD && d->ab_stride_t >= d->n_v_heads &&
                    d->y_stride_t >= (int64_t)d->n_v_heads * kD,
                "row strides shorter than the rows");
  return CEV_OK;
}

}  // namespace

extern "C" int32_t cev_gdn_desc_init(cev_gdn_desc* d, int32_t dtype, int32_t batch, int32_t t, int32_t n_k_heads, int32_t n_v_heads,
                                     int32_t head_k_dim, int32_t head_v_dim, int32_t conv_kernel, float eps) {
  CEV_CHECK_ARG(d != nullptr, "cev_gdn_desc_init: null descriptor");
  memset(d, 0, sizeof(*d));
  d->dtype = dtype;
  d->batch = batch;
  d->t = t;
  d->n_k_heads = n_k_heads;
  d->n_v_heads = n_v_heads;
  d->head_k_dim = head_k_dim;
  d->head_v_dim = head_v_dim;
  d->conv_kernel = conv_kernel;
  d->eps = eps;
  const int64_t conv_dim = 2LL * n_k_heads * head_k_dim + (int64_t)n_v_heads * head_v_dim;
  const int64_t vdim = (int64_t)n_v_heads * head_v_dim;
  d->mixed_stride_t = conv_dim;
  d->mixed_stride_b = conv_dim * t;
  d->z_stride_t = vdim;
  d->z_stride_b = vdim * t;
  d->ab_stride_t = n_v_heads;
  d->ab_stride_b = (int64_t)n_v_heads * t;
  d->conv_in_stride_b = conv_dim * (conv_kernel - 1);
  d->s_in_stride_b = (int64_t)n_v_heads * head_k_dim * head_v_dim;
  d->y_stride_t = vdim;
  d->y_stride_b = vdim * t;
  return check_gdn(d);
}

extern "C" int32_t cev_gdn_workspace_size(const cev_gdn_desc* d, size_t* bytes) {
  int32_t rc = check_gdn(d);
  if (rc) return rc;
  CEV_CHECK_ARG(bytes != nullptr, "cev_gdn_workspace_size: null output");
  *bytes = gdn_layout(d).total;
  return CEV_OK;
}

extern "C" int32_t cev_gdn_forward(const cev_gdn_desc* d, const void* mixed, const void* z, const void* b, const void* a,
                                   const void* conv_w, const float* neg_a, const float* dt_bias, const float* norm_w,
                                   const void* conv_in, const float* s_in, void* y, void* conv_out, float* s_out, void* workspace,
                                   size_t workspace_bytes, cev_stream stream) {
  int32_t rc = check_gdn(d);
  if (rc) return rc;
  CEV_CHECK_ARG(mixed && z && b && a && conv_w && neg_a && dt_bias && norm_w && y && conv_out && s_out,
                "cev_gdn_forward: null input or output");
  const GdnLayout L = gdn_layout(d);
  CEV_CHECK_ARG(workspace != nullptr, "cev_gdn_forward: null workspace");
  if (workspace_bytes < L.total) return cev_fail(CEV_ERR_SPACE, "workspace of %zu bytes, the layer needs %zu", workspace_bytes, L.total);
  const size_t esz = d->dtype == CEV_BF16 ? 2 : 4;
  const uintptr_t al = esz * 8 - 1;  // 8-element vector reads of the conv input
  CEV_CHECK_ARG(((uintptr_t)mixed & al) == 0 && (d->mixed_stride_t % 8) == 0 && (d->mixed_stride_b % 8) == 0,
                "cev_gdn_forward: the conv input rows must be 8-element aligned");
  CEV_CHECK_ARG(((uintptr_t)workspace & 255) == 0, "cev_gdn_forward: workspace must be 256-byte aligned");
  CEV_CHECK_ARG(((uintptr_t)norm_w & 7) == 0, "cev_gdn_forward: norm_w must be 8-byte aligned");
  GdnArgs g;
  g.mixed = mixed;
  g.z = z;
  g.b = b;
  g.a = a;
  g.conv_w = conv_w;
  g.neg_a = neg_a;
  g.dt_bias = dt_bias;
  g.norm_w = norm_w;
  g.conv_in = conv_in;
  g.s_in = s_in;
  g.y = y;
  g.conv_out = conv_out;
  g.s_out = s_out;
  g.conved = (char*)workspace + L.conved;
  g.rec = (float*)((char*)workspace + L.rec);
  g.core = (float*)((char*)workspace + L.core);
  g.mixed_sb = d->mixed_stride_b;
  g.mixed_st = d->mixed_stride_t;
  g.z_sb = d->z_stride_b;
  g.z_st = d->z_stride_t;
  g.ab_sb = d->ab_stride_b;
  g.ab_st = d->ab_stride_t;
  g.conv_in_sb = d->conv_in_stride_b;
  g.s_in_sb = d->s_in_stride_b;
  g.y_sb = d->y_stride_b;
  g.y_st = d->y_stride_t;
  g.batch = d->batch;
  g.t = d->t;
  g.nk = d->n_k_heads;
  g.nv = d->n_v_heads;
  g.kernel = d->conv_kernel;
  g.conv_dim = 2 * d->n_k_heads * kD + d->n_v_heads * kD;
  g.n_chunks = (d->t + kC - 1) / kC;
  g.eps = d->eps;
  hipStream_t s = (hipStream_t)stream;
  const int conv_wg = conv_threads(g.kernel);
  auto conv_items_of = [&](int run) { return (int64_t)g.batch * ((g.t + run - 1) / run) * (g.conv_dim / 8); };
  g.conv_run = kConvRunMax;
  while (g.conv_run > 4 && conv_items_of(g.conv_run) < (int64_t)kConvCus * conv_wg) g.conv_run /= 2;
  const int64_t conv_items = conv_items_of(g.conv_run);
  const int64_t recs = (int64_t)g.batch * g.nv * g.n_chunks;
  // scan grid: (bf16, many chunks) groups of value heads per key head, rounded up to the 8 XCDs, x group size x slices
  const int64_t grp = d->dtype == CEV_BF16 && g.n_chunks > 1 ? g.nv / g.nk : 1;
  const int64_t slices = ((int64_t)g.batch * g.nv / grp + kXcds - 1) / kXcds * kXcds * grp * (kD / kW);
  const int64_t norm_items = (int64_t)g.batch * g.t * g.nv;
  if (recs > INT32_MAX || (conv_items + 511) / 512 > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "GDN grid too large");
  if (d->dtype == CEV_BF16) {
    launch_conv<__bf16>(g, conv_items, s);
    hipLaunchKernelGGL(gdn_prep_kernel<__bf16>, dim3((unsigned)recs), dim3(kPrepThreads), 0, s, g);
  } else {
    launch_conv<float>(g, conv_items, s);
    hipLaunchKernelGGL(gdn_prep_kernel<float>, dim3((unsigned)recs), dim3(kPrepThreads), 0, s, g);
  }
  const bool bf = d->dtype == CEV_BF16;
  if (g.n_chunks > 1) {
    if (bf)
      hipLaunchKernelGGL(gdn_scan_kernel<true>, dim3((unsigned)slices), dim3(kScanThreads), 0, s, g);
    else
      hipLaunchKernelGGL(gdn_scan_kernel<false>, dim3((unsigned)slices), dim3(kScanThreads), 0, s, g);
  } else {
    if (bf)
      hipLaunchKernelGGL(gdn_scan_one_chunk_kernel<true>, dim3((unsigned)slices), dim3(kScanThreads), 0, s, g);
    else
      hipLaunchKernelGGL(gdn_scan_one_chunk_kernel<false>, dim3((unsigned)slices), dim3(kScanThreads), 0, s, g);
  }
  // 16-byte aligned rows of z and y (and norm_w) for the vector norm
  const int64_t vec = d->dtype == CEV_BF16 ? 8 : 4;
  const bool norm_vec = ((uintptr_t)g.z | (uintptr_t)g.y | (uintptr_t)g.norm_w) % 16 == 0 && g.z_sb % vec == 0 && g.z_st % vec == 0 &&
                        g.y_sb % vec == 0 && g.y_st % vec == 0;
  if (norm_vec) {
    const dim3 grid((unsigned)((norm_items + 16 * kNormRows - 1) / (16 * kNormRows)));
    if (d->dtype == CEV_BF16)
      hipLaunchKernelGGL(gdn_norm_vec_kernel<__bf16>, grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL(gdn_norm_vec_kernel<float>, grid, dim3(256), 0, s, g);
  } else if (d->dtype == CEV_BF16) {
    hipLaunchKernelGGL(gdn_norm_kernel<__bf16>, dim3((unsigned)((norm_items + 3) / 4)), dim3(256), 0, s, g);
  } else {
    hipLaunchKernelGGL(gdn_norm_kernel<float>, dim3((unsigned)((norm_items + 3) / 4)), dim3(256), 0, s, g);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "GDN launch: %s", hipGetErrorString(e));
  return CEV_OK;
}
