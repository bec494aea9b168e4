// Linear layers and row gathers around the attention path: the candle ops
// that surround Attention::attend in the reference's forward passes.
//   cev_linear      x . w^T (+ scale): Linear::forward of the q/k/v/o
//                   projections and the MLP (crates/cev-model/src/qwen3.rs:175-178,
//                   :229-233), the code head (crates/cev-model/src/engine.rs:463)
//                   and the d3 readout `answers.matmul(weight.t()) / temperature`
//                   (crates/cev-model/src/hybrid.rs:657).
//   cev_gather_rows table rows by index with a dtype conversion: Embedding
//                   rows (qwen3.rs:288-293), the gather of the answer rows
//                   (qwen3.rs:399, hybrid.rs:634), `to_dtype(F32)`
//                   (qwen3.rs:400) and the code head's rows of the tied
//                   embedding (engine.rs:155).
//
// Row counts of up to kRowsSmall (decode-like readouts, the code head of a
// few questions) run on this file's own kernel, which streams every weight
// row once; larger products are plain library GEMMs (hipBLASLt), f32
// accumulation, the result rounded once to the output dtype as candle's
// matmul does.
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <type_traits>
#include <vector>

#include "cev_device.h"
#include "cev_internal.h"

namespace {

constexpr int kRowsSmall = 8;
constexpr int kLinWaves = 4;  // output columns per workgroup of the small-row kernel

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t x) {
  return bf16_from_bits(x);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float x) {
  return bf16_bits(x);
}

struct LinArgs {
  const void* x;
  const void* w;
  void* y;
  int64_t m, n, k, ldx, ldw, ldy;
  float alpha;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One wave per output column j: the lanes stream w's row j in 16-byte
// chunks (read once), multiply it with each of the m <= MR input rows (hot
// in L2) and reduce across the wave.  f32 accumulation; k a multiple of the
// 16-byte chunk (checked by the launcher).  A lane's chunks are loaded NB at
// a time with clamped indices (rows past m read row m - 1, chunks past k the
// last chunk), so every load of a batch is unconditional and in flight
// together; only the accumulation skips them.  Each lane still adds its
// chunks in order.
template <typename T, typename TO, int MR, int NB>
__global__ __launch_bounds__(kLinWaves * 64) void linear_rows_kernel(LinArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const int lane = threadIdx.x & 63;
  const int64_t j = (int64_t)blockIdx.x * kLinWaves + (threadIdx.x >> 6);
  if (j >= a.n) return;
  const T* wr = (const T*)a.w + j * a.ldw;
  float acc[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) acc[r] = 0.0f;
  for (int64_t e0 = (int64_t)lane * VEC; e0 < a.k; e0 += (int64_t)NB * 64 * VEC) {
    uint4 wv[NB], xv[MR][NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int64_t ec = min(e0 + (int64_t)b * 64 * VEC, a.k - VEC);
      wv[b] = *(const uint4*)(wr + ec);
#pragma unroll
      for (int r = 0; r < MR; ++r) xv[r][b] = *(const uint4*)((const T*)a.x + (int64_t)min(r, (int)a.m - 1) * a.ldx + ec);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (e0 + (int64_t)b * 64 * VEC < a.k) {
        const T* w8 = (const T*)&wv[b];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const T* x8 = (const T*)&xv[r][b];
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[r] = __builtin_fmaf(to_f32<T>(x8[i]), to_f32<T>(w8[i]), acc[r]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    const float s = wave_sum(acc[r]);
    if (r < a.m && lane == 0) ((TO*)a.y)[r * a.ldy + j] = from_f32<TO>(s * a.alpha);
  }
}

struct GatherArgs {
  const void* table;
  const int32_t* ids;
  void* out;
  int64_t n, width, ld_table, table_rows, ld_out;
};

// One thread per element: out[i][e] = table[ids[i]][e] in the output dtype;
// an index outside the table gives a NaN row instead of a stray read.
template <typename T, typename TO>
__global__ __launch_bounds__(256) void gather_rows_kernel(GatherArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.n * a.width) return;
  const int64_t i = idx / a.width, e = idx % a.width;
  const int64_t r = a.ids ? (int64_t)a.ids[i] : i;
  const float v = (r >= 0 && r < a.table_rows) ? to_f32<T>(((const T*)a.table)[r * a.ld_table + e]) : __builtin_nanf("");
  ((TO*)a.out)[i * a.ld_out + e] = from_f32<TO>(v);
}

// hipBLASLt state of one cev_blas handle: the library handle and, per
// problem shape, the matmul descriptor, layouts and the heuristic's algo.
// al256: x, w and y all 256-byte aligned (the alignment the picks below
// were measured at); part of the key, so a plan is never reused on less
// aligned operands than it was made for.
struct GemmKey {
  int dtype, out_dtype;
  int64_t m, n, k, ldx, ldw, ldy;
  size_t ws;
  bool al256;
  bool operator<(const GemmKey& o) const {
    return std::tie(dtype, out_dtype, m, n, k, ldx, ldw, ldy, ws, al256) <
           std::tie(o.dtype, o.out_dtype, o.m, o.n, o.k, o.ldx, o.ldw, o.ldy, o.ws, o.al256);
  }
};
struct GemmPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo;
  size_t ws = 0;
};

// Per-shape algorithm picks for bf16 projections of the config-2 pass
// (Qwen3-1.7B: 3584 pass tokens), measured offline with gemm_probe.cpp
// (make gemm-probe): the fastest candidate's hipBLASLt solution index and
// the FNV-1a hash of its kernel name, with the probe's median times of the
// heuristic's first pick and of the pick, in us.  Indices number the
// kernels of one loaded hipBLASLt instance: a pick is used only where its
// index names the same kernel (by hash) in the instance this process
// loaded.  The entries are ROCm 7.2's hipBLASLt (what a host that does not
// load torch binds to); in a torch process libcev_hip.so binds to torch's
// own copy, whose heuristic first picks the probe measured within 2 % of
// its fastest candidate on these shapes, so it has no entries.
// The probe ran every candidate on exactly these shapes and layouts
// (leading dimensions k, k and n, bf16 output, 256-byte aligned operands,
// the 32 MiB workspace); a pick applies to nothing else.  Before use it
// must come back from getAlgosFromIndex, name the recorded kernel and pass
// matmulIsAlgoSupported for the call's layouts with a workspace no larger
// than the caller's; otherwise the heuristic's first pick stays.  The
// library never times candidates itself.
struct GemmPick {
  int64_t m, n, k;
  int index;
  uint64_t name_hash;
};
constexpr GemmPick kPicks[] = {
    {3584, 4096, 2048, 440058, 0x2d1baa9a7bbf205aull},  // q/k/v projection   48.1 -> 45.8
    {3584, 2048, 2048, 440090, 0x1eb4eec7c4241052ull},  // o_proj             34.6 -> 28.0
    {3584, 2048, 6144, 440091, 0x58ff78e43625b963ull},  // down               103.6 -> 74.2
};

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

const GemmPick* find_pick(const GemmKey& key) {
  if (key.dtype != CEV_BF16 || key.out_dtype != CEV_BF16 || !key.al256 || key.ldx != key.k || key.ldw != key.k || key.ldy != key.n)
    return nullptr;
  for (const GemmPick& p : kPicks)
    if (p.m == key.m && p.n == key.n && p.k == key.k) return &p;
  return nullptr;
}
struct Blas {
  hipblasLtHandle_t lt = nullptr;
  std::mutex mu;
  std::map<GemmKey, GemmPlan> plans;
};

hipDataType hip_type(int dtype) { return dtype == CEV_BF16 ? HIP_R_16BF : HIP_R_32F; }

int32_t blas_status(hipblasStatus_t st, const char* what) {
  if (st == HIPBLAS_STATUS_SUCCESS) return CEV_OK;
  return cev_fail(st == HIPBLAS_STATUS_NOT_SUPPORTED ? CEV_ERR_UNSUPPORTED : CEV_ERR_HIP, "cev_linear: %s failed (hipBLAS status %d)", what,
                  (int)st);
}

void destroy_plan(GemmPlan& p) {
  if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
  if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
  if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
}

// y (m, n) row-major is y^T (n, m) column-major = w (n, k) . x^T: A = w
// read as a (k, n) column-major matrix, transposed; B = x read as (k, m).
int32_t gemm_plan(Blas& b, const GemmKey& key, GemmPlan** out) {
  auto it = b.plans.find(key);
  if (it != b.plans.end()) {
    *out = &it->second;
    return CEV_OK;
  }
  GemmPlan p;
  int32_t rc = blas_status(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "hipblasLtMatmulDescCreate");
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (!rc) rc = blas_status(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta), "TRANSA");
  if (!rc) rc = blas_status(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb), "TRANSB");
  if (!rc) rc = blas_status(hipblasLtMatrixLayoutCreate(&p.la, hip_type(key.dtype), key.k, key.n, key.ldw), "layout A");
  if (!rc) rc = blas_status(hipblasLtMatrixLayoutCreate(&p.lb, hip_type(key.dtype), key.k, key.m, key.ldx), "layout B");
  if (!rc) rc = blas_status(hipblasLtMatrixLayoutCreate(&p.lc, hip_type(key.out_dtype), key.n, key.m, key.ldy), "layout C");
  hipblasLtMatmulPreference_t pref = nullptr;
  if (!rc) rc = blas_status(hipblasLtMatmulPreferenceCreate(&pref), "preference");
  const uint64_t ws = key.ws;
  if (!rc)
    rc = blas_status(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof ws), "workspace pref");
  hipblasLtMatmulHeuristicResult_t heur[1];
  int found = 0;
  if (!rc)
    rc = blas_status(hipblasLtMatmulAlgoGetHeuristic(b.lt, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, heur, &found), "heuristic");
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (!rc && found < 1) rc = cev_fail(CEV_ERR_UNSUPPORTED, "cev_linear: hipBLASLt has no kernel for this product");
  if (rc) {
    destroy_plan(p);
    return rc;
  }
  p.algo = heur[0].algo;
  p.ws = heur[0].workspaceSize;
  if (const GemmPick* pk = find_pick(key)) {
    std::vector<int> idx{pk->index};
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    const float one = 1.0f, zero = 0.0f;
    size_t need = 0;
    if (hipblaslt_ext::getAlgosFromIndex(b.lt, idx, res) == HIPBLAS_STATUS_SUCCESS && !res.empty() &&
        fnv1a(hipblaslt_ext::getKernelNameFromAlgo(b.lt, res[0].algo)) == pk->name_hash &&
        hipblaslt_ext::matmulIsAlgoSupported(b.lt, p.desc, &one, p.la, p.lb, &zero, p.lc, p.lc, res[0].algo, need) ==
            HIPBLAS_STATUS_SUCCESS &&
        need <= key.ws) {
      p.algo = res[0].algo;
      p.ws = need;
    }
  }
  *out = &(b.plans[key] = p);
  return CEV_OK;
}

bool aligned256(const void* p) { return ((uintptr_t)p & 255) == 0; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
int32_t launch_rows(const LinArgs& a, int out_dtype, hipStream_t s) {
  const dim3 grid((unsigned)((a.n + kLinWaves - 1) / kLinWaves)), block(kLinWaves * 64);
  // rows held per lane and chunks loaded per batch: fewer rows, deeper batches
  auto go = [&](auto mr_c, auto nb_c) {
    constexpr int MR = decltype(mr_c)::value, NB = decltype(nb_c)::value;
    if (out_dtype == CEV_F32)
      hipLaunchKernelGGL((linear_rows_kernel<T, float, MR, NB>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((linear_rows_kernel<T, T, MR, NB>), grid, block, 0, s, a);
  };
  using std::integral_constant;
  if (a.m <= 1)
    go(integral_constant<int, 1>{}, integral_constant<int, 8>{});
  else if (a.m <= 2)
    go(integral_constant<int, 2>{}, integral_constant<int, 8>{});
  else if (a.m <= 4)
    go(integral_constant<int, 4>{}, integral_constant<int, 4>{});
  else
    go(integral_constant<int, kRowsSmall>{}, integral_constant<int, 4>{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_linear launch: %s", hipGetErrorString(e));
  return CEV_OK;
}

}  // namespace

extern "C" int32_t cev_blas_create(cev_blas* handle) {
  CEV_CHECK_ARG(handle != nullptr, "cev_blas_create: null output");
  Blas* b = new Blas;
  int32_t rc = blas_status(hipblasLtCreate(&b->lt), "hipblasLtCreate");
  if (rc) {
    delete b;
    return rc;
  }
  *handle = b;
  return CEV_OK;
}

extern "C" int32_t cev_blas_destroy(cev_blas handle) {
  if (!handle) return CEV_OK;
  Blas* b = (Blas*)handle;
  for (auto& kv : b->plans) destroy_plan(kv.second);
  int32_t rc = blas_status(hipblasLtDestroy(b->lt), "hipblasLtDestroy");
  delete b;
  return rc;
}

extern "C" int32_t cev_linear(cev_blas handle, int32_t dtype, int32_t out_dtype, int64_t m, int64_t n, int64_t k, const void* x, int64_t ldx,
                              const void* w, int64_t ldw, float alpha, void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                              cev_stream stream) {
  if (dtype != CEV_F32 && dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_linear: dtype %d", dtype);
  if (out_dtype != CEV_F32 && out_dtype != dtype)
    return cev_fail(CEV_ERR_UNSUPPORTED, "cev_linear: output dtype %d for input dtype %d", out_dtype, dtype);
  const int vec = dtype == CEV_BF16 ? 8 : 4;
  CEV_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "cev_linear: negative size");
  CEV_CHECK_ARG(k % vec == 0, "cev_linear: k %lld must be a multiple of %d", (long long)k, vec);
  CEV_CHECK_ARG(std::isfinite(alpha), "cev_linear: alpha must be finite");
  if (m == 0 || n == 0) return CEV_OK;
  CEV_CHECK_ARG(x && w && y, "cev_linear: null buffer");
  CEV_CHECK_ARG(ldx >= k && ldw >= k && ldy >= n && ldx % vec == 0 && ldw % vec == 0, "cev_linear: leading dimensions");
  CEV_CHECK_ARG(aligned16(x) && aligned16(w), "cev_linear: x and w must be 16-byte aligned");
  CEV_CHECK_ARG(n <= INT32_MAX && m <= INT32_MAX && k <= INT32_MAX, "cev_linear: size beyond int32");
  hipStream_t s = (hipStream_t)stream;
  if (k == 0 || m <= kRowsSmall) {
    if (k == 0) CEV_CHECK_ARG(m <= kRowsSmall, "cev_linear: k = 0 supported for at most %d rows", kRowsSmall);
    const int64_t grid = (n + kLinWaves - 1) / kLinWaves;
    if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_linear: n too large");
    LinArgs a{x, w, y, m, n, k, ldx, ldw, ldy, alpha};
    if (dtype == CEV_BF16) return launch_rows<uint16_t>(a, out_dtype, s);
    return launch_rows<float>(a, out_dtype, s);
  }
  // The hipBLASLt algorithm is chosen once per shape and kept, so every
  // operand of that path meets the same alignment (the cached choice never
  // meets a less aligned y than it was chosen for).
  const int ovec = out_dtype == CEV_BF16 ? 8 : 4;
  CEV_CHECK_ARG(aligned16(y) && ldy % ovec == 0, "cev_linear: with more than %d rows y must be 16-byte aligned and ldy a multiple of %d",
                kRowsSmall, ovec);
  CEV_CHECK_ARG(handle != nullptr, "cev_linear: more than %d rows need a cev_blas handle", kRowsSmall);
  CEV_CHECK_ARG(workspace_bytes == 0 || workspace != nullptr, "cev_linear: null workspace of %zu bytes", workspace_bytes);
  Blas* b = (Blas*)handle;
  std::lock_guard<std::mutex> lock(b->mu);
  GemmPlan* p = nullptr;
  const bool al256 = aligned256(x) && aligned256(w) && aligned256(y);
  int32_t rc = gemm_plan(*b, GemmKey{dtype, out_dtype, m, n, k, ldx, ldw, ldy, workspace_bytes, al256}, &p);
  if (rc) return rc;
  const float beta = 0.0f;
  return blas_status(hipblasLtMatmul(b->lt, p->desc, &alpha, w, p->la, x, p->lb, &beta, y, p->lc, y, p->lc, &p->algo, workspace,
                                     workspace_bytes, s),
                     "hipblasLtMatmul");
}

extern "C" int32_t cev_gather_rows(int32_t dtype, int32_t out_dtype, int64_t n, int64_t width, const void* table, int64_t ld_table,
                                   int64_t table_rows, const int32_t* ids, void* out, int64_t ld_out, cev_stream stream) {
  if (dtype != CEV_F32 && dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_gather_rows: dtype %d", dtype);
  if (out_dtype != CEV_F32 && out_dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_gather_rows: output dtype %d", out_dtype);
  CEV_CHECK_ARG(n >= 0 && width >= 0 && table_rows >= 0, "cev_gather_rows: negative size");
  if (n == 0 || width == 0) return CEV_OK;
  CEV_CHECK_ARG(table && out, "cev_gather_rows: null buffer");
  CEV_CHECK_ARG(ld_table >= width && ld_out >= width, "cev_gather_rows: leading dimensions");
  CEV_CHECK_ARG(ids || n <= table_rows, "cev_gather_rows: %lld rows from a %lld-row table without ids", (long long)n,
                (long long)table_rows);
  const int64_t grid = (n * width + 255) / 256;
  if (grid > INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_gather_rows: too many elements");
  GatherArgs a{table, ids, out, n, width, ld_table, table_rows, ld_out};
  hipStream_t s = (hipStream_t)stream;
  const dim3 g((unsigned)grid), blk(256);
  if (dtype == CEV_BF16 && out_dtype == CEV_BF16)
    hipLaunchKernelGGL((gather_rows_kernel<uint16_t, uint16_t>), g, blk, 0, s, a);
  else if (dtype == CEV_BF16)
    hipLaunchKernelGGL((gather_rows_kernel<uint16_t, float>), g, blk, 0, s, a);
  else if (out_dtype == CEV_BF16)
    hipLaunchKernelGGL((gather_rows_kernel<float, uint16_t>), g, blk, 0, s, a);
  else
    hipLaunchKernelGGL((gather_rows_kernel<float, float>), g, blk, 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return cev_fail(CEV_ERR_HIP, "cev_gather_rows launch: %s", hipGetErrorString(e));
  return CEV_OK;
}
