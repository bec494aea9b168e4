// Offline probe of hipBLASLt's candidates for the bf16 projections of the
// config-2 pass (Qwen3-1.7B shapes: hidden 2048, q/k/v 4096 wide, gate/up
// 12288 wide, down from 6144), laid out as cev_linear lays them out: y (m, n)
// = x (m, k) . w (n, k)^T, row-major, leading dimensions k, k and n, f32
// accumulation, the cev_linear workspace of 32 MiB.
//
// For every shape it asks the heuristic for up to 16 candidates, keeps those
// that hipblaslt_ext::matmulIsAlgoSupported accepts with a workspace of at
// most 32 MiB, times them round-robin over seeded N(0,1) operands (median
// of 7 rounds of 20 runs each) and prints one `pick` line per shape: the
// solution index of the fastest candidate and the times of it and of the
// heuristic's first pick.  The picks table in
// linear.hip is copied from those lines; the library itself never times
// candidates.
//
// Solution indices belong to the hipBLASLt instance that is loaded: a
// process that imports torch first runs libcev_hip.so on torch's own
// libhipblaslt.so (same soname, its own kernel set and numbering), any other
// process on ROCm's.  So the probe runs once in each setting and prints the
// kernel name's hash beside each index; linear.hip uses a pick only where
// the index names that kernel in the loaded instance.
//   make gemm-probe
//   build/gemm_probe [m ...]                         ROCm's hipBLASLt
//   python3 gemm_probe.py [m ...]                    torch's (imports torch, then
//                                                    calls cev_gemm_probe in
//                                                    build/libgemm_probe.so)
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#define CHECK_HIP(x)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)
#define CHECK_BLAS(x)                                                          \
  do {                                                                         \
    hipblasStatus_t s_ = (x);                                                  \
    if (s_ != HIPBLAS_STATUS_SUCCESS) {                                        \
      fprintf(stderr, "%s:%d %s: status %d\n", __FILE__, __LINE__, #x, (int)s_); \
      exit(1);                                                                 \
    }                                                                          \
  } while (0)

namespace {

constexpr size_t kWorkspace = (size_t)32 << 20;

uint16_t to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)u;
}

void fill(void* dev, size_t n, uint32_t seed) {
  std::mt19937 rng(seed);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  std::vector<uint16_t> h(n);
  for (auto& v : h) v = to_bf16(nd(rng));
  CHECK_HIP(hipMemcpy(dev, h.data(), n * 2, hipMemcpyHostToDevice));
}

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

struct Shape {
  const char* name;
  int64_t n, k;
};

}  // namespace

extern "C" int cev_gemm_probe(int argc, const char* const* argv) {
  std::vector<int64_t> ms;
  for (int i = 0; i < argc; ++i) ms.push_back(atoll(argv[i]));
  if (ms.empty()) ms = {3584, 512};  // the pass (512 tail + 48 x 64 questions) and a prefill chunk
  const Shape shapes[] = {{"qkv", 4096, 2048}, {"o_proj", 2048, 2048}, {"gate_up", 12288, 2048}, {"down", 2048, 6144}};
  const int64_t max_m = *std::max_element(ms.begin(), ms.end());

  void *x, *w, *y, *ws;
  CHECK_HIP(hipMalloc(&x, (size_t)max_m * 6144 * 2));
  CHECK_HIP(hipMalloc(&w, (size_t)12288 * 6144 * 2));
  CHECK_HIP(hipMalloc(&y, (size_t)max_m * 12288 * 2));
  CHECK_HIP(hipMalloc(&ws, kWorkspace));
  fill(x, (size_t)max_m * 6144, 1);
  fill(w, (size_t)12288 * 6144, 2);
  hipStream_t s;
  CHECK_HIP(hipStreamCreate(&s));
  hipEvent_t e0, e1;
  CHECK_HIP(hipEventCreate(&e0));
  CHECK_HIP(hipEventCreate(&e1));
  hipblasLtHandle_t lt;
  CHECK_BLAS(hipblasLtCreate(&lt));
  int version = 0;
  CHECK_BLAS(hipblasLtGetVersion(lt, &version));
  printf("hipBLASLt version %d\n", version);

  const float alpha = 1.0f, beta = 0.0f;
  for (int64_t m : ms) {
    for (const Shape& sh : shapes) {
      const int64_t n = sh.n, k = sh.k;
      hipblasLtMatmulDesc_t desc;
      hipblasLtMatrixLayout_t la, lb, lc;
      CHECK_BLAS(hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
      const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
      CHECK_BLAS(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta));
      CHECK_BLAS(hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb));
      CHECK_BLAS(hipblasLtMatrixLayoutCreate(&la, HIP_R_16BF, k, n, k));
      CHECK_BLAS(hipblasLtMatrixLayoutCreate(&lb, HIP_R_16BF, k, m, k));
      CHECK_BLAS(hipblasLtMatrixLayoutCreate(&lc, HIP_R_16BF, n, m, n));
      hipblasLtMatmulPreference_t pref;
      CHECK_BLAS(hipblasLtMatmulPreferenceCreate(&pref));
      const uint64_t wsb = kWorkspace;
      CHECK_BLAS(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof wsb));
      hipblasLtMatmulHeuristicResult_t heur[16];
      int found = 0;
      CHECK_BLAS(hipblasLtMatmulAlgoGetHeuristic(lt, desc, la, lb, lc, lc, pref, 16, heur, &found));
      hipblasLtMatmulPreferenceDestroy(pref);

      // Candidates the check accepts, then timed round-robin: every round
      // runs each candidate 20 times, and a candidate's time is its median
      // over the rounds (a candidate timed alone right after a shape change
      // read up to 30 % slow).
      std::vector<int> ok;
      for (int r = 0; r < found; ++r) {
        size_t need = 0;
        if (hipblaslt_ext::matmulIsAlgoSupported(lt, desc, &alpha, la, lb, &beta, lc, lc, heur[r].algo, need) != HIPBLAS_STATUS_SUCCESS ||
            need > kWorkspace) {
          printf("  %s m=%lld rank %d: not supported here (workspace %zu)\n", sh.name, (long long)m, r, need);
          continue;
        }
        ok.push_back(r);
      }
      auto run = [&](int r) {
        CHECK_BLAS(hipblasLtMatmul(lt, desc, &alpha, w, la, x, lb, &beta, y, lc, y, lc, &heur[r].algo, ws, kWorkspace, s));
      };
      for (int r : ok)
        for (int i = 0; i < 5; ++i) run(r);
      const int rounds = 7, iters = 20;
      std::vector<std::vector<double>> t(found);
      for (int round = 0; round < rounds; ++round)
        for (int r : ok) {
          CHECK_HIP(hipEventRecord(e0, s));
          for (int i = 0; i < iters; ++i) run(r);
          CHECK_HIP(hipEventRecord(e1, s));
          CHECK_HIP(hipEventSynchronize(e1));
          float ms_total = 0.0f;
          CHECK_HIP(hipEventElapsedTime(&ms_total, e0, e1));
          t[r].push_back(1000.0 * ms_total / iters);
        }
      double first_us = -1.0, best_us = 1e30;
      int best_index = -1, best_rank = -1;
      uint64_t best_hash = 0;
      for (int r : ok) {
        std::sort(t[r].begin(), t[r].end());
        const double us = t[r][rounds / 2];
        const int index = hipblaslt_ext::getIndexFromAlgo(heur[r].algo);
        printf("  %s m=%lld rank %d index %d: median %.2f us (min %.2f, max %.2f) %s\n", sh.name, (long long)m, r, index, us,
               t[r].front(), t[r].back(), hipblaslt_ext::getKernelNameFromAlgo(lt, heur[r].algo).c_str());
        if (r == 0) first_us = us;
        if (us < best_us) {
          best_us = us;
          best_index = index;
          best_rank = r;
          best_hash = fnv1a(hipblaslt_ext::getKernelNameFromAlgo(lt, heur[r].algo));
        }
      }
      fflush(stdout);
      printf("pick %s version=%d dtype=bf16 m=%lld n=%lld k=%lld index=%d name_hash=0x%016llx rank=%d us=%.2f first_us=%.2f\n", sh.name,
             version, (long long)m, (long long)n, (long long)k, best_index, (unsigned long long)best_hash, best_rank, best_us, first_us);
      fflush(stdout);
      // The pick as the library gets it back: from its index, checked
      // against this problem.
      if (best_index >= 0) {
        std::vector<int> idx{best_index};
        std::vector<hipblasLtMatmulHeuristicResult_t> res;
        const hipblasStatus_t st = hipblaslt_ext::getAlgosFromIndex(lt, idx, res);
        size_t need = 0;
        const hipblasStatus_t sup = (st == HIPBLAS_STATUS_SUCCESS && !res.empty())
                                        ? hipblaslt_ext::matmulIsAlgoSupported(lt, desc, &alpha, la, lb, &beta, lc, lc, res[0].algo, need)
                                        : HIPBLAS_STATUS_INVALID_VALUE;
        printf("  %s m=%lld index %d from index: status %d, %zu results, supported %d, workspace %zu\n", sh.name, (long long)m,
               best_index, (int)st, res.size(), (int)sup, need);
        fflush(stdout);
      }
      hipblasLtMatrixLayoutDestroy(la);
      hipblasLtMatrixLayoutDestroy(lb);
      hipblasLtMatrixLayoutDestroy(lc);
      hipblasLtMatmulDescDestroy(desc);
    }
  }
  hipblasLtDestroy(lt);
  CHECK_HIP(hipFree(x));
  CHECK_HIP(hipFree(w));
  CHECK_HIP(hipFree(y));
  CHECK_HIP(hipFree(ws));
  return 0;
}

#ifndef CEV_GEMM_PROBE_LIB
int main(int argc, char** argv) { return cev_gemm_probe(argc - 1, argv + 1); }
#endif
