/* The CPU baseline's attention: the same candle op sequence as orc_attend
 * (qwen3.rs:206-220 / qwen35.rs:563-579, see cev_oracle.c), computed the way
 * a CPU BLAS path computes it: the score product and the P.V product as
 * register-blocked AVX2/FMA micro-kernels over cache blocks of keys, OpenMP
 * over (query head, block of rows).  Test infrastructure: bench.py times it
 * as the CPU baseline and tests/test_oracle_pinning.py checks it against
 * orc_attend.  Its f32 sums run in another order than orc_attend's (FMA,
 * blocked), so the two agree to f32 rounding, and to one bf16 ulp where a
 * value lands on a rounding boundary. */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf16_rne(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return x;
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}
static inline float rnd_b(float x, int bf16) { return bf16 ? bf16_rne(x) : x; }

static inline float hsum(__m256 v) {
  __m128 a = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  a = _mm_add_ps(a, _mm_movehl_ps(a, a));
  a = _mm_add_ss(a, _mm_movehdup_ps(a));
  return _mm_cvtss_f32(a);
}

enum { RB = 16, KB = 64, VB = 256 };

/* q (b, hq, t, d), k/v (b, hkv, s, d), mask (b, t, s) as in orc_attend; rows
 * [row0, row0 + nrows) of every (batch row, head).  d must be a multiple of
 * 32. */
void orc_attend_blocked(const float* q, const float* k, const float* v, const float* m, int b, int hq, int hkv, int t, int s, int d,
                        int64_t q_bs, int64_t kv_bs, int64_t m_bs, int bf16, int row0, int nrows, float* out) {
  const int g = hq / hkv;
  const float scale = (float)(1.0 / sqrt((double)d));
  const int nblk = (nrows + RB - 1) / RB;
  const int64_t njobs = (int64_t)b * hq * nblk;
#pragma omp parallel
  {
    float* sc = (float*)aligned_alloc(64, sizeof(float) * RB * (size_t)((s + 3) / 4 * 4));
    float* acc_o = (float*)aligned_alloc(64, sizeof(float) * RB * (size_t)d);
    float* qpad = (float*)aligned_alloc(64, sizeof(float) * RB * (size_t)d);
#pragma omp for schedule(dynamic, 1)
    for (int64_t job = 0; job < njobs; ++job) {
      const int blk = (int)(job % nblk);
      const int h = (int)((job / nblk) % hq);
      const int bi = (int)(job / ((int64_t)nblk * hq));
      const int kvh = h / g;
      const float* kb = k + bi * kv_bs + (int64_t)kvh * s * d;
      const float* vb = v + bi * kv_bs + (int64_t)kvh * s * d;
      const float* qb = q + bi * q_bs + (int64_t)h * t * d;
      const float* mb = m + bi * m_bs;
      const int r0 = row0 + blk * RB;
      const int nr = r0 + RB <= row0 + nrows ? RB : row0 + nrows - r0;
      const int nr2 = (nr + 1) & ~1;
      const int ss = (s + 3) / 4 * 4;
      for (int r = 0; r < nr2; ++r) memcpy(qpad + (int64_t)r * d, qb + (int64_t)(r0 + (r < nr ? r : 0)) * d, sizeof(float) * d);
      /* scores: 2 rows x 4 keys per micro-kernel, f32 sums over d, keys in
       * cache blocks of KB shared by every row pair */
      for (int j0 = 0; j0 < s; j0 += KB) {
        const int j1 = j0 + KB < s ? j0 + KB : s;
        for (int r = 0; r < nr2; r += 2) {
          const float* q0 = qpad + (int64_t)r * d;
          const float* q1 = q0 + d;
          for (int j = j0; j < j1; j += 4) {
            const float* kr[4];
            for (int c = 0; c < 4; ++c) kr[c] = kb + (int64_t)(j + c < s ? j + c : s - 1) * d;
            __m256 a0[4], a1[4];
            for (int c = 0; c < 4; ++c) a0[c] = a1[c] = _mm256_setzero_ps();
            for (int i = 0; i < d; i += 8) {
              const __m256 x0 = _mm256_load_ps(q0 + i), x1 = _mm256_load_ps(q1 + i);
              for (int c = 0; c < 4; ++c) {
                const __m256 kv = _mm256_loadu_ps(kr[c] + i);
                a0[c] = _mm256_fmadd_ps(x0, kv, a0[c]);
                a1[c] = _mm256_fmadd_ps(x1, kv, a1[c]);
              }
            }
            for (int c = 0; c < 4; ++c) {
              sc[(int64_t)r * ss + j + c] = hsum(a0[c]);
              sc[(int64_t)(r + 1) * ss + j + c] = hsum(a1[c]);
            }
          }
        }
      }
      for (int r = 0; r < nr; ++r) {
        float* row = sc + (int64_t)r * ss;
        const float* mrow = mb + (int64_t)(r0 + r) * s;
        float mx = -INFINITY;
        for (int j = 0; j < s; ++j) {
          float x = rnd_b(row[j], bf16);
          x = x * scale + 0.0f;
          x = x + mrow[j];
          row[j] = x;
          mx = x > mx ? x : mx;
        }
        float sum = 0.0f;
        for (int j = 0; j < s; ++j) {
          row[j] = expf(row[j] - mx);
          sum += row[j];
        }
        for (int j = 0; j < s; ++j) row[j] = rnd_b(row[j] / sum, bf16);
      }
      for (int r = nr; r < nr2; ++r) memset(sc + (int64_t)r * ss, 0, sizeof(float) * s);
      /* P.V: 2 rows x 32 head-dim values per micro-kernel, keys in cache
       * blocks of VB; the running sums live in acc_o between blocks */
      memset(acc_o, 0, sizeof(float) * RB * d);
      for (int j0 = 0; j0 < s; j0 += VB) {
        const int j1 = j0 + VB < s ? j0 + VB : s;
        for (int r = 0; r < nr2; r += 2) {
          const float* p0 = sc + (int64_t)r * ss;
          const float* p1 = p0 + ss;
          for (int c = 0; c < d; c += 32) {
            float* o0 = acc_o + (int64_t)r * d + c;
            float* o1 = o0 + d;
            __m256 a0[4], a1[4];
            for (int e = 0; e < 4; ++e) {
              a0[e] = _mm256_load_ps(o0 + 8 * e);
              a1[e] = _mm256_load_ps(o1 + 8 * e);
            }
            for (int j = j0; j < j1; ++j) {
              const float* vj = vb + (int64_t)j * d + c;
              const __m256 w0 = _mm256_set1_ps(p0[j]), w1 = _mm256_set1_ps(p1[j]);
              for (int e = 0; e < 4; ++e) {
                const __m256 vv = _mm256_loadu_ps(vj + 8 * e);
                a0[e] = _mm256_fmadd_ps(w0, vv, a0[e]);
                a1[e] = _mm256_fmadd_ps(w1, vv, a1[e]);
              }
            }
            for (int e = 0; e < 4; ++e) {
              _mm256_store_ps(o0 + 8 * e, a0[e]);
              _mm256_store_ps(o1 + 8 * e, a1[e]);
            }
          }
        }
      }
      for (int r = 0; r < nr; ++r) {
        float* o = out + bi * q_bs + ((int64_t)h * t + r0 + r) * d;
        for (int i = 0; i < d; ++i) o[i] = rnd_b(acc_o[(int64_t)r * d + i], bf16);
      }
    }
    free(sc);
    free(acc_o);
    free(qpad);
  }
}
