/*
 * CPU oracle for cev's packed-prefill attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only to check
 * results against or as the timed CPU baseline -- never as the product path.
 *
 * What it restates (all paths relative to the reference checkout):
 *   - the RoPE cos/sin table        crates/cev-model/src/qwen3.rs:107-118,
 *                                   crates/cev-model/src/qwen35.rs:188-228
 *   - RoPE (rotate-half)            qwen3.rs:121-123, qwen35.rs:230-240
 *   - QK RMSNorm (w and 1 + w)      qwen3.rs:193-194, qwen35.rs:160-176
 *   - the dense additive masks      qwen3.rs:153-169 (segment_mask),
 *                                   crates/cev-model/src/engine.rs:389-442 (packed pass),
 *                                   qwen35.rs:469-479 (branch), qwen35.rs:481-498 (bidirectional)
 *   - attend (candle op sequence)   qwen3.rs:206-220, qwen35.rs:563-579
 *   - the Gated DeltaNet chunk rule qwen35.rs:243-368, 414-453 and its
 *     token recurrence check        qwen35.rs:776-822
 *
 * candle-core / candle-nn 0.11.0 (Cargo.lock:428-431, 486-489) execute the
 * arithmetic in the reference and are not part of the checkout.  Their CPU
 * op semantics are restated from the published algorithms: f32 products and
 * sums, bf16 = round-to-nearest-even of the f32 result at every op boundary
 * (half 2.7.1), softmax as max / exp / sum / divide.  The summation order
 * inside candle's GEMM (the gemm crate) and reductions is not reproduced
 * bit-for-bit; it sits inside the f32 1e-5 and bf16 2e-2 budgets.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so a*b - c*d is never
 * fused, matching Rust, which never contracts to FMA).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Planted mistakes.  The oracle's own pinning tests switch one of these on
 * and check that some pinning check then fails.  0 = exact restatement. */
enum {
  MUT_NONE = 0,
  MUT_ROPE_SIN_SIGN = 1,   /* rope: x1*c + x2*s instead of x1*c - x2*s   */
  MUT_ATTN_KV_MODULO = 2,  /* repeat_kv: kv head h % Hkv instead of h / G */
  MUT_ATTN_NO_SCALE = 3,   /* attend: scores not multiplied by 1/sqrt(D) */
  MUT_ATTN_V_SHIFT = 4,    /* attend: p_j multiplies v[j+1]              */
  MUT_MASK_NO_DIAG = 5,    /* engine mask: a question token misses itself */
  MUT_NORM_DIM_M1 = 6,     /* rms_norm: mean over D-1 instead of D       */
  MUT_TABLE_POS = 7,       /* rope table: angle from (p+1)               */
  MUT_GDN_NO_DECAY = 8,    /* gdn chunk rule: drops the chunk decay      */
};
static int g_mut = MUT_NONE;
void orc_set_mutation(int m) { g_mut = m; }
int orc_get_mutation(void) { return g_mut; }

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------ */
/* bf16: round-to-nearest-even of an f32, NaN kept quiet (half::bf16::from_f32). */
static inline float bf16r(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    u |= 0x00400000u;
    u &= 0xffff0000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  float y;
  memcpy(&y, &u, 4);
  return y;
}
static inline float rnd(float x, int bf16) { return bf16 ? bf16r(x) : x; }

float bf16r_ext(float x) { return bf16r(x); }

void orc_round_bf16(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = bf16r(x[i]);
}

/* ------------------------------------------------------------------ */
/* RoPE cos/sin table, qwen3.rs:107-118.
 *   inv_i   = 1f32 / (theta.powf(2i / dim) as f32)           (qwen3.rs:109-112)
 *   angle   = (p as f32) * inv_i, one f32 product             (qwen3.rs:115-116, K=1 matmul)
 *   cos/sin = f32 cos/sin of the angle, then to model dtype   (qwen3.rs:117)
 * qwen35.rs:188-228 builds the same values for text positions: the three
 * mrope axes carry the same position and the one-hot sum adds exact zeros.
 * cos/sin: (n_pos, rot/2) row-major. */
void orc_rope_table(double theta, int rot, int n_pos, int bf16, float* cos_out, float* sin_out) {
  int half = rot / 2;
  float* inv = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
  for (int i = 0; i < half; ++i) inv[i] = 1.0f / (float)pow(theta, (double)(2 * i) / (double)rot);
  for (int p = 0; p < n_pos; ++p) {
    float fp = (float)(g_mut == MUT_TABLE_POS ? p + 1 : p);
    for (int i = 0; i < half; ++i) {
      float a = fp * inv[i];
      cos_out[(int64_t)p * half + i] = rnd(cosf(a), bf16);
      sin_out[(int64_t)p * half + i] = rnd(sinf(a), bf16);
    }
  }
  free(inv);
}

/* ------------------------------------------------------------------ */
/* RMSNorm over the last dim (candle_nn::ops::rms_norm as called by
 * qwen3.rs:193-194 through RmsNorm::forward on a contiguous tensor, and by
 * qwen35.rs:173-175 with scale = (1 + w) rounded to the weight dtype,
 * qwen35.rs:169):
 *   sum2 = sum_i x_i^2 (f32);  m = sqrt(sum2 / D + eps) -> model dtype;
 *   y_i  = (x_i / m) * scale_i, each op in the model dtype.
 * x, y: (rows, d); w: (d) already holding model-dtype values. */
void orc_rms_norm(const float* x, int64_t rows, int d, const float* w, int plus_one, float eps, int bf16, float* y) {
  float* scale = (float*)malloc(sizeof(float) * (size_t)d);
  for (int i = 0; i < d; ++i) scale[i] = plus_one ? rnd(w[i] + 1.0f, bf16) : w[i];
  float denom = (float)(g_mut == MUT_NORM_DIM_M1 ? d - 1 : d);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * d;
    float sum2 = 0.0f;
    for (int i = 0; i < d; ++i) sum2 += xr[i] * xr[i];
    float m = rnd(sqrtf(sum2 / denom + eps), bf16);
    float* yr = y + r * d;
    for (int i = 0; i < d; ++i) yr[i] = rnd(rnd(xr[i] / m, bf16) * scale[i], bf16);
  }
  free(scale);
}

/* ------------------------------------------------------------------ */
/* RoPE, rotate-half on the first `rot` dims (candle_nn::rotary_emb::rope,
 * qwen3.rs:121-123; partial form qwen35.rs:230-240):
 *   y_i        = x_i * c - x_{i+h} * s
 *   y_{i+h}    = x_i * s + x_{i+h} * c        (h = rot/2, each op in model dtype)
 * x: (t, heads, d) token-major, in place.  pos: (t).  cos/sin: (n_pos, h). */
void orc_rope(float* x, int t, int heads, int d, int rot, const int32_t* pos, const float* cos_t, const float* sin_t, int bf16) {
  int half = rot / 2;
#pragma omp parallel for schedule(static)
  for (int64_t th = 0; th < (int64_t)t * heads; ++th) {
    int tok = (int)(th / heads);
    float* xr = x + th * d;
    const float* c = cos_t + (int64_t)pos[tok] * half;
    const float* s = sin_t + (int64_t)pos[tok] * half;
    for (int i = 0; i < half; ++i) {
      float a = xr[i], b = xr[i + half];
      float y1, y2;
      if (g_mut == MUT_ROPE_SIN_SIGN) {
        y1 = rnd(rnd(a * c[i], bf16) + rnd(b * s[i], bf16), bf16);
      } else {
        y1 = rnd(rnd(a * c[i], bf16) - rnd(b * s[i], bf16), bf16);
      }
      y2 = rnd(rnd(a * s[i], bf16) + rnd(b * c[i], bf16), bf16);
      xr[i] = y1;
      xr[i + half] = y2;
    }
  }
}

/* ------------------------------------------------------------------ */
/* Dense additive masks (0 visible, -inf hidden), f32. */

/* qwen3.rs:157-169: n new tokens after `past` cached ones; a new token sees
 * every cached token and earlier new tokens of its own segment. (n, past+n) */
void orc_segment_mask(const uint32_t* seg, int n, int past, float* m) {
  int w = past + n;
  for (int i = 0; i < n; ++i) {
    float* row = m + (int64_t)i * w;
    for (int j = 0; j < w; ++j) row[j] = 0.0f;
    for (int j = 0; j < n; ++j)
      if (j > i || seg[j] != seg[i]) row[past + j] = -INFINITY;
  }
}

/* engine.rs:365-442, the packed pass.  Plans p (in plan order) carry
 *   past_len[p]   tokens of already computed K/V the plan may read,
 *   prefix_len[p] tokens of its whole prefix,
 *   tail_start[p] first prefix token not yet computed (== prefix_len: no tail).
 * The batch lists (plan, question length) items.  Tails ride first, in plan
 * order, then the questions (engine.rs:393-416).  Outputs:
 *   pos (n)      RoPE positions: tail.start + j, or prefix_len + j (restart, :411)
 *   gather (nb)  last token of each question (:415)
 *   mask (n, past_total + n)                   (:418-442)
 * Returns n, the number of new tokens. */
int orc_engine_pass(int n_plans, const int32_t* past_len, const int32_t* prefix_len, const int32_t* tail_start, int nb, const int32_t* item_plan,
                    const int32_t* item_len, int32_t* pos, int32_t* gather, int32_t* owner, int32_t* seg, float* mask) {
  int past_total = 0;
  int* past_off = (int*)malloc(sizeof(int) * (size_t)(n_plans > 0 ? n_plans : 1));
  for (int p = 0; p < n_plans; ++p) {
    past_off[p] = past_total;
    past_total += past_len[p];
  }
  int n = 0;
  int* tail_at_start = (int*)malloc(sizeof(int) * (size_t)(n_plans > 0 ? n_plans : 1));
  int* tail_at_len = (int*)malloc(sizeof(int) * (size_t)(n_plans > 0 ? n_plans : 1));
  for (int p = 0; p < n_plans; ++p) {
    tail_at_start[p] = -1;
    tail_at_len[p] = 0;
    int tl = prefix_len[p] - tail_start[p];
    if (tl <= 0) continue;
    tail_at_start[p] = n;
    tail_at_len[p] = tl;
    for (int j = 0; j < tl; ++j) {
      pos[n] = tail_start[p] + j;
      owner[n] = p;
      seg[n] = 0;
      ++n;
    }
  }
  for (int k = 0; k < nb; ++k) {
    int p = item_plan[k];
    for (int j = 0; j < item_len[k]; ++j) {
      pos[n] = prefix_len[p] + j;
      owner[n] = p;
      seg[n] = k + 1;
      ++n;
    }
    gather[k] = n - 1;
  }
  if (mask) {
    int64_t w = (int64_t)past_total + n;
    for (int i = 0; i < n; ++i) {
      float* row = mask + (int64_t)i * w;
      for (int64_t j = 0; j < w; ++j) row[j] = -INFINITY;
      int p = owner[i];
      for (int j = 0; j < past_len[p]; ++j) row[past_off[p] + j] = 0.0f;
      if (tail_at_start[p] >= 0) {
        int start = tail_at_start[p], len = tail_at_len[p];
        int end = seg[i] == 0 ? i + 1 : start + len;
        for (int j = start; j < end; ++j) row[past_total + j] = 0.0f;
      }
      if (seg[i] != 0) {
        int j = i;
        for (;;) {
          if (!(g_mut == MUT_MASK_NO_DIAG && j == i)) row[past_total + j] = 0.0f;
          if (j == 0 || seg[j - 1] != seg[i]) break;
          --j;
        }
      }
    }
  }
  free(past_off);
  free(tail_at_start);
  free(tail_at_len);
  return n;
}

/* qwen35.rs:471-479: (t, past + t), branch tokens see every past token and
 * earlier tokens of their own row. */
void orc_branch_mask(int t, int past, float* m) {
  int w = past + t;
  for (int i = 0; i < t; ++i)
    for (int j = 0; j < w; ++j) m[(int64_t)i * w + j] = (j >= past && j - past > i) ? -INFINITY : 0.0f;
}

/* qwen35.rs:483-498: (b, t, t) bidirectional rows, padding columns hidden,
 * a fully padded query row keeps its diagonal. */
void orc_bidirectional_mask(int t, const int32_t* lengths, int b, float* m) {
  for (int r = 0; r < b; ++r) {
    int len = lengths[r];
    for (int i = 0; i < t; ++i) {
      float* row = m + ((int64_t)r * t + i) * t;
      for (int j = 0; j < t; ++j) row[j] = j >= len ? -INFINITY : 0.0f;
      if (i >= len) row[i] = 0.0f;
    }
  }
}

/* ------------------------------------------------------------------ */
/* attend, the candle op sequence of qwen3.rs:206-220 / qwen35.rs:563-579:
 *   k, v = repeat_kv(k, v, G)                  head h reads kv head h / G (qwen3.rs:145-151)
 *   s    = q . k^T  (model dtype out)  -> f32   (f32 accumulate; bf16: rounded once)
 *   s    = s * (f32)(1/sqrt(D)) + mask          (affine then broadcast_add, :217)
 *   p    = softmax_last_dim(s) -> model dtype   (max, exp, sum, divide in f32; :218)
 *   out  = p . v  (model dtype out)             (:219)
 * Shapes (b = batch rows, strides in elements so a stride of 0 broadcasts,
 * which is what LayerState::broadcast materialises, decoder.rs:74-88):
 *   q   (b, hq, t, d)     at q  + bi*q_bs
 *   k,v (b, hkv, s, d)    at k  + bi*kv_bs
 *   m   (b, t, s)         at m  + bi*m_bs     (0 / -inf)
 *   out (b, hq, t, d)
 * Rows are independent, so `row0, nrows` restrict the work to query rows
 * [row0, row0 + nrows) of every (bi, h); out still uses full-t indexing. */
static inline float dot_f32(const float* a, const float* b, int d) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i + 8 <= d; i += 8)
    for (int u = 0; u < 8; ++u) acc[u] += a[i + u] * b[i + u];
  float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  for (; i < d; ++i) s += a[i] * b[i];
  return s;
}

void orc_attend(const float* q, const float* k, const float* v, const float* m, int b, int hq, int hkv, int t, int s, int d, int64_t q_bs,
                int64_t kv_bs, int64_t m_bs, int bf16, int row0, int nrows, float* out) {
  const int g = hq / hkv;
  const float scale = g_mut == MUT_ATTN_NO_SCALE ? 1.0f : (float)(1.0 / sqrt((double)d));
  const int chunk = 8;
  const int nchunks = (nrows + chunk - 1) / chunk;
  const int64_t njobs = (int64_t)b * hq * nchunks;
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)chunk * (size_t)s);
    float* acc = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(dynamic, 1)
    for (int64_t job = 0; job < njobs; ++job) {
      int ci = (int)(job % nchunks);
      int h = (int)((job / nchunks) % hq);
      int bi = (int)(job / ((int64_t)nchunks * hq));
      int kvh = g_mut == MUT_ATTN_KV_MODULO ? h % hkv : h / g;
      const float* kb = k + bi * kv_bs + (int64_t)kvh * s * d;
      const float* vb = v + bi * kv_bs + (int64_t)kvh * s * d;
      const float* qb = q + bi * q_bs + (int64_t)h * t * d;
      const float* mb = m + bi * m_bs;
      int r0 = row0 + ci * chunk;
      int r1 = r0 + chunk;
      if (r1 > row0 + nrows) r1 = row0 + nrows;
      int nr = r1 - r0;
      /* scores for nr rows, dense over all s keys (the reference computes the
       * whole T x S product before masking) */
      for (int j = 0; j < s; ++j) {
        const float* kj = kb + (int64_t)j * d;
        for (int r = 0; r < nr; ++r) {
          float x = dot_f32(qb + (int64_t)(r0 + r) * d, kj, d);
          x = rnd(x, bf16);
          x = x * scale + 0.0f;
          x = x + mb[(int64_t)(r0 + r) * s + j];
          sc[(int64_t)r * s + j] = x;
        }
      }
      for (int r = 0; r < nr; ++r) {
        float* row = sc + (int64_t)r * s;
        float mx = -INFINITY;
        for (int j = 0; j < s; ++j) mx = row[j] > mx ? row[j] : mx;
        float sum = 0.0f;
        for (int j = 0; j < s; ++j) {
          row[j] = expf(row[j] - mx);
          sum += row[j];
        }
        for (int j = 0; j < s; ++j) row[j] = rnd(row[j] / sum, bf16);
        for (int i = 0; i < d; ++i) acc[i] = 0.0f;
        for (int j = 0; j < s; ++j) {
          float p = row[j];
          if (p == 0.0f) continue; /* exact: 0 * finite adds nothing */
          int jj = j;
          if (g_mut == MUT_ATTN_V_SHIFT) jj = (j + 1) % s;
          const float* vj = vb + (int64_t)jj * d;
          for (int i = 0; i < d; ++i) acc[i] += p * vj[i];
        }
        float* o = out + bi * q_bs + ((int64_t)h * t + r0 + r) * d;
        for (int i = 0; i < d; ++i) o[i] = rnd(acc[i], bf16);
      }
    }
    free(sc);
    free(acc);
  }
}

/* Textbook attention in f64: softmax over the keys the mask leaves visible
 * (m == 0), scores q.k / sqrt(D), for the same layouts as orc_attend.
 * Independent of the candle op order; the two must agree to f32 rounding. */
void orc_attend_f64(const float* q, const float* k, const float* v, const float* m, int b, int hq, int hkv, int t, int s, int d, int64_t q_bs,
                    int64_t kv_bs, int64_t m_bs, int row0, int nrows, double* out) {
  const int g = hq / hkv;
  const double scale = 1.0 / sqrt((double)d);
  const int64_t njobs = (int64_t)b * hq * nrows;
#pragma omp parallel
  {
    double* w = (double*)malloc(sizeof(double) * (size_t)s);
    double* acc = (double*)malloc(sizeof(double) * (size_t)d);
#pragma omp for schedule(dynamic, 16)
    for (int64_t job = 0; job < njobs; ++job) {
      int r = row0 + (int)(job % nrows);
      int h = (int)((job / nrows) % hq);
      int bi = (int)(job / ((int64_t)nrows * hq));
      int kvh = h / g;
      const float* kb = k + bi * kv_bs + (int64_t)kvh * s * d;
      const float* vb = v + bi * kv_bs + (int64_t)kvh * s * d;
      const float* qr = q + bi * q_bs + ((int64_t)h * t + r) * d;
      const float* mr = m + bi * m_bs + (int64_t)r * s;
      double mx = -INFINITY;
      for (int j = 0; j < s; ++j) {
        if (mr[j] != 0.0f) {
          w[j] = -INFINITY;
          continue;
        }
        double x = 0.0;
        const float* kj = kb + (int64_t)j * d;
        for (int i = 0; i < d; ++i) x += (double)qr[i] * (double)kj[i];
        x *= scale;
        w[j] = x;
        if (x > mx) mx = x;
      }
      double sum = 0.0;
      for (int j = 0; j < s; ++j) {
        w[j] = w[j] == -INFINITY ? 0.0 : exp(w[j] - mx);
        sum += w[j];
      }
      for (int i = 0; i < d; ++i) acc[i] = 0.0;
      for (int j = 0; j < s; ++j) {
        if (w[j] == 0.0) continue;
        const float* vj = vb + (int64_t)j * d;
        double p = w[j] / sum;
        for (int i = 0; i < d; ++i) acc[i] += p * (double)vj[i];
      }
      double* o = out + bi * q_bs + ((int64_t)h * t + r) * d;
      for (int i = 0; i < d; ++i) o[i] = acc[i];
    }
    free(w);
    free(acc);
  }
}

/* Sigmoid output gate, qwen35.rs:556-558: out (t, h*d) in the model dtype is
 * multiplied by candle_nn::ops::sigmoid(gate), computed as 1 / (1 + exp(-g))
 * in the model dtype, op by op. */
void orc_sigmoid_gate(float* out, const float* gate, int64_t n, int bf16) {
  for (int64_t i = 0; i < n; ++i) {
    float e = rnd(expf(-gate[i]), bf16);
    float den = rnd(e + 1.0f, bf16);
    float sg = rnd(1.0f / den, bf16);
    out[i] = rnd(out[i] * sg, bf16);
  }
}
