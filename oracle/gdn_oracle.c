/*
 * CPU oracle for the Gated DeltaNet layer of Qwen3.5 hybrid prefixes.
 *
 * TEST INFRASTRUCTURE ONLY (same rules as cev_oracle.c: loaded by tests/,
 * smoke() and bench.py's cpu_baseline leg, never by the product path).
 *
 * Restates, in f32 like the reference:
 *   l2norm                     crates/cev-model/src/qwen35.rs:250-254
 *   softplus                   qwen35.rs:243-248
 *   inv_unit_lower             qwen35.rs:256-296 (recursive block inversion)
 *   chunk_gated_delta_rule     qwen35.rs:298-368
 *   depthwise conv + conv tail qwen35.rs:428-430, decoder.rs:137-151
 *   gated RMSNorm . SiLU(z)    qwen35.rs:447-451
 *   the token recurrence used by the reference's own check, qwen35.rs:776-822
 *
 * Parity unpinned (no offline reference test covers them): the bf16
 * rounding points of the conv (each product and partial sum, then candle's
 * bf16 SiLU as v / (1 + exp(-v)) with each op rounded) and of the gated
 * norm's final cast; they follow candle's per-op bf16 arithmetic.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int orc_get_mutation(void);
float bf16r_ext(float x);
#define MUT_GDN_NO_DECAY 8

/* x / sqrt(sum x^2 + 1e-6) over the last dim (qwen35.rs:251-254). */
void orc_l2norm(const float* x, int64_t rows, int d, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    float s = 0.0f;
    for (int i = 0; i < d; ++i) s += x[r * d + i] * x[r * d + i];
    float n = sqrtf(s + 1e-6f);
    for (int i = 0; i < d; ++i) y[r * d + i] = x[r * d + i] / n;
  }
}

/* max(x, 0) + ln(1 + e^{-|x|}) (qwen35.rs:243-248). */
float orc_softplus(float x) {
  float pos = x > 0.0f ? x : 0.0f;
  float neg = expf(-fabsf(x));
  return pos + logf(neg + 1.0f);
}

/* c (m, n) = a (m, k) . b (k, n), f32, k ascending. */
static void mm(const float* a, const float* b, float* c, int m, int k, int n) {
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j) {
      float s = 0.0f;
      for (int t = 0; t < k; ++t) s += a[i * k + t] * b[t * n + j];
      c[i * n + j] = s;
    }
}

/* (I + m)^-1 for m (n, n) strictly lower, by the recursive split of
 * qwen35.rs:277-296:  [A 0; C B]^-1 = [A^-1 0; -(B^-1 C) A^-1  B^-1]. */
static void inv_strict(const float* m, int n, int ld, float* out, int ldo) {
  if (n == 1) {
    out[0] = 1.0f;
    return;
  }
  int h = n / 2, r = n - h;
  float* ai = (float*)calloc((size_t)h * h, sizeof(float));
  float* di = (float*)calloc((size_t)r * r, sizeof(float));
  float* a = (float*)malloc(sizeof(float) * (size_t)h * h);
  float* c = (float*)malloc(sizeof(float) * (size_t)r * h);
  float* d = (float*)malloc(sizeof(float) * (size_t)r * r);
  for (int i = 0; i < h; ++i)
    for (int j = 0; j < h; ++j) a[i * h + j] = m[i * ld + j];
  for (int i = 0; i < r; ++i)
    for (int j = 0; j < h; ++j) c[i * h + j] = m[(h + i) * ld + j];
  for (int i = 0; i < r; ++i)
    for (int j = 0; j < r; ++j) d[i * r + j] = m[(h + i) * ld + h + j];
  inv_strict(a, h, h, ai, h);
  inv_strict(d, r, r, di, r);
  float* dc = (float*)malloc(sizeof(float) * (size_t)r * h);
  float* ll = (float*)malloc(sizeof(float) * (size_t)r * h);
  mm(di, c, dc, r, r, h);
  mm(dc, ai, ll, r, h, h);
  for (int i = 0; i < n; ++i)
    for (int j = 0; j < n; ++j) out[i * ldo + j] = 0.0f;
  for (int i = 0; i < h; ++i)
    for (int j = 0; j < h; ++j) out[i * ldo + j] = ai[i * h + j];
  for (int i = 0; i < r; ++i)
    for (int j = 0; j < h; ++j) out[(h + i) * ldo + j] = -ll[i * h + j];
  for (int i = 0; i < r; ++i)
    for (int j = 0; j < r; ++j) out[(h + i) * ldo + h + j] = di[i * r + j];
  free(ai);
  free(di);
  free(a);
  free(c);
  free(d);
  free(dc);
  free(ll);
}

/* inv_unit_lower (qwen35.rs:266-274): keeps the strict lower triangle of
 * each (n, n) matrix of `m` and returns (I + L)^-1.  m, out: (batch, n, n). */
void orc_inv_unit_lower(const float* m, int batch, int n, float* out) {
  float* strict = (float*)malloc(sizeof(float) * (size_t)n * n);
  for (int b = 0; b < batch; ++b) {
    const float* mb = m + (int64_t)b * n * n;
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < n; ++j) strict[i * n + j] = j < i ? mb[i * n + j] : 0.0f;
    inv_strict(strict, n, n, out + (int64_t)b * n * n, n);
  }
  free(strict);
}

/* chunk_gated_delta_rule (qwen35.rs:301-368), all f32, one (batch x head)
 * sequence per call slice:
 *   q, k (h, t, dk); v (h, t, dv); g, beta (h, t); s0 (h, dk, dv) or NULL.
 *   out (h, t, dv); s_out (h, dk, dv).
 * q and k are l2-normalised here, q also scaled by dk^-0.5 (:306-307). */
void orc_chunk_gated_delta_rule(const float* q_in, const float* k_in, const float* v, const float* g, const float* beta, const float* s0, int h,
                                int t, int dk, int dv, int chunk, float* out, float* s_out) {
  const int C = chunk;
  const int pad = (C - t % C) % C;
  const int tp = t + pad;
  const int n = tp / C;
  const float qscale = (float)pow((double)dk, -0.5);
  int mut_no_decay = orc_get_mutation() == MUT_GDN_NO_DECAY;
  /* Heads are independent: one thread per head, each with its own scratch. */
#pragma omp parallel
  {
    float* q = (float*)calloc((size_t)tp * dk, sizeof(float));
    float* k = (float*)calloc((size_t)tp * dk, sizeof(float));
    float* vb = (float*)calloc((size_t)tp * dv, sizeof(float));
    float* kb = (float*)calloc((size_t)tp * dk, sizeof(float));
    float* gp = (float*)calloc((size_t)tp, sizeof(float));
    float* cum = (float*)malloc(sizeof(float) * (size_t)tp);
    float* pair = (float*)malloc(sizeof(float) * (size_t)C * C);
    float* ut = (float*)malloc(sizeof(float) * (size_t)C * C);
    float* intra = (float*)malloc(sizeof(float) * (size_t)n * C * C);
    float* inv = (float*)malloc(sizeof(float) * (size_t)C * C);
    float* nv = (float*)malloc(sizeof(float) * (size_t)tp * dv);
    float* kcd = (float*)malloc(sizeof(float) * (size_t)tp * dk);
    float* dkb = (float*)malloc(sizeof(float) * (size_t)C * dk);
    float* S = (float*)malloc(sizeof(float) * (size_t)dk * dv);
    float* vnew = (float*)malloc(sizeof(float) * (size_t)C * dv);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)C * (dv > dk ? dv : dk));
    float* wdec = (float*)malloc(sizeof(float) * (size_t)C);
#pragma omp for schedule(dynamic, 1)
    for (int hh = 0; hh < h; ++hh) {
      const float* qh = q_in + (int64_t)hh * t * dk;
      const float* kh = k_in + (int64_t)hh * t * dk;
      const float* vh = v + (int64_t)hh * t * dv;
      const float* gh = g + (int64_t)hh * t;
      const float* bh = beta + (int64_t)hh * t;
      memset(q, 0, sizeof(float) * (size_t)tp * dk);
      memset(k, 0, sizeof(float) * (size_t)tp * dk);
      memset(vb, 0, sizeof(float) * (size_t)tp * dv);
      memset(kb, 0, sizeof(float) * (size_t)tp * dk);
      memset(gp, 0, sizeof(float) * (size_t)tp);
      orc_l2norm(qh, t, dk, q);
      for (int64_t i = 0; i < (int64_t)t * dk; ++i) q[i] = q[i] * qscale + 0.0f;
      orc_l2norm(kh, t, dk, k);
      for (int i = 0; i < t; ++i) {
        for (int e = 0; e < dv; ++e) vb[(int64_t)i * dv + e] = vh[(int64_t)i * dv + e] * bh[i];
        for (int e = 0; e < dk; ++e) kb[(int64_t)i * dk + e] = k[(int64_t)i * dk + e] * bh[i];
        gp[i] = gh[i];
      }
      for (int c = 0; c < n; ++c) {
        float acc = 0.0f;
        for (int i = 0; i < C; ++i) {
          acc += gp[c * C + i];
          cum[c * C + i] = acc;
        }
      }
      /* per chunk: pair, ut, intra, inverse, new values, k_cumdecay */
      for (int c = 0; c < n; ++c) {
        const float* cu = cum + c * C;
        for (int i = 0; i < C; ++i)
          for (int j = 0; j < C; ++j) pair[i * C + j] = j <= i ? expf(cu[i] - cu[j]) : 0.0f;
        const float* kc = k + (int64_t)c * C * dk;
        const float* kbc = kb + (int64_t)c * C * dk;
        const float* qc = q + (int64_t)c * C * dk;
        for (int i = 0; i < C; ++i)
          for (int j = 0; j < C; ++j) {
            float a = 0.0f, b = 0.0f;
            for (int e = 0; e < dk; ++e) {
              a += kbc[i * dk + e] * kc[j * dk + e];
              b += qc[i * dk + e] * kc[j * dk + e];
            }
            ut[i * C + j] = a * pair[i * C + j];
            intra[(int64_t)c * C * C + i * C + j] = b * pair[i * C + j];
          }
        orc_inv_unit_lower(ut, 1, C, inv);
        mm(inv, vb + (int64_t)c * C * dv, nv + (int64_t)c * C * dv, C, C, dv);
        for (int i = 0; i < C; ++i) {
          float e = expf(cu[i]);
          for (int x = 0; x < dk; ++x) dkb[i * dk + x] = kbc[i * dk + x] * e;
        }
        mm(inv, dkb, kcd + (int64_t)c * C * dk, C, C, dk);
      }
      /* state scan over chunks (:346-365) */
      float* Sh = S;
      if (s0)
        memcpy(Sh, s0 + (int64_t)hh * dk * dv, sizeof(float) * (size_t)dk * dv);
      else
        memset(Sh, 0, sizeof(float) * (size_t)dk * dv);
      for (int c = 0; c < n; ++c) {
        const float* cu = cum + c * C;
        float last = cu[C - 1];
        /* v_new = new_values - k_cumdecay . S */
        mm(kcd + (int64_t)c * C * dk, Sh, tmp, C, dk, dv);
        for (int i = 0; i < C * dv; ++i) vnew[i] = nv[(int64_t)c * C * dv + i] - tmp[i];
        /* inter = (q * e^cum) . S ; out = inter + intra . v_new */
        for (int i = 0; i < C; ++i) {
          float e = expf(cu[i]);
          for (int j = 0; j < dv; ++j) {
            float s = 0.0f;
            for (int x = 0; x < dk; ++x) s += (q[((int64_t)c * C + i) * dk + x] * e) * Sh[x * dv + j];
            float s2 = 0.0f;
            for (int x = 0; x < C; ++x) s2 += intra[(int64_t)c * C * C + i * C + x] * vnew[x * dv + j];
            int row = c * C + i;
            if (row < t) out[((int64_t)hh * t + row) * dv + j] = s + s2;
          }
        }
        /* S = S * e^last + (k * e^(last - cum))^T . v_new */
        float decay = mut_no_decay ? 1.0f : expf(last);
        for (int i = 0; i < C; ++i) wdec[i] = expf(last - cu[i]);
        for (int x = 0; x < dk; ++x)
          for (int j = 0; j < dv; ++j) {
            float s = 0.0f;
            for (int i = 0; i < C; ++i) s += (k[((int64_t)c * C + i) * dk + x] * wdec[i]) * vnew[i * dv + j];
            Sh[x * dv + j] = Sh[x * dv + j] * decay + s;
          }
      }
      memcpy(s_out + (int64_t)hh * dk * dv, Sh, sizeof(float) * (size_t)dk * dv);
    }
    free(q);
    free(k);
    free(vb);
    free(kb);
    free(gp);
    free(cum);
    free(pair);
    free(ut);
    free(intra);
    free(inv);
    free(nv);
    free(kcd);
    free(dkb);
    free(S);
    free(vnew);
    free(tmp);
    free(wdec);
  }
}

/* The token-by-token gated delta recurrence that the reference checks its
 * chunked rule against (qwen35.rs:796-821), on already-normalised q, k:
 *   S <- S * e^{g_t};  delta = (v_t - S^T k_t) * beta_t;  S <- S + k_t delta^T;
 *   o_t = S^T q_t.
 * q, k (h, t, dk) normalised (q also scaled); v (h, t, dv); s0 or NULL. */
void orc_gdn_recurrence(const float* qn, const float* kn, const float* v, const float* g, const float* beta, const float* s0, int h, int t, int dk,
                        int dv, float* out, float* s_out) {
  float* s = (float*)malloc(sizeof(float) * (size_t)dk * dv);
  float* mem = (float*)malloc(sizeof(float) * (size_t)dv);
  for (int hh = 0; hh < h; ++hh) {
    if (s0)
      memcpy(s, s0 + (int64_t)hh * dk * dv, sizeof(float) * (size_t)dk * dv);
    else
      memset(s, 0, sizeof(float) * (size_t)dk * dv);
    for (int ti = 0; ti < t; ++ti) {
      const float* kt = kn + ((int64_t)hh * t + ti) * dk;
      const float* qt = qn + ((int64_t)hh * t + ti) * dk;
      const float* vt = v + ((int64_t)hh * t + ti) * dv;
      float gt = expf(g[(int64_t)hh * t + ti]);
      for (int i = 0; i < dk * dv; ++i) s[i] *= gt;
      float bt = beta[(int64_t)hh * t + ti];
      for (int j = 0; j < dv; ++j) {
        float m = 0.0f;
        for (int i = 0; i < dk; ++i) m += s[i * dv + j] * kt[i];
        mem[j] = (vt[j] - m) * bt;
      }
      for (int i = 0; i < dk; ++i)
        for (int j = 0; j < dv; ++j) s[i * dv + j] += kt[i] * mem[j];
      for (int j = 0; j < dv; ++j) {
        float o = 0.0f;
        for (int i = 0; i < dk; ++i) o += s[i * dv + j] * qt[i];
        out[((int64_t)hh * t + ti) * dv + j] = o;
      }
    }
    memcpy(s_out + (int64_t)hh * dk * dv, s, sizeof(float) * (size_t)dk * dv);
  }
  free(s);
  free(mem);
}

/* Depthwise causal conv over [tail || x] then SiLU, and the new tail
 * (qwen35.rs:428-430 with decoder.rs:137-151):
 *   x (c, t) channel-major; tail (c, kw-1) or NULL (zeros); w (c, kw).
 *   y[c][i] = silu( sum_{u<kw} full[c][i+u] * w[c][u] ), full = [tail || x]
 *   new_tail = last kw-1 columns of full.
 * bf16 != 0 rounds each product and partial sum to bf16 (model dtype ops)
 * and evaluates SiLU as bf16 ops. */
void orc_conv_silu(const float* x, const float* tail, const float* w, int c, int t, int kw, int bf16, float* y, float* new_tail) {
  int L = t + kw - 1;
  float* full = (float*)malloc(sizeof(float) * (size_t)L);
  for (int ch = 0; ch < c; ++ch) {
    for (int i = 0; i < kw - 1; ++i) full[i] = tail ? tail[(int64_t)ch * (kw - 1) + i] : 0.0f;
    for (int i = 0; i < t; ++i) full[kw - 1 + i] = x[(int64_t)ch * t + i];
    for (int i = 0; i < t; ++i) {
      float acc = 0.0f;
      for (int u = 0; u < kw; ++u) {
        float term = full[i + u] * w[(int64_t)ch * kw + u];
        if (bf16) term = bf16r_ext(term);
        acc = u == 0 ? term : acc + term;
        if (bf16) acc = bf16r_ext(acc);
      }
      float sv;
      if (bf16) {
        /* candle's bf16 SiLU: v / (1 + exp(-v)), each op in bf16 */
        float e = bf16r_ext(expf(-acc));
        float den = bf16r_ext(1.0f + e);
        sv = bf16r_ext(acc / den);
      } else {
        sv = acc / (1.0f + expf(-acc));
      }
      y[(int64_t)ch * t + i] = sv;
    }
    for (int i = 0; i < kw - 1; ++i) new_tail[(int64_t)ch * (kw - 1) + i] = full[t + i];
  }
  free(full);
}

/* Gated RMSNorm per head (qwen35.rs:447-451), f32 like the reference:
 *   y = core / sqrt(mean(core^2) + eps) * w * silu(z),  silu(z) = z / (1 + e^-z)
 * core, z: (rows, dv) f32 (z already cast from the model dtype); w: (dv).
 * bf16 != 0 rounds y to bf16 (the final .to_dtype(x.dtype())). */
void orc_gated_rmsnorm(const float* core, const float* z, const float* w, int64_t rows, int dv, float eps, int bf16, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* c = core + r * dv;
    float s = 0.0f;
    for (int i = 0; i < dv; ++i) s += c[i] * c[i];
    float den = sqrtf(s / (float)dv + eps);
    for (int i = 0; i < dv; ++i) {
      float zz = z[r * dv + i];
      float g = zz / (1.0f + expf(-zz));
      float v = c[i] / den * w[i] * g;
      y[r * dv + i] = bf16 ? bf16r_ext(v) : v;
    }
  }
}
