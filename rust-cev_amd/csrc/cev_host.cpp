// Host half of libcev_hip.so: error reporting, descriptors, the block-offset
// table builders, the attention planner and the RoPE table.  Nothing here
// touches the GPU.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <utility>
#include <string>
#include <vector>

#include "cev_internal.h"
#include "cev_plan.h"

namespace {
thread_local std::string g_error;
}

int32_t cev_fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

void cev_clear_error() { g_error.clear(); }

extern "C" const char* cev_last_error(void) { return g_error.c_str(); }
extern "C" int32_t cev_abi_version(void) { return CEV_ABI_VERSION; }

// ---------------------------------------------------------------------
// Descriptors

extern "C" int32_t cev_attn_desc_init(cev_attn_desc* d, int32_t dtype, int32_t hq, int32_t hkv, int32_t hd, int32_t t, int32_t s_cache,
                                      int32_t has_gate) {
  CEV_CHECK_ARG(d != nullptr, "cev_attn_desc_init: null descriptor");
  memset(d, 0, sizeof *d);
  d->dtype = dtype;
  d->n_q_heads = hq;
  d->n_kv_heads = hkv;
  d->head_dim = hd;
  d->t = t;
  d->s_cache = s_cache;
  d->scale = (float)(1.0 / sqrt((double)(hd > 0 ? hd : 1)));
  d->has_gate = has_gate;
  d->q_stride_t = (int64_t)hq * hd;
  d->q_stride_h = hd;
  d->kc_stride_s = hd;
  d->kc_stride_h = (int64_t)s_cache * hd;
  d->vc_stride_s = hd;
  d->vc_stride_h = (int64_t)s_cache * hd;
  d->kn_stride_t = (int64_t)hkv * hd;
  d->kn_stride_h = hd;
  d->vn_stride_t = (int64_t)hkv * hd;
  d->vn_stride_h = hd;
  d->g_stride_t = (int64_t)hq * hd;
  d->g_stride_h = hd;
  d->o_stride_t = (int64_t)hq * hd;
  d->o_stride_h = hd;
  return CEV_OK;
}

extern "C" int32_t cev_qknorm_desc_init(cev_qknorm_desc* d, int32_t dtype, int32_t hq, int32_t hkv, int32_t hd, int32_t t, int32_t rot,
                                        int32_t n_pos, int32_t plus_one, float eps, int32_t gated_q) {
  CEV_CHECK_ARG(d != nullptr, "cev_qknorm_desc_init: null descriptor");
  memset(d, 0, sizeof *d);
  d->dtype = dtype;
  d->n_q_heads = hq;
  d->n_kv_heads = hkv;
  d->head_dim = hd;
  d->t = t;
  d->rotary_dim = rot;
  d->n_pos = n_pos;
  d->weight_plus_one = plus_one;
  d->eps = eps;
  int64_t qh = gated_q ? 2 * (int64_t)hd : hd;
  d->qi_stride_t = hq * qh;
  d->qi_stride_h = qh;
  d->ki_stride_t = (int64_t)hkv * hd;
  d->ki_stride_h = hd;
  d->qo_stride_t = (int64_t)hq * hd;
  d->qo_stride_h = hd;
  d->ko_stride_t = (int64_t)hkv * hd;
  d->ko_stride_h = hd;
  return CEV_OK;
}

// ---------------------------------------------------------------------
// RoPE table (qwen3.rs:107-118)

static inline uint16_t f32_to_bf16_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

extern "C" int32_t cev_rope_table(double theta, int32_t rot, int32_t n_pos, int32_t dtype, void* cos_out, void* sin_out) {
  CEV_CHECK_ARG(cos_out && sin_out, "cev_rope_table: null output");
  CEV_CHECK_ARG(rot > 0 && rot % 2 == 0, "cev_rope_table: rotary_dim %d must be positive and even", rot);
  CEV_CHECK_ARG(n_pos >= 0, "cev_rope_table: n_pos %d < 0", n_pos);
  CEV_CHECK_ARG(theta > 0.0, "cev_rope_table: theta must be positive");
  if (dtype != CEV_F32 && dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "cev_rope_table: dtype %d", dtype);
  const int half = rot / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i) inv[i] = 1.0f / (float)pow(theta, (double)(2 * i) / (double)rot);
  for (int64_t p = 0; p < n_pos; ++p) {
    const float fp = (float)p;
    for (int i = 0; i < half; ++i) {
      volatile float a = fp * inv[i];  // one rounded f32 product, never fused
      float c = cosf(a), s = sinf(a);
      int64_t k = p * half + i;
      if (dtype == CEV_F32) {
        ((float*)cos_out)[k] = c;
        ((float*)sin_out)[k] = s;
      } else {
        ((uint16_t*)cos_out)[k] = f32_to_bf16_bits(c);
        ((uint16_t*)sin_out)[k] = f32_to_bf16_bits(s);
      }
    }
  }
  return CEV_OK;
}

// ---------------------------------------------------------------------
// Table validation and planning

namespace {

struct Ival {
  int32_t b, e;  // [b, e)
};

}  // namespace

int32_t cev_check_attn_desc(const cev_attn_desc* d) {
  CEV_CHECK_ARG(d != nullptr, "null attention descriptor");
  if (d->dtype != CEV_F32 && d->dtype != CEV_BF16) return cev_fail(CEV_ERR_UNSUPPORTED, "dtype %d not supported", d->dtype);
  if (d->head_dim != 128 && d->head_dim != 256) return cev_fail(CEV_ERR_UNSUPPORTED, "head_dim %d not supported (128, 256)", d->head_dim);
  if (d->dtype == CEV_F32 && d->head_dim != 128) return cev_fail(CEV_ERR_UNSUPPORTED, "f32 attention supports head_dim 128 only");
  CEV_CHECK_ARG(d->n_q_heads > 0 && d->n_kv_heads > 0, "head counts must be positive (hq %d, hkv %d)", d->n_q_heads, d->n_kv_heads);
  CEV_CHECK_ARG(d->n_q_heads % d->n_kv_heads == 0, "hq %d is not a multiple of hkv %d", d->n_q_heads, d->n_kv_heads);
  int g = d->n_q_heads / d->n_kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return cev_fail(CEV_ERR_UNSUPPORTED, "GQA group %d not supported (1, 2, 4, 8)", g);
  CEV_CHECK_ARG(d->t >= 0 && d->s_cache >= 0, "negative t %d or s_cache %d", d->t, d->s_cache);
  CEV_CHECK_ARG((int64_t)d->t + d->s_cache <= INT32_MAX, "t + s_cache overflows the key index");
  CEV_CHECK_ARG(d->scale > 0.0f && isfinite(d->scale), "scale must be finite and positive");
  const int64_t* st[] = {&d->q_stride_t, &d->q_stride_h, &d->kc_stride_s, &d->kc_stride_h, &d->vc_stride_s, &d->vc_stride_h,
                         &d->kn_stride_t, &d->kn_stride_h, &d->vn_stride_t, &d->vn_stride_h, &d->o_stride_t, &d->o_stride_h};
  for (const int64_t* s : st) CEV_CHECK_ARG(*s >= 0, "negative stride");
  // 16-byte vector loads need every row start aligned to 8 elements (bf16)
  // or 4 (f32).
  const int64_t al = d->dtype == CEV_BF16 ? 8 : 4;
  for (const int64_t* s : st)
    if (*s % al) return cev_fail(CEV_ERR_UNSUPPORTED, "strides must be multiples of %lld elements", (long long)al);
  // K/V tiles are fetched with buffer loads whose byte range ends at the
  // tile's last valid key: rows must not overlap, and a tile of keys must
  // span less than 2 GiB.
  const int64_t esz = d->dtype == CEV_BF16 ? 2 : 4;
  const int64_t span_max = (INT32_MAX / 2) / 64 / esz;
  const int64_t* rows_c[] = {&d->kc_stride_s, &d->vc_stride_s};
  const int64_t* rows_n[] = {&d->kn_stride_t, &d->vn_stride_t};
  for (const int64_t* s : rows_c)
    if (d->s_cache > 0 && (*s < d->head_dim || *s > span_max))
      return cev_fail(CEV_ERR_UNSUPPORTED, "cache row stride %lld outside [head_dim, %lld]", (long long)*s, (long long)span_max);
  for (const int64_t* s : rows_n)
    if (d->t > 0 && (*s < d->head_dim || *s > span_max))
      return cev_fail(CEV_ERR_UNSUPPORTED, "new K/V row stride %lld outside [head_dim, %lld]", (long long)*s, (long long)span_max);
  if (d->has_gate) {
    CEV_CHECK_ARG(d->g_stride_t >= 0 && d->g_stride_h >= 0, "negative gate stride");
    if (d->g_stride_t % al || d->g_stride_h % al) return cev_fail(CEV_ERR_UNSUPPORTED, "gate strides must be multiples of %lld", (long long)al);
  }
  return CEV_OK;
}

namespace {

int32_t check_blocks(const cev_attn_desc* d, const cev_block* blocks, int32_t n) {
  CEV_CHECK_ARG(n >= 0, "negative block count %d", n);
  CEV_CHECK_ARG(n == 0 || blocks != nullptr, "null block table");
  const int64_t keys = (int64_t)d->s_cache + d->t;
  // Interval ends in int64: a begin near INT32_MAX plus a length must not
  // wrap to a small end that passes the range checks.
  struct Iv64 {
    int64_t b, e;
  };
  auto ov = [](Iv64 x, Iv64 y) { return x.b < y.e && y.b < x.e; };
  for (int32_t i = 0; i < n; ++i) {
    const cev_block& b = blocks[i];
    CEV_CHECK_ARG(b.q_len >= 1, "block %d: q_len %d < 1", i, b.q_len);
    CEV_CHECK_ARG(b.q_begin >= 0 && (int64_t)b.q_begin + b.q_len <= d->t, "block %d: rows [%d, %lld) outside [0, %d)", i, b.q_begin,
                  (long long)b.q_begin + b.q_len, d->t);
    CEV_CHECK_ARG(b.causal == 0 || b.causal == 1, "block %d: causal must be 0 or 1", i);
    if (b.causal)
      CEV_CHECK_ARG(b.valid_len == b.q_len, "block %d: a causal block has valid_len == q_len", i);
    else
      CEV_CHECK_ARG(b.valid_len >= 0 && b.valid_len <= b.q_len, "block %d: valid_len %d outside [0, %d]", i, b.valid_len, b.q_len);
    CEV_CHECK_ARG(b.n_spans >= 0 && b.n_spans <= CEV_MAX_SPANS, "block %d: n_spans %d outside [0, %d]", i, b.n_spans, CEV_MAX_SPANS);
    const Iv64 local{b.local_begin, (int64_t)b.local_begin + b.q_len};
    CEV_CHECK_ARG(b.local_begin >= 0 && local.e <= keys, "block %d: local keys [%d, %lld) outside [0, %lld)", i, b.local_begin,
                  (long long)local.e, (long long)keys);
    for (int s = 0; s < b.n_spans; ++s) {
      const Iv64 sp{b.spans[s].begin, (int64_t)b.spans[s].begin + b.spans[s].len};
      CEV_CHECK_ARG(b.spans[s].len >= 0 && sp.b >= 0 && sp.e <= keys, "block %d span %d: keys [%lld, %lld) outside [0, %lld)", i, s,
                    (long long)sp.b, (long long)sp.e, (long long)keys);
      if (b.spans[s].len == 0) continue;
      CEV_CHECK_ARG(!ov(sp, local), "block %d span %d overlaps the block's own keys", i, s);
      for (int s2 = 0; s2 < s; ++s2) {
        const Iv64 o{b.spans[s2].begin, (int64_t)b.spans[s2].begin + b.spans[s2].len};
        CEV_CHECK_ARG(!ov(sp, o), "block %d: spans %d and %d overlap", i, s2, s);
      }
    }
  }
  return CEV_OK;
}

bool same_spans(const cev_block& a, const cev_block& b) {
  if (a.n_spans != b.n_spans) return false;
  for (int s = 0; s < a.n_spans; ++s)
    if (a.spans[s].begin != b.spans[s].begin || a.spans[s].len != b.spans[s].len) return false;
  return true;
}

struct Plan {
  std::vector<int32_t> tiles, segs, rows;
  int32_t n_tiles = 0, n_segs = 0, tile_rows = 0, n_splits = 1, block_n = 0;
};

void push_seg(Plan& p, int32_t b, int32_t e, int32_t masked, int32_t s_cache) {
  if (e <= b) return;
  if (b < s_cache && e > s_cache) {
    push_seg(p, b, s_cache, masked, s_cache);
    push_seg(p, s_cache, e, masked, s_cache);
    return;
  }
  p.segs.insert(p.segs.end(), {b, e, masked, 0});
  p.n_segs++;
}

// A local run shorter than this is processed as one masked segment instead
// of an unmasked part plus a masked remainder: a short unmasked part would
// cost a mostly empty key tile of its own.
constexpr int32_t kMinFullLocal = 128;

int32_t build_plan(const cev_attn_desc* d, const cev_block* blocks, int32_t n, Plan& p) {
  int32_t rc = cev_check_attn_desc(d);
  if (rc) return rc;
  rc = check_blocks(d, blocks, n);
  if (rc) return rc;
  CEV_CHECK_ARG(d->max_splits >= 0, "max_splits %d < 0", d->max_splits);
  const int g = d->n_q_heads / d->n_kv_heads;
  p.tile_rows = cev_attn_tile_rows(g);
  p.block_n = cev_attn_block_n(d->dtype, d->head_dim);
  p.rows.assign((size_t)d->t * 4, 0);
  std::vector<int32_t> owner((size_t)d->t, -1);
  for (int32_t i = 0; i < d->t; ++i) p.rows[(size_t)i * 4 + 2] = -1;
  for (int32_t bi = 0; bi < n; ++bi) {
    const cev_block& b = blocks[bi];
    for (int32_t j = 0; j < b.q_len; ++j) {
      int32_t r = b.q_begin + j;
      if (owner[r] >= 0) return cev_fail(CEV_ERR_INVALID, "blocks %d and %d share query row %d", owner[r], bi, r);
      owner[r] = bi;
      int32_t* rw = &p.rows[(size_t)r * 4];
      if (b.causal) {
        rw[0] = b.local_begin;
        rw[1] = b.local_begin + j + 1;
        rw[2] = -1;
      } else {
        rw[0] = b.local_begin;
        rw[1] = b.local_begin + b.valid_len;
        rw[2] = j >= b.valid_len ? b.local_begin + j : -1;
      }
    }
  }
  std::vector<int32_t> order(n);
  for (int32_t i = 0; i < n; ++i) order[i] = i;
  std::sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return blocks[a].q_begin < blocks[b].q_begin; });
  // Runs of adjacent blocks sharing their span list: [order[oi], order[oj]).
  std::vector<std::pair<size_t, size_t>> runs;
  for (size_t oi = 0; oi < order.size();) {
    size_t oj = oi + 1;
    while (oj < order.size()) {
      const cev_block& prev = blocks[order[oj - 1]];
      const cev_block& cur = blocks[order[oj]];
      if (cur.q_begin != prev.q_begin + prev.q_len || !same_spans(cur, blocks[order[oi]])) break;
      ++oj;
    }
    runs.push_back({oi, oj});
    oi = oj;
  }
  auto run_rows = [&](std::pair<size_t, size_t> u) {
    const cev_block& first = blocks[order[u.first]];
    const cev_block& last = blocks[order[u.second - 1]];
    return std::make_pair(first.q_begin, last.q_begin + last.q_len);
  };
  // Rows per tile: a workgroup's tile_rows, or half of it for f32 plans whose
  // full tiles would fill at most half of one round of kSplitTargetWorkgroups.
  // An f32 key tile is MFMA-heavy, so a half-full workgroup takes about half
  // the time per key tile, and twice the workgroups spread the work over more
  // CUs (c1: K2 41.6 -> 32.4 us).  bf16 key tiles are fetch-bound: half-full
  // tiles measured slower than splitting the key stream (c5a: 261 against
  // 202 us), and on a full GPU half-full tiles would idle half the waves.
  int64_t full_tiles = 0;
  for (auto u : runs) {
    const auto rr = run_rows(u);
    full_tiles += (rr.second - rr.first + p.tile_rows - 1) / p.tile_rows;
  }
  const bool half = d->dtype == CEV_F32 && 2 * full_tiles * d->n_kv_heads <= kSplitTargetWorkgroups && p.tile_rows >= 2;
  const int32_t step = half ? p.tile_rows / 2 : p.tile_rows;
  for (auto u : runs) {
    const cev_block& first = blocks[order[u.first]];
    const int32_t r0 = run_rows(u).first, r1 = run_rows(u).second;
    for (int32_t tr = r0; tr < r1; tr += step) {
      const int32_t te = std::min(r1, tr + step);
      const int32_t seg_begin = p.n_segs;
      for (int s = 0; s < first.n_spans; ++s) push_seg(p, first.spans[s].begin, first.spans[s].begin + first.spans[s].len, 0, d->s_cache);
      // Local keys of the tile's rows: the part every row sees, and the union.
      int32_t full_b = INT32_MIN, full_e = INT32_MAX;
      std::vector<Ival> iv;
      for (int32_t r = tr; r < te; ++r) {
        const int32_t* rw = &p.rows[(size_t)r * 4];
        full_b = std::max(full_b, rw[0]);
        full_e = std::min(full_e, rw[1]);
        if (rw[1] > rw[0]) iv.push_back({rw[0], rw[1]});
        if (rw[2] >= 0) iv.push_back({rw[2], rw[2] + 1});
      }
      std::sort(iv.begin(), iv.end(), [](Ival a, Ival b) { return a.b < b.b; });
      std::vector<Ival> uni;
      for (Ival x : iv) {
        if (!uni.empty() && x.b <= uni.back().e)
          uni.back().e = std::max(uni.back().e, x.e);
        else
          uni.push_back(x);
      }
      const bool has_full = full_e - full_b >= kMinFullLocal;
      for (Ival u : uni) {
        if (has_full && full_b >= u.b && full_e <= u.e) {
          push_seg(p, u.b, full_b, 1, d->s_cache);
          push_seg(p, full_b, full_e, 0, d->s_cache);
          push_seg(p, full_e, u.e, 1, d->s_cache);
        } else {
          push_seg(p, u.b, u.e, 1, d->s_cache);
        }
      }
      int32_t chunks = 0;
      for (int32_t si = seg_begin; si < p.n_segs; ++si) {
        const int32_t len = p.segs[(size_t)si * 4 + 1] - p.segs[(size_t)si * 4];
        chunks += (len + p.block_n - 1) / p.block_n;
      }
      p.tiles.insert(p.tiles.end(), {tr, te - tr, seg_begin, p.n_segs - seg_begin, chunks, 0, 0, 0});
      p.n_tiles++;
    }
  }
  // Split the key stream of every tile when that shortens the launch (few
  // long-prefix rows leave the GPU underfilled): each part still gets at
  // least kSplitMinChunks (f32: kSplitMinChunksF32) key tiles.
  int32_t max_chunks = 0;
  for (int32_t ti = 0; ti < p.n_tiles; ++ti) max_chunks = std::max(max_chunks, p.tiles[(size_t)ti * 8 + 4]);
  const int64_t items = (int64_t)p.n_tiles * d->n_kv_heads;
  int64_t split = 1;
  if (items > 0 && d->max_splits != 1) {
    // Unsplit, or split into parts that fit one round of
    // kSplitTargetWorkgroups workgroups, whichever has the smaller modelled
    // time: rounds x the longest part's chunks, plus the merge pass when
    // split; on a tie the larger part count (a fuller round).
    const int min_chunks = d->dtype == CEV_F32 ? kSplitMinChunksF32 : kSplitMinChunks;
    int64_t cap = std::min<int64_t>(std::max(1, max_chunks / min_chunks), kSplitMax);
    if (d->max_splits > 1) cap = std::min<int64_t>(cap, d->max_splits);
    cap = std::min<int64_t>(cap, std::max<int64_t>(1, kSplitTargetWorkgroups / items));
    int64_t best = -1;
    for (int64_t sp = 1; sp <= cap; ++sp) {
      const int64_t rounds = (items * sp + kSplitTargetWorkgroups - 1) / kSplitTargetWorkgroups;
      const int64_t cost = rounds * ((max_chunks + sp - 1) / sp) + (sp > 1 ? kSplitMergeChunks : 0);
      if (best < 0 || cost <= best) {
        best = cost;
        split = sp;
      }
    }
  }
  p.n_splits = (int32_t)split;
  return CEV_OK;
}

size_t plan_bytes(const Plan& p) { return sizeof(cev_plan_header) + 4 * (p.tiles.size() + p.segs.size() + p.rows.size()); }

}  // namespace

extern "C" int32_t cev_attn_plan_size(const cev_attn_desc* d, const cev_block* blocks, int32_t n_blocks, size_t* bytes) {
  CEV_CHECK_ARG(bytes != nullptr, "cev_attn_plan_size: null output");
  Plan p;
  int32_t rc = build_plan(d, blocks, n_blocks, p);
  if (rc) return rc;
  *bytes = plan_bytes(p);
  return CEV_OK;
}

extern "C" int32_t cev_attn_plan_build(const cev_attn_desc* d, const cev_block* blocks, int32_t n_blocks, void* plan, size_t bytes) {
  CEV_CHECK_ARG(plan != nullptr, "cev_attn_plan_build: null plan buffer");
  CEV_CHECK_ARG(((uintptr_t)plan & 15) == 0, "cev_attn_plan_build: plan buffer must be 16-byte aligned");
  Plan p;
  int32_t rc = build_plan(d, blocks, n_blocks, p);
  if (rc) return rc;
  const size_t need = plan_bytes(p);
  if (bytes < need) return cev_fail(CEV_ERR_SPACE, "plan needs %zu bytes, buffer has %zu", need, bytes);
  if (need > (size_t)INT32_MAX) return cev_fail(CEV_ERR_UNSUPPORTED, "plan of %zu bytes is too large", need);
  cev_plan_header h;
  memset(&h, 0, sizeof h);
  h.magic = CEV_PLAN_MAGIC;
  h.version = CEV_PLAN_VERSION;
  h.n_tiles = p.n_tiles;
  h.n_segs = p.n_segs;
  h.t = d->t;
  h.s_cache = d->s_cache;
  h.tile_rows = p.tile_rows;
  h.dtype = d->dtype;
  h.head_dim = d->head_dim;
  h.n_q_heads = d->n_q_heads;
  h.n_kv_heads = d->n_kv_heads;
  h.tiles_off = sizeof(cev_plan_header) / 4;
  h.segs_off = h.tiles_off + (int32_t)p.tiles.size();
  h.rows_off = h.segs_off + (int32_t)p.segs.size();
  h.bytes = (int32_t)need;
  h.n_splits = p.n_splits;
  h.block_n = p.block_n;
  int32_t* out = (int32_t*)plan;
  memcpy(out, &h, sizeof h);
  if (!p.tiles.empty()) memcpy(out + h.tiles_off, p.tiles.data(), 4 * p.tiles.size());
  if (!p.segs.empty()) memcpy(out + h.segs_off, p.segs.data(), 4 * p.segs.size());
  if (!p.rows.empty()) memcpy(out + h.rows_off, p.rows.data(), 4 * p.rows.size());
  out[kPlanSigWord] = (int32_t)cev_plan_signature(out, (int32_t)(need / 4), kPlanSigWord);
  return CEV_OK;
}

extern "C" int32_t cev_attn_workspace_size(const void* plan_host, size_t* bytes) {
  CEV_CHECK_ARG(plan_host != nullptr && bytes != nullptr, "cev_attn_workspace_size: null argument");
  const cev_plan_header* h = (const cev_plan_header*)plan_host;
  CEV_CHECK_ARG(h->magic == CEV_PLAN_MAGIC && h->version == CEV_PLAN_VERSION, "cev_attn_workspace_size: not a plan");
  *bytes = h->n_splits > 1 ? (size_t)h->t * h->n_q_heads * h->n_splits * cev_attn_record_bytes(h->dtype, h->head_dim) : 0;
  return CEV_OK;
}

// ---------------------------------------------------------------------
// Table builders

extern "C" int32_t cev_table_from_plans(int32_t n_plans, const int32_t* past_len, const int32_t* prefix_len, const int32_t* tail_start,
                                        int32_t n_items, const int32_t* item_plan, const int32_t* item_len, cev_block* blocks,
                                        int32_t max_blocks, int32_t* n_out_blocks, int32_t* pos, int32_t max_tokens, int32_t* n_tokens,
                                        int32_t* gather) {
  CEV_CHECK_ARG(n_plans >= 0 && n_items >= 0, "negative plan or item count");
  CEV_CHECK_ARG(n_plans == 0 || (past_len && prefix_len && tail_start), "null plan arrays");
  CEV_CHECK_ARG(n_items == 0 || (item_plan && item_len), "null item arrays");
  // Past K/V of every plan, concatenated in plan order (engine.rs:367-387).
  std::vector<int64_t> past_off(n_plans);
  int64_t past_total = 0;
  for (int32_t p = 0; p < n_plans; ++p) {
    CEV_CHECK_ARG(past_len[p] >= 0 && prefix_len[p] >= 0, "plan %d: negative length", p);
    CEV_CHECK_ARG(tail_start[p] >= 0 && tail_start[p] <= prefix_len[p], "plan %d: tail_start %d outside [0, %d]", p, tail_start[p],
                  prefix_len[p]);
    CEV_CHECK_ARG(past_len[p] <= tail_start[p], "plan %d: past %d covers tail_start %d", p, past_len[p], tail_start[p]);
    past_off[p] = past_total;
    past_total += past_len[p];
  }
  // Tokens: tails first (segment 0), then questions (engine.rs:393-416).
  int64_t n = 0;
  int32_t nb = 0;
  std::vector<int64_t> tail_at(n_plans, -1);
  for (int32_t p = 0; p < n_plans; ++p) {
    int32_t tl = prefix_len[p] - tail_start[p];
    if (tl == 0) continue;
    tail_at[p] = n;
    n += tl;
    nb++;
  }
  for (int32_t k = 0; k < n_items; ++k) {
    CEV_CHECK_ARG(item_plan[k] >= 0 && item_plan[k] < n_plans, "item %d: plan %d outside [0, %d)", k, item_plan[k], n_plans);
    CEV_CHECK_ARG(item_len[k] >= 1, "item %d: empty question", k);
    n += item_len[k];
    nb++;
  }
  CEV_CHECK_ARG(past_total + n <= INT32_MAX, "pass too large");
  if (n_tokens) *n_tokens = (int32_t)n;
  if (n_out_blocks) *n_out_blocks = nb;
  if (!blocks && !pos && !gather) return CEV_OK;
  if (blocks && max_blocks < nb) return cev_fail(CEV_ERR_SPACE, "table needs %d blocks, buffer has %d", nb, max_blocks);
  if (pos && max_tokens < n) return cev_fail(CEV_ERR_SPACE, "pass has %lld tokens, buffer has %d", (long long)n, max_tokens);
  const int32_t s_cache = (int32_t)past_total;
  int32_t bi = 0;
  int64_t tok = 0;
  auto past_span = [&](int32_t p, cev_block& b) {
    if (past_len[p] > 0) b.spans[b.n_spans++] = {(int32_t)past_off[p], past_len[p]};
  };
  for (int32_t p = 0; p < n_plans; ++p) {
    if (tail_at[p] < 0) continue;
    int32_t tl = prefix_len[p] - tail_start[p];
    if (blocks) {
      cev_block& b = blocks[bi];
      memset(&b, 0, sizeof b);
      b.q_begin = (int32_t)tok;
      b.q_len = tl;
      b.valid_len = tl;
      b.causal = 1;  // a tail token sees its plan's tail causally (engine.rs:429)
      b.local_begin = s_cache + (int32_t)tok;
      past_span(p, b);
    }
    if (pos)
      for (int32_t j = 0; j < tl; ++j) pos[tok + j] = tail_start[p] + j;
    tok += tl;
    bi++;
  }
  for (int32_t k = 0; k < n_items; ++k) {
    int32_t p = item_plan[k];
    if (blocks) {
      cev_block& b = blocks[bi];
      memset(&b, 0, sizeof b);
      b.q_begin = (int32_t)tok;
      b.q_len = item_len[k];
      b.valid_len = item_len[k];
      b.causal = 1;  // earlier tokens of its own question (engine.rs:432-441)
      b.local_begin = s_cache + (int32_t)tok;
      past_span(p, b);
      if (tail_at[p] >= 0) b.spans[b.n_spans++] = {s_cache + (int32_t)tail_at[p], prefix_len[p] - tail_start[p]};
    }
    if (pos)
      for (int32_t j = 0; j < item_len[k]; ++j) pos[tok + j] = prefix_len[p] + j;  // restart (engine.rs:411)
    tok += item_len[k];
    if (gather) gather[k] = (int32_t)tok - 1;
    bi++;
  }
  return CEV_OK;
}

extern "C" int32_t cev_table_from_slots(int32_t n_plans, const int32_t* kv_begin, const int32_t* prefix_len, const int32_t* tail_start,
                                        int32_t n_items, const int32_t* item_plan, const int32_t* item_len, const int32_t* item_slot,
                                        int32_t capacity, cev_block* blocks, int32_t max_blocks, int32_t* n_out_blocks, int32_t* pos,
                                        int32_t* slots, int32_t max_tokens, int32_t* n_tokens, int32_t* gather) {
  CEV_CHECK_ARG(n_plans >= 0 && n_items >= 0 && capacity >= 0, "negative plan count, item count or capacity");
  CEV_CHECK_ARG(n_plans == 0 || (kv_begin && prefix_len && tail_start), "null plan arrays");
  CEV_CHECK_ARG(n_items == 0 || (item_plan && item_len && item_slot), "null item arrays");
  // Slot ranges this pass reads (computed prefixes) and writes (tails and
  // questions): inside the cache, and no written range may overlap another
  // range of the pass.
  struct Iv {
    int64_t b, e;
    bool write;
  };
  std::vector<Iv> iv;
  int64_t n = 0;
  int32_t nb = 0;
  for (int32_t p = 0; p < n_plans; ++p) {
    CEV_CHECK_ARG(prefix_len[p] >= 0 && tail_start[p] >= 0 && tail_start[p] <= prefix_len[p], "plan %d: tail_start %d outside [0, %d]", p,
                  tail_start[p], prefix_len[p]);
    CEV_CHECK_ARG(kv_begin[p] >= 0 && (int64_t)kv_begin[p] + prefix_len[p] <= capacity, "plan %d: slots [%d, %lld) outside [0, %d)", p,
                  kv_begin[p], (long long)kv_begin[p] + prefix_len[p], capacity);
    if (tail_start[p] > 0) iv.push_back({kv_begin[p], (int64_t)kv_begin[p] + tail_start[p], false});
    if (prefix_len[p] > tail_start[p]) {
      iv.push_back({(int64_t)kv_begin[p] + tail_start[p], (int64_t)kv_begin[p] + prefix_len[p], true});
      n += prefix_len[p] - tail_start[p];
      nb++;
    }
  }
  for (int32_t k = 0; k < n_items; ++k) {
    CEV_CHECK_ARG(item_plan[k] >= 0 && item_plan[k] < n_plans, "item %d: plan %d outside [0, %d)", k, item_plan[k], n_plans);
    CEV_CHECK_ARG(item_len[k] >= 1, "item %d: empty question", k);
    CEV_CHECK_ARG(item_slot[k] >= 0 && (int64_t)item_slot[k] + item_len[k] <= capacity, "item %d: slots [%d, %lld) outside [0, %d)", k,
                  item_slot[k], (long long)item_slot[k] + item_len[k], capacity);
    iv.push_back({item_slot[k], (int64_t)item_slot[k] + item_len[k], true});
    n += item_len[k];
    nb++;
  }
  std::sort(iv.begin(), iv.end(), [](const Iv& a, const Iv& b) { return a.b < b.b; });
  for (size_t i = 1; i < iv.size(); ++i)
    for (size_t j = i; j-- > 0;) {
      if (iv[j].e <= iv[i].b) break;
      if (iv[i].write || iv[j].write)
        return cev_fail(CEV_ERR_INVALID, "slots [%lld, %lld) written by this pass overlap [%lld, %lld)", (long long)iv[i].b,
                        (long long)iv[i].e, (long long)iv[j].b, (long long)iv[j].e);
    }
  CEV_CHECK_ARG((int64_t)capacity + n <= INT32_MAX, "pass too large");
  if (n_tokens) *n_tokens = (int32_t)n;
  if (n_out_blocks) *n_out_blocks = nb;
  if (!blocks && !pos && !slots && !gather) return CEV_OK;
  if (blocks && max_blocks < nb) return cev_fail(CEV_ERR_SPACE, "table needs %d blocks, buffer has %d", nb, max_blocks);
  if ((pos || slots) && max_tokens < n) return cev_fail(CEV_ERR_SPACE, "pass has %lld tokens, buffer has %d", (long long)n, max_tokens);
  // Tokens: tails first in plan order, then questions (engine.rs:393-416).
  int32_t bi = 0;
  int64_t tok = 0;
  for (int32_t p = 0; p < n_plans; ++p) {
    const int32_t tl = prefix_len[p] - tail_start[p];
    if (tl == 0) continue;
    if (blocks) {
      cev_block& b = blocks[bi];
      memset(&b, 0, sizeof b);
      b.q_begin = (int32_t)tok;
      b.q_len = tl;
      b.valid_len = tl;
      b.causal = 1;  // the tail sees its plan's past, and itself causally (engine.rs:429)
      b.local_begin = kv_begin[p] + tail_start[p];
      if (tail_start[p] > 0) b.spans[b.n_spans++] = {kv_begin[p], tail_start[p]};
    }
    for (int32_t j = 0; j < tl; ++j) {
      if (pos) pos[tok + j] = tail_start[p] + j;
      if (slots) slots[tok + j] = kv_begin[p] + tail_start[p] + j;
    }
    tok += tl;
    bi++;
  }
  for (int32_t k = 0; k < n_items; ++k) {
    const int32_t p = item_plan[k];
    if (blocks) {
      cev_block& b = blocks[bi];
      memset(&b, 0, sizeof b);
      b.q_begin = (int32_t)tok;
      b.q_len = item_len[k];
      b.valid_len = item_len[k];
      b.causal = 1;
      b.local_begin = item_slot[k];
      // the plan's past and tail are one contiguous run of slots
      if (prefix_len[p] > 0) b.spans[b.n_spans++] = {kv_begin[p], prefix_len[p]};
    }
    for (int32_t j = 0; j < item_len[k]; ++j) {
      if (pos) pos[tok + j] = prefix_len[p] + j;  // restart (engine.rs:411)
      if (slots) slots[tok + j] = item_slot[k] + j;
    }
    tok += item_len[k];
    if (gather) gather[k] = (int32_t)tok - 1;
    bi++;
  }
  return CEV_OK;
}

extern "C" int32_t cev_table_from_rows(int32_t b, int32_t t, int32_t past, int32_t causal, const int32_t* lengths, cev_block* blocks,
                                       int32_t max_blocks) {
  CEV_CHECK_ARG(b >= 0 && t >= 1 && past >= 0, "bad row batch (b %d, t %d, past %d)", b, t, past);
  CEV_CHECK_ARG(blocks != nullptr, "null block buffer");
  if (max_blocks < b) return cev_fail(CEV_ERR_SPACE, "table needs %d blocks, buffer has %d", b, max_blocks);
  CEV_CHECK_ARG((int64_t)b * t + past <= INT32_MAX, "row batch too large");
  if (!causal) {
    CEV_CHECK_ARG(past == 0, "bidirectional rows cannot continue a prefix state (qwen35.rs:547-549)");
    CEV_CHECK_ARG(lengths != nullptr, "bidirectional rows need lengths");
  }
  for (int32_t r = 0; r < b; ++r) {
    cev_block& bl = blocks[r];
    memset(&bl, 0, sizeof bl);
    bl.q_begin = r * t;
    bl.q_len = t;
    bl.causal = causal ? 1 : 0;
    bl.local_begin = past + r * t;
    if (causal) {
      bl.valid_len = t;
      if (past > 0) bl.spans[bl.n_spans++] = {0, past};
    } else {
      CEV_CHECK_ARG(lengths[r] >= 0 && lengths[r] <= t, "row %d: length %d outside [0, %d]", r, lengths[r], t);
      bl.valid_len = lengths[r];
    }
  }
  return CEV_OK;
}

extern "C" int32_t cev_table_from_segment_ids(const uint32_t* seg, int32_t n, int32_t past, cev_block* blocks, int32_t max_blocks,
                                              int32_t* n_out_blocks) {
  CEV_CHECK_ARG(n >= 0 && past >= 0, "negative n or past");
  CEV_CHECK_ARG(n == 0 || seg != nullptr, "null segment ids");
  std::vector<uint32_t> seen;
  int32_t nb = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (i > 0 && seg[i] == seg[i - 1]) continue;
    if (std::find(seen.begin(), seen.end(), seg[i]) != seen.end())
      return cev_fail(CEV_ERR_UNSUPPORTED, "segment %u reappears at token %d: only contiguous segments form blocks", seg[i], i);
    seen.push_back(seg[i]);
    nb++;
  }
  if (n_out_blocks) *n_out_blocks = nb;
  if (!blocks) return CEV_OK;
  if (max_blocks < nb) return cev_fail(CEV_ERR_SPACE, "table needs %d blocks, buffer has %d", nb, max_blocks);
  int32_t bi = -1;
  for (int32_t i = 0; i < n; ++i) {
    if (i == 0 || seg[i] != seg[i - 1]) {
      ++bi;
      cev_block& b = blocks[bi];
      memset(&b, 0, sizeof b);
      b.q_begin = i;
      b.causal = 1;
      b.local_begin = past + i;
      if (past > 0) b.spans[b.n_spans++] = {0, past};
    }
    blocks[bi].q_len++;
    blocks[bi].valid_len++;
  }
  return CEV_OK;
}

extern "C" int32_t cev_table_to_dense_mask(const cev_block* blocks, int32_t n_blocks, int32_t t, int32_t s_cache, float* mask) {
  cev_attn_desc d;
  cev_attn_desc_init(&d, CEV_F32, 1, 1, 128, t, s_cache, 0);
  CEV_CHECK_ARG(mask != nullptr, "null mask buffer");
  int32_t rc = check_blocks(&d, blocks, n_blocks);
  if (rc) return rc;
  const int64_t w = (int64_t)s_cache + t;
  for (int64_t i = 0; i < (int64_t)t * w; ++i) mask[i] = -INFINITY;
  for (int32_t bi = 0; bi < n_blocks; ++bi) {
    const cev_block& b = blocks[bi];
    for (int32_t j = 0; j < b.q_len; ++j) {
      float* row = mask + (int64_t)(b.q_begin + j) * w;
      for (int s = 0; s < b.n_spans; ++s)
        for (int32_t k = 0; k < b.spans[s].len; ++k) row[b.spans[s].begin + k] = 0.0f;
      const int32_t hi = b.causal ? j + 1 : b.valid_len;
      for (int32_t k = 0; k < hi; ++k) row[b.local_begin + k] = 0.0f;
      if (!b.causal && j >= b.valid_len) row[b.local_begin + j] = 0.0f;
    }
  }
  return CEV_OK;
}

// A row of the dense mask as its visible runs.
static void row_runs(const float* row, int64_t w, std::vector<Ival>& runs) {
  runs.clear();
  int64_t j = 0;
  while (j < w) {
    if (row[j] != 0.0f) {
      ++j;
      continue;
    }
    int64_t k = j;
    while (k < w && row[k] == 0.0f) ++k;
    runs.push_back({(int32_t)j, (int32_t)k});
    j = k;
  }
}

static bool runs_contain(const std::vector<Ival>& v, int32_t x) {
  for (Ival r : v)
    if (r.b <= x && x < r.e) return true;
  return false;
}

// v with key x added (x not in v), runs kept merged.
static std::vector<Ival> runs_add(const std::vector<Ival>& v, int32_t x) {
  std::vector<Ival> out;
  bool placed = false;
  for (Ival r : v) {
    if (!placed && x < r.b) {
      out.push_back({x, x + 1});
      placed = true;
    }
    out.push_back(r);
  }
  if (!placed) out.push_back({x, x + 1});
  std::vector<Ival> m;
  for (Ival r : out) {
    if (!m.empty() && r.b <= m.back().e)
      m.back().e = std::max(m.back().e, r.e);
    else
      m.push_back(r);
  }
  return m;
}

// v minus the keys [b, e).
static std::vector<Ival> runs_sub(const std::vector<Ival>& v, int32_t b, int32_t e) {
  std::vector<Ival> out;
  for (Ival r : v) {
    if (r.e <= b || r.b >= e) {
      out.push_back(r);
      continue;
    }
    if (r.b < b) out.push_back({r.b, b});
    if (r.e > e) out.push_back({e, r.e});
  }
  return out;
}

static bool runs_eq(const std::vector<Ival>& a, const std::vector<Ival>& b) {
  if (a.size() != b.size()) return false;
  for (size_t i = 0; i < a.size(); ++i)
    if (a[i].b != b[i].b || a[i].e != b[i].e) return false;
  return true;
}

extern "C" int32_t cev_table_from_dense_mask(const float* mask, int32_t t, int32_t s_cache, cev_block* blocks, int32_t max_blocks,
                                             int32_t* n_out_blocks) {
  CEV_CHECK_ARG(mask != nullptr && t >= 0 && s_cache >= 0, "bad dense mask arguments");
  const int64_t w = (int64_t)s_cache + t;
  for (int64_t i = 0; i < (int64_t)t * w; ++i)
    if (mask[i] != 0.0f && !(isinf(mask[i]) && mask[i] < 0))
      return cev_fail(CEV_ERR_UNSUPPORTED, "mask entry %lld is neither 0 nor -inf", (long long)i);
  std::vector<std::vector<Ival>> vis((size_t)t);
  for (int32_t i = 0; i < t; ++i) row_runs(mask + (int64_t)i * w, w, vis[i]);
  // Blocks start at a row r0 whose own key s_cache + r0 is its first local
  // key.  A causal block grows by one key (the row's own) per row; a
  // bidirectional block keeps one visible set for its real rows, and each
  // padded row adds its own key to it.
  std::vector<cev_block> out;
  int32_t i = 0;
  while (i < t) {
    const int32_t lb = s_cache + i;
    if (!runs_contain(vis[i], lb)) return cev_fail(CEV_ERR_UNSUPPORTED, "row %d does not see its own key", i);
    cev_block b;
    memset(&b, 0, sizeof b);
    b.q_begin = i;
    b.local_begin = lb;
    int32_t j = i + 1;
    const bool bidir = j < t && runs_eq(vis[j], vis[i]) && runs_contain(vis[i], s_cache + j);
    std::vector<Ival> spans;
    if (!bidir) {
      while (j < t && !runs_contain(vis[j - 1], s_cache + j) && runs_eq(vis[j], runs_add(vis[j - 1], s_cache + j))) ++j;
      b.causal = 1;
      b.q_len = j - i;
      b.valid_len = b.q_len;
      spans = runs_sub(vis[i], lb, lb + 1);
    } else {
      while (j < t && runs_eq(vis[j], vis[i]) && runs_contain(vis[i], s_cache + j)) ++j;
      const int32_t valid = j - i;
      for (int32_t k = 0; k < valid; ++k)
        if (!runs_contain(vis[i], lb + k)) return cev_fail(CEV_ERR_UNSUPPORTED, "row %d: bidirectional keys are not contiguous", i);
      while (j < t && !runs_contain(vis[i], s_cache + j) && runs_eq(vis[j], runs_add(vis[i], s_cache + j))) ++j;
      b.causal = 0;
      b.q_len = j - i;
      b.valid_len = valid;
      spans = runs_sub(vis[i], lb, lb + valid);
    }
    if (spans.size() > CEV_MAX_SPANS) return cev_fail(CEV_ERR_UNSUPPORTED, "row %d has %zu spans", i, spans.size());
    b.n_spans = (int32_t)spans.size();
    for (size_t s = 0; s < spans.size(); ++s) b.spans[s] = {spans[s].b, spans[s].e - spans[s].b};
    out.push_back(b);
    i = j;
  }
  if (n_out_blocks) *n_out_blocks = (int32_t)out.size();
  if (!blocks) return CEV_OK;
  if (max_blocks < (int32_t)out.size()) return cev_fail(CEV_ERR_SPACE, "table needs %zu blocks, buffer has %d", out.size(), max_blocks);
  memcpy(blocks, out.data(), sizeof(cev_block) * out.size());
  return CEV_OK;
}
