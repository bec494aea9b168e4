// Attention plan blob shared by the host planner (cev_host.cpp) and the
// packed-attention launcher / kernel (packed_attn.hip).
//
// Layout (all int32, 16-byte aligned sections):
//   header                 16 x int32
//   tiles[n_tiles]         {row_begin, row_count, seg_begin, seg_count,
//                           n_chunks, 0, 0, 0}
//   segs[n_segs]           {key_begin, key_end, masked, 0}   global key index, end exclusive
//   rows[t]                {lo, hi, diag, 0}                 local keys a row sees:
//                          [lo, hi) plus diag (diag < 0: none)
// A tile is a run of query rows whose blocks share their span list; its
// segments are the spans (unmasked) and its rows' local keys (masked where
// not every row of the tile sees them).  No segment crosses s_cache.  A
// tile's keys are visited in key tiles of block_n keys (n_chunks of them);
// with n_splits > 1 each tile's chunks are cut into n_splits contiguous
// parts, one workgroup per (tile, part, kv head).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define CEV_HD __host__ __device__
#else
#define CEV_HD
#endif

#define CEV_PLAN_MAGIC 0x50564543  // "CEVP"
#define CEV_PLAN_VERSION 3

// Signature of a plan blob: FNV-1a over its int32 words with the `sig`
// word itself taken as zero.  The launcher passes the host plan's
// signature to the kernels, which compare it with the device copy's.
CEV_HD static inline uint32_t cev_plan_signature(const int32_t* words, int32_t n_words, int32_t sig_index) {
  uint32_t h = 2166136261u;
  for (int32_t i = 0; i < n_words; ++i) {
    const uint32_t w = i == sig_index ? 0u : (uint32_t)words[i];
    for (int b = 0; b < 4; ++b) {
      h ^= (w >> (8 * b)) & 0xffu;
      h *= 16777619u;
    }
  }
  return h;
}

struct cev_plan_header {
  int32_t magic, version, n_tiles, n_segs;
  int32_t t, s_cache, tile_rows, dtype;
  int32_t head_dim, n_q_heads, n_kv_heads, tiles_off;  // offsets in int32 units
  int32_t segs_off, rows_off, bytes, n_splits;
  int32_t block_n, sig, reserved[2];
};
static_assert(sizeof(cev_plan_header) == 80, "plan header is 80 bytes");
constexpr int32_t kPlanSigWord = 17;  // index of `sig` among the plan's int32 words
static_assert(__builtin_offsetof(cev_plan_header, sig) == 4 * kPlanSigWord, "sig word index");

// Waves per workgroup and query rows per tile for a GQA group size g:
// every wave owns 32 rows of one query head, the 8 waves of a workgroup
// cover all g heads of one KV head, so each staged K/V tile feeds 256
// queries (g heads x 256/g rows).
constexpr int kAttnWaves = 8;
CEV_HD static inline int cev_attn_tile_rows(int g) { return 32 * kAttnWaves / g; }

// Keys per LDS key tile: 64 for bf16 d=128, 32 otherwise (LDS and
// register budget of the two head dims and of f32).
CEV_HD static inline int cev_attn_block_n(int dtype, int head_dim) { return (dtype == 1 && head_dim == 128) ? 64 : 32; }

// Bytes per (row, head, part) partial record in the split workspace.  The
// workspace holds two regions, both indexed by (row * n_q_heads + head) *
// n_splits + part: first every record's unnormalised output (head_dim
// values: bf16 for bf16 models, f32 for f32 models; 256 or 512 bytes, so
// each output starts on a 128-byte line and no line is shared by two
// parts), then every record's running max m (log2 units) and sum l as two
// f32.  The merge rounds its result to the model dtype, so a bf16 model's
// partial output loses nothing it keeps.
CEV_HD static inline int64_t cev_attn_record_out_bytes(int dtype, int head_dim) {
  return (dtype == 1 ? 2 : 4) * (int64_t)head_dim;
}
CEV_HD static inline int64_t cev_attn_record_bytes(int dtype, int head_dim) { return cev_attn_record_out_bytes(dtype, head_dim) + 8; }

// Split policy.  One attention workgroup fills a CU (its LDS and 8 waves of
// >128 VGPRs), so a launch runs in rounds of 256 workgroups on MI355X.  The
// planner keeps the tiles whole or splits them into parts that fit one
// round, whichever minimises rounds x chunks of the longest part + the
// merge pass (counted as kSplitMergeChunks chunk steps), never cutting a key
// stream into parts of fewer than kSplitMinChunks chunks (kSplitMinChunksF32
// for f32, whose 32-key chunk is about eight times the work of a bf16
// 64-key chunk).  Measured: the 32k-prefix x 16-token shape (8 tile x head
// items) 32 parts 38 us, 64 parts 49 us; the 28-layer Qwen3-1.7B-shaped pass's attention (224
// items) unsplit 86.7 us, 2 parts 119.8 us; the f32 12 x 32-token shape
// after a 256-token prefix (24 items of 12 chunks) 3 parts 50 us, 6 parts
// 38 us, 10 parts 39 us; 512 workgroups (two rounds) were slower on every
// shape tried.
constexpr int kSplitTargetWorkgroups = 256;
constexpr int kSplitMinChunks = 4;
constexpr int kSplitMinChunksF32 = 2;
constexpr int kSplitMergeChunks = 3;
constexpr int kSplitMax = 256;
