// Attention plan blob shared by the host planner (cev_host.cpp) and the
// packed-attention launcher / kernel (packed_attn.hip).
//
// Layout (all int32, 16-byte aligned sections):
//   header                 16 x int32
//   tiles[n_tiles]         {row_begin, row_count, seg_begin, seg_count}
//   segs[n_segs]           {key_begin, key_end, masked, 0}   global key index, end exclusive
//   rows[t]                {lo, hi, diag, 0}                 local keys a row sees:
//                          [lo, hi) plus diag (diag < 0: none)
// A tile is a run of query rows whose blocks share their span list; its
// segments are the spans (unmasked) and its rows' local keys (masked where
// not every row of the tile sees them).  No segment crosses s_cache.
#pragma once
#include <stdint.h>

#define CEV_PLAN_MAGIC 0x50564543  // "CEVP"
#define CEV_PLAN_VERSION 1

struct cev_plan_header {
  int32_t magic, version, n_tiles, n_segs;
  int32_t t, s_cache, tile_rows, dtype;
  int32_t head_dim, n_q_heads, n_kv_heads, tiles_off;  // offsets in int32 units
  int32_t segs_off, rows_off, bytes, reserved;
};
static_assert(sizeof(cev_plan_header) == 64, "plan header is 64 bytes");

// Waves per workgroup and query rows per tile for a GQA group size g:
// every wave owns 32 rows of one query head, the 8 waves of a workgroup
// cover all g heads of one KV head, so each staged K/V tile feeds 256
// queries (g heads x 256/g rows).
constexpr int kAttnWaves = 8;
static inline int cev_attn_tile_rows(int g) { return 32 * kAttnWaves / g; }
