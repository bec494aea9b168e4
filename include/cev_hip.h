/*
 * cev_hip.h -- C ABI of the MI355X (gfx950) packed-prefill attention path.
 *
 * The library (libcev_hip.so) replaces the tensor ops under the reference's
 * attention call: the QK-norm + RoPE prologue of Attention::forward and the
 * matmul -> softmax -> matmul core of Attention::attend, with the dense
 * additive mask replaced by a block-offset table.  Reference sites (paths
 * relative to the reference checkout):
 *   crates/cev-model/src/qwen3.rs:187-220   Qwen3 Attention::forward / attend
 *   crates/cev-model/src/qwen35.rs:526-579  Qwen3.5 gated Attention::forward / attend
 *   crates/cev-model/src/engine.rs:389-442  the packed pass's dense mask
 *   crates/cev-model/src/qwen3.rs:153-169   segment_mask (chunked prefill)
 *   crates/cev-model/src/qwen35.rs:469-498  branch_mask / bidirectional_mask
 *
 * Conventions
 *   - Every entry point returns an int32 status: CEV_OK (0) or a negative
 *     CEV_ERR_*; cev_last_error() gives a thread-local message.  Nothing
 *     throws across the ABI.
 *   - Device pointers are caller-owned, borrowed for the stream-ordered
 *     launch and never retained.  Launchers allocate nothing.
 *   - Host functions (no stream argument) touch no GPU state.
 *   - Launchers keep no mutable global state: calls on distinct streams may
 *     run concurrently from several threads.
 *   - A stream is a hipStream_t passed as an opaque pointer (NULL = default).
 */
#ifndef CEV_HIP_H
#define CEV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CEV_ABI_VERSION 1

enum {
  CEV_OK = 0,
  CEV_ERR_INVALID = -1,     /* malformed argument, table or plan            */
  CEV_ERR_UNSUPPORTED = -2, /* a shape or dtype the kernels do not cover     */
  CEV_ERR_HIP = -3,         /* a HIP runtime error                           */
  CEV_ERR_SPACE = -4        /* caller buffer too small (see *_size)          */
};

enum { CEV_F32 = 0, CEV_BF16 = 1 };

#define CEV_MAX_SPANS 4

typedef void* cev_stream;
typedef void* cev_event; /* a hipEvent_t */

/* ------------------------------------------------------------------ */
/* Block-offset table.
 *
 * Keys live in one index space: [0, s_cache) are cached keys (the prefix
 * K/V, several plans' pasts concatenated as engine.rs:367-387 does), and
 * [s_cache, s_cache + t) are the keys of the t new tokens of this call.
 * A block is a run of packed query rows [q_begin, q_begin + q_len).  Row j
 * of the block (0-based) sees:
 *   - every key of every span (fully visible key ranges: the plan's past,
 *     the plan's prefix tail for question tokens);
 *   - causal != 0: local keys [local_begin, local_begin + j];
 *   - causal == 0 (bidirectional): local keys [local_begin, local_begin +
 *     valid_len), and a padded row (j >= valid_len) also its own key
 *     local_begin + j, so it never attends to nothing (qwen35.rs:491-494).
 * This expresses engine.rs:418-442, qwen3.rs:157-169 and qwen35.rs:469-498.
 * Spans must be disjoint from each other and from the block's own local
 * keys; blocks must not overlap.  Rows outside every block are left
 * untouched in the output. */
typedef struct {
  int32_t begin; /* first key (global key index) */
  int32_t len;   /* number of keys, >= 0        */
} cev_span;

typedef struct {
  int32_t q_begin;
  int32_t q_len;       /* >= 1 */
  int32_t valid_len;   /* bidirectional: real rows (0..q_len); causal: q_len */
  int32_t causal;      /* 1 causal, 0 bidirectional */
  int32_t local_begin; /* global key index of the block's own first token */
  int32_t n_spans;     /* 0..CEV_MAX_SPANS */
  cev_span spans[CEV_MAX_SPANS];
} cev_block;

/* ------------------------------------------------------------------ */
/* Attention descriptor.  Strides are in elements.  Shapes (reference
 * layout in brackets):
 *   q       (t, hq, d)          element (i, h, e) at q[i*q_stride_t + h*q_stride_h + e]
 *                               [(1, hq, t, d) in qwen3.rs:193]
 *   k/v_cache (hkv, s_cache, d) at (h, j, e): [h*kc_stride_h + j*kc_stride_s + e]
 *   k/v_new (t, hkv, d)         at (i, h, e): [i*kn_stride_t + h*kn_stride_h + e]
 *                               [the cat of qwen3.rs:197-200 is not needed]
 *   gate    (t, hq, d)          optional sigmoid gate (qwen35.rs:556-558)
 *   out     (t, hq, d)          [(1, hq, t, d) transposed for o_proj, qwen3.rs:202]
 * head h reads kv head h / (hq / hkv) (repeat_kv, qwen3.rs:145-151).
 * scale is applied to q.k before the softmax (reference: 1/sqrt(d) as f32,
 * qwen3.rs:207). */
typedef struct {
  int32_t dtype;      /* CEV_F32 or CEV_BF16: q, k, v, gate, out */
  int32_t n_q_heads;  /* hq */
  int32_t n_kv_heads; /* hkv, divides hq, hq/hkv <= 8 */
  int32_t head_dim;   /* 128 or 256 (f32: 128) */
  int32_t t;          /* packed new tokens = query rows */
  int32_t s_cache;    /* cached keys before the new tokens */
  float scale;
  int32_t has_gate;
  int64_t q_stride_t, q_stride_h;
  int64_t kc_stride_s, kc_stride_h;
  int64_t vc_stride_s, vc_stride_h;
  int64_t kn_stride_t, kn_stride_h;
  int64_t vn_stride_t, vn_stride_h;
  int64_t g_stride_t, g_stride_h;
  int64_t o_stride_t, o_stride_h;
  /* Key-range splitting: 0 lets the planner choose (split a tile's keys
   * over several workgroups when there are too few tiles to fill the GPU),
   * 1 disables it, n > 1 caps the parts per tile at n.  Split parts write
   * partial results to the workspace and a merge pass combines them, so
   * results can differ from an unsplit run in the last bits. */
  int32_t max_splits;
  int32_t reserved;
} cev_attn_desc;

/* Fills `d` with dense strides for the layouts above (token-major q, gate,
 * out; head-major cache; token-major new K/V), scale = 1/sqrt(head_dim). */
int32_t cev_attn_desc_init(cev_attn_desc* d, int32_t dtype, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t t,
                           int32_t s_cache, int32_t has_gate);

/* ------------------------------------------------------------------ */
/* Attention plan: the table compiled into work tiles (host only).
 * cev_attn_plan_size reports the bytes cev_attn_plan_build writes; both
 * validate the descriptor and the table and fail before anything runs.
 * The caller copies the plan to device memory (any copy API) and passes
 * both copies to cev_packed_attention: the host copy is read for
 * validation and the grid size, the device copy by the kernel. */
int32_t cev_attn_plan_size(const cev_attn_desc* d, const cev_block* blocks, int32_t n_blocks, size_t* bytes);
int32_t cev_attn_plan_build(const cev_attn_desc* d, const cev_block* blocks, int32_t n_blocks, void* plan, size_t bytes);

/* Device workspace bytes a plan needs (0 when no tile is split). */
int32_t cev_attn_workspace_size(const void* plan_host, size_t* bytes);

/* Packed-prefill attention: replaces Attention::attend
 * (qwen3.rs:206-220, qwen35.rs:563-579) plus the output gate of
 * qwen35.rs:556-558 when has_gate.  k_cache/v_cache may be NULL when
 * s_cache == 0, gate NULL when !has_gate, workspace NULL when the plan
 * needs none.  Calls sharing one workspace must not overlap. */
int32_t cev_packed_attention(const cev_attn_desc* d, const void* plan_host, const void* plan_dev, const void* q, const void* k_cache,
                             const void* v_cache, const void* k_new, const void* v_new, const void* gate, void* out, void* workspace,
                             size_t workspace_bytes, cev_stream stream);

/* Allocation-free variant of cev_packed_attention, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, hosts that forbid hipMalloc).  It has no counterpart in the
 * reference.  Same arguments, results and validation as
 * cev_packed_attention, but a split plan's partial records go to a static
 * device buffer of CEV_ATTN_SCRATCH_BYTES inside the library (one per GPU,
 * held until the process ends) instead of a caller workspace: a plan whose
 * cev_attn_workspace_size exceeds it fails with CEV_ERR_SPACE.  It calls no
 * hipMalloc / hipFree.  The first call on each device that needs the buffer
 * looks up its device address (hipGetSymbolAddress): make that call once
 * outside HIP graph capture (a warm-up); later calls, captured or not, make
 * no runtime call besides the launches.  Every call on one GPU shares the
 * buffer: calls that overlap in time on one GPU (several streams or
 * threads) race and must be serialised by the caller.  A call made while
 * another host thread is inside this function for the same device fails
 * with CEV_ERR_SPACE; work already queued on other streams is not seen. */
#define CEV_ATTN_SCRATCH_BYTES ((size_t)64 << 20)
int32_t cev_packed_attention_noalloc(const cev_attn_desc* d, const void* plan_host, const void* plan_dev, const void* q,
                                     const void* k_cache, const void* v_cache, const void* k_new, const void* v_new, const void* gate,
                                     void* out, cev_stream stream);

/* ------------------------------------------------------------------ */
/* Fused QK RMSNorm + RoPE with per-token positions: replaces
 * q_norm / k_norm + Rotary::apply of qwen3.rs:193-196 and the Qwen3.5 form
 * of qwen35.rs:529-539 (weight 1 + w, partial rotary, [q | gate] heads).
 *   q_in  (t, hq, d)  at q_in[i*qi_stride_t + h*qi_stride_h + e]   (gated q_proj: qi_stride_h = 2d)
 *   k_in  (t, hkv, d) at k_in[i*ki_stride_t + h*ki_stride_h + e]
 *   q_out, k_out likewise with qo_* / ko_* strides (k_out may point into
 *   the K/V cache).  pos (t) int32 positions; cos/sin (n_pos, rotary_dim/2)
 *   in the model dtype as built by cev_rope_table. */
typedef struct {
  int32_t dtype;
  int32_t n_q_heads, n_kv_heads, head_dim;
  int32_t t;
  int32_t rotary_dim;   /* even, <= head_dim */
  int32_t n_pos;        /* rows of the cos/sin table */
  int32_t weight_plus_one; /* 0: x*w (Qwen3); 1: x*(1+w) (Qwen3.5) */
  float eps;
  int64_t qi_stride_t, qi_stride_h;
  int64_t ki_stride_t, ki_stride_h;
  int64_t qo_stride_t, qo_stride_h;
  int64_t ko_stride_t, ko_stride_h;
} cev_qknorm_desc;

int32_t cev_qknorm_desc_init(cev_qknorm_desc* d, int32_t dtype, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t t,
                             int32_t rotary_dim, int32_t n_pos, int32_t weight_plus_one, float eps, int32_t gated_q);

int32_t cev_qknorm_rope(const cev_qknorm_desc* d, const void* q_in, const void* k_in, const void* w_q, const void* w_k, const int32_t* pos,
                        const void* cos, const void* sin, void* q_out, void* k_out, cev_stream stream);

/* cev_qknorm_rope plus the KV-cache store of the new tokens
 * (qwen3.rs:193-200 / qwen35.rs:536-544 up to the cat): q as above; the
 * normalised, rotated k row of token i and its v row (copied unchanged from
 * v_in (t, hkv, d) with strides vi_stride_t / vi_stride_h) are written to row
 * slots[i] of k_out and of v_out (strides ko_* and vo_stride_t /
 * vo_stride_h), e.g. a token's slot in a (hkv, capacity, d) cache.  slots
 * NULL writes row i; a slot outside [0, n_slots) stores neither row.  v rows
 * 16-byte aligned.  One launch. */
int32_t cev_qknorm_rope_kv(const cev_qknorm_desc* d, const void* q_in, const void* k_in, const void* v_in, int64_t vi_stride_t,
                           int64_t vi_stride_h, const void* w_q, const void* w_k, const int32_t* pos, const void* cos, const void* sin,
                           const int32_t* slots, int32_t n_slots, void* q_out, void* k_out, void* v_out, int64_t vo_stride_t,
                           int64_t vo_stride_h, cev_stream stream);

/* RoPE cos/sin table exactly as Rotary::new builds it (qwen3.rs:107-118):
 * inv_i = 1 / (theta^(2i/rotary_dim) in f64, rounded to f32), angle =
 * f32(p) * inv_i in f32, cos/sin in f32, then rounded to dtype.  Host only;
 * cos/sin are (n_pos, rotary_dim/2) arrays of f32 or bf16 (uint16 bits). */
int32_t cev_rope_table(double theta, int32_t rotary_dim, int32_t n_pos, int32_t dtype, void* cos, void* sin);

/* ------------------------------------------------------------------ */
/* Gated DeltaNet layer core (Qwen3.5 linear-attention layers): replaces
 * GatedDeltaNet::forward (crates/cev-model/src/qwen35.rs:414-453) between
 * the input projections and out_proj, i.e. the depthwise conv + SiLU with
 * its state (qwen35.rs:428-430, decoder.rs:137-151), l2norm / sigmoid /
 * softplus gates, chunk_gated_delta_rule (qwen35.rs:301-368) and the gated
 * RMSNorm (qwen35.rs:447-451). */
typedef struct cev_gdn_desc {
  int32_t dtype;       /* model dtype: projections, conv weight, conv state, y */
  int32_t batch;       /* rows B */
  int32_t t;           /* tokens per row */
  int32_t n_k_heads;   /* linear_num_key_heads */
  int32_t n_v_heads;   /* linear_num_value_heads, a multiple of n_k_heads */
  int32_t head_k_dim;  /* 128 */
  int32_t head_v_dim;  /* 128 */
  int32_t conv_kernel; /* linear_conv_kernel_dim, 2..8 */
  float eps;           /* rms_norm_eps of the gated norm */
  int32_t reserved;
  /* element strides; the channel stride is 1 */
  int64_t mixed_stride_b, mixed_stride_t; /* in_proj_qkv output (B, T, 2 nk dk + nv dv) */
  int64_t z_stride_b, z_stride_t;         /* in_proj_z output (B, T, nv dv) */
  int64_t ab_stride_b, ab_stride_t;       /* in_proj_b / in_proj_a outputs (B, T, nv) */
  int64_t conv_in_stride_b;               /* conv state (B, conv_dim, K-1); 0 broadcasts one state */
  int64_t s_in_stride_b;                  /* recurrent state (B, nv, dk, dv) f32; 0 broadcasts */
  int64_t y_stride_b, y_stride_t;         /* output (B, T, nv dv) */
} cev_gdn_desc;

/* Fills d with contiguous strides and validates it. */
int32_t cev_gdn_desc_init(cev_gdn_desc* d, int32_t dtype, int32_t batch, int32_t t, int32_t n_k_heads, int32_t n_v_heads,
                          int32_t head_k_dim, int32_t head_v_dim, int32_t conv_kernel, float eps);
int32_t cev_gdn_workspace_size(const cev_gdn_desc* d, size_t* bytes);

/* One layer for B rows of T tokens.  mixed, z, b, a, conv_w (conv_dim, K),
 * conv_in and y are in the model dtype; neg_a = -exp(A_log), dt_bias and
 * norm_w are f32 (as GatedDeltaNet::new holds them, qwen35.rs:393-395);
 * s_in / s_out are (B, nv, dk, dv) f32.  conv_in == NULL / s_in == NULL
 * start from zero state (qwen35.rs:426).  conv_out is (B, conv_dim, K-1)
 * contiguous.  Workspace of cev_gdn_workspace_size bytes, 256-byte
 * aligned. */
int32_t cev_gdn_forward(const cev_gdn_desc* d, const void* mixed, const void* z, const void* b, const void* a, const void* conv_w,
                        const float* neg_a, const float* dt_bias, const float* norm_w, const void* conv_in, const float* s_in, void* y,
                        void* conv_out, float* s_out, void* workspace, size_t workspace_bytes, cev_stream stream);

/* ------------------------------------------------------------------ */
/* Decoder-layer pieces around attention (the Qwen3 decoder stack's packed passes). */

/* RMSNorm of `rows` rows of `hidden` elements, candle_nn RmsNorm in the
 * model dtype (input_layernorm / post_attention_layernorm / final norm,
 * crates/cev-model/src/qwen3.rs:254-255, :400): y = dtype(dtype(x / m) * w),
 * m = dtype(sqrt(sum x^2 / hidden + eps)).
 * With h != NULL the residual add before the norm is fused in
 * (qwen3.rs:261 in mlp_block, :358 and :397): x_out = dtype(x + h) is written
 * (x_out may alias x) and normalised.  weight_plus_one selects 1 + w.
 * Strides are in elements; rows and buffers 16-byte aligned.
 * cev_rms_norm sums the squares in tree order (one wave per row; rows up to
 * 16 x 64 16-byte chunks, wider rows take the sequential sum);
 * cev_rms_norm_seq sums them in element order like candle's CPU kernel, so
 * its results are the sequential sum's bit for bit (validation). */
int32_t cev_rms_norm(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h, int64_t h_stride,
                     void* x_out, int64_t x_out_stride, const void* w, float eps, int32_t weight_plus_one, void* y, int64_t y_stride,
                     cev_stream stream);
int32_t cev_rms_norm_seq(int32_t dtype, int64_t rows, int32_t hidden, const void* x, int64_t x_stride, const void* h, int64_t h_stride,
                         void* x_out, int64_t x_out_stride, const void* w, float eps, int32_t weight_plus_one, void* y, int64_t y_stride,
                         cev_stream stream);

/* The SwiGLU of Mlp::forward (qwen3.rs:230-233): out = dtype(silu(gate) * up),
 * silu(v) = v / (1 + exp(-v)) with each op in the model dtype.  gate and up
 * share the row stride in_stride (e.g. the two halves of one fused GEMM
 * output). */
int32_t cev_swiglu(int32_t dtype, int64_t rows, int32_t inter, const void* gate, const void* up, int64_t in_stride, void* out,
                   int64_t out_stride, cev_stream stream);

/* Debiased readout scores: Service::run_debiased's averaging over rotated
 * question variants (crates/cev-runtime/src/service.rs:330-345) with
 * math::log_softmax in f64 (crates/cev-core/src/math.rs:14-18).  Question q
 * owns variants span_begin[q] .. span_begin[q] + span_len[q] - 1 and
 * n_options[q] options (1..min(ld, 64)); for each of its variants v in
 * order and position p < n_options[q]:
 *   scores[q][order[v][p]] += (log_softmax(logits[v])[p] - log_softmax(calib[v])[p]) / span_len[q]
 * (the calib term is 0 when calib is NULL: no calibration twins), then the
 * f64 sums are stored as f32.  logits, calib and order are (n_variants, ld)
 * row-major, scores (n_questions, ld); all device memory.  A question whose
 * span lies outside [0, n_variants), whose option count is out of range or
 * whose order is not a permutation of its options gets NaN scores. */
int32_t cev_debias_scores(int32_t n_questions, int32_t n_variants, const int32_t* span_begin, const int32_t* span_len,
                          const int32_t* n_options, const float* logits, const float* calib, const int32_t* order, int32_t ld,
                          float* scores, cev_stream stream);

/* Linear layers and row gathers (the candle ops around the attention call
 * in the device-resident stack and the readouts).
 *
 * cev_blas is a hipBLASLt context for products of more than 8 rows; it
 * caches one algorithm per problem shape.  Use a handle from one thread at a
 * time. */
typedef void* cev_blas;
int32_t cev_blas_create(cev_blas* handle);
int32_t cev_blas_destroy(cev_blas handle);

/* y = out_dtype(alpha * x . w^T): Linear::forward without bias
 * (crates/cev-model/src/qwen3.rs:175-178, :229-233), the code head
 * hidden . code_head^T (engine.rs:463) and the d3 readout
 * answers . weight^T / temperature (hybrid.rs:657, alpha = 1 / temperature
 * rounded to f32).  x (m, k) row stride ldx, w (n, k) row stride ldw, y (m, n)
 * row stride ldy, all row-major; x and w in `dtype`, y in out_dtype (CEV_F32
 * or dtype); f32 accumulation, one rounding to the output dtype.  m <= 8
 * runs this library's own kernel (handle may be NULL, no workspace); larger
 * m a hipBLASLt GEMM on `handle` with the caller's workspace
 * (CEV_LINEAR_WORKSPACE_BYTES recommended; 0 allowed).  x and w must be
 * 16-byte aligned with ldx, ldw multiples of 8 (bf16) or 4 (f32) elements;
 * for m > 8 the same holds for y and ldy in the output dtype. */
#define CEV_LINEAR_WORKSPACE_BYTES ((size_t)32 << 20)
int32_t cev_linear(cev_blas handle, int32_t dtype, int32_t out_dtype, int64_t m, int64_t n, int64_t k, const void* x, int64_t ldx,
                   const void* w, int64_t ldw, float alpha, void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                   cev_stream stream);

/* out[i] = out_dtype(table[ids[i]]) for i < n, rows of `width` elements:
 * Embedding::forward's rows (qwen3.rs:288-293), index_select of the answer
 * rows (qwen3.rs:399), to_dtype(F32) (qwen3.rs:400, ids NULL = identity)
 * and the code head's rows of the tied embedding (engine.rs:155).  ids is
 * a device int32 array; an id outside [0, table_rows) gives a NaN row. */
int32_t cev_gather_rows(int32_t dtype, int32_t out_dtype, int64_t n, int64_t width, const void* table, int64_t ld_table, int64_t table_rows,
                        const int32_t* ids, void* out, int64_t ld_out, cev_stream stream);

/* ------------------------------------------------------------------ */
/* Table builders (host only). */

/* The packed pass of engine.rs:365-442.  Plans p = 0..n_plans-1 in plan
 * order carry past_len[p] computed tokens (stored in the cache at the plan
 * order concatenation offset), prefix_len[p] and tail_start[p] (the first
 * prefix token not yet computed; == prefix_len[p] means no tail).  Items
 * k = 0..n_items-1 are questions (item_plan[k], item_len[k]).  Writes one
 * block per tail and per question (tails first, in plan order, then
 * questions in item order, as the reference packs tokens), pos[n] with the
 * per-question RoPE restart at prefix_len (engine.rs:411) and gather[k]
 * (engine.rs:415).  *n_tokens / *n_out_blocks receive the counts; with
 * NULL outputs only the counts are computed. */
int32_t cev_table_from_plans(int32_t n_plans, const int32_t* past_len, const int32_t* prefix_len, const int32_t* tail_start, int32_t n_items,
                             const int32_t* item_plan, const int32_t* item_len, cev_block* blocks, int32_t max_blocks, int32_t* n_out_blocks,
                             int32_t* pos, int32_t max_tokens, int32_t* n_tokens, int32_t* gather);

/* The packed pass of engine.rs:365-442 over slot-addressed K/V caches (a
 * cev_prefix_store): keys are cache slots, so a plan's past is read where
 * it lies and its tail is written next to it (no cat, engine.rs:375-387,
 * :449-457).  Plan p's prefix occupies slots [kv_begin[p], kv_begin[p] +
 * prefix_len[p]), its first tail_start[p] tokens already computed; the
 * rest (its tail) is computed by this pass.  Question k's tokens take slots
 * item_slot[k] .. + item_len[k] - 1.  Token order, positions (restarting
 * at prefix_len per question, engine.rs:411) and gather are those of
 * cev_table_from_plans; slots[i] receives the cache slot of pass token i
 * (for cev_qknorm_rope_kv).  Attend with s_cache = capacity (every key is a
 * cache slot) and t = *n_tokens.  A written slot range that overlaps any
 * other range of the pass is rejected.  A chunk of a prefix's prefill is a
 * plan with no questions whose tail is the chunk (qwen3.rs:346-362). */
int32_t cev_table_from_slots(int32_t n_plans, const int32_t* kv_begin, const int32_t* prefix_len, const int32_t* tail_start, int32_t n_items,
                             const int32_t* item_plan, const int32_t* item_len, const int32_t* item_slot, int32_t capacity, cev_block* blocks,
                             int32_t max_blocks, int32_t* n_out_blocks, int32_t* pos, int32_t* slots, int32_t max_tokens, int32_t* n_tokens,
                             int32_t* gather);

/* Device prefix store: the engine's PrefixCache (engine.rs:474-503) over
 * slot ranges of per-layer (hkv, capacity, d) device caches that the caller
 * owns; host bookkeeping only, thread-safe.  LRU by total cached tokens
 * (budget) with PrefixCache's get / put semantics; a range a pass holds
 * (get hit or reserve) stays allocated until released, also if evicted
 * meanwhile.  When no free run fits a reservation the oldest unheld entries
 * are evicted until one does; CEV_ERR_SPACE if none fits even then. */
typedef void* cev_prefix_store;
int32_t cev_prefix_store_create(int32_t capacity, int64_t budget, cev_prefix_store* store);
int32_t cev_prefix_store_destroy(cev_prefix_store store);
/* PrefixCache::get: *found = 1 and *begin = its first slot on a hit (now
 * most recently used, and held until released). */
int32_t cev_prefix_store_get(cev_prefix_store store, const uint32_t* tokens, int32_t n, int32_t* begin, int32_t* found);
/* n contiguous slots for this pass (a prefix being computed, question
 * tokens), held until released. */
int32_t cev_prefix_store_reserve(cev_prefix_store store, int32_t n, int32_t* begin);
/* PrefixCache::put of a held reservation of exactly n slots holding the
 * K/V of `tokens`; a key longer than the budget is not cached. */
int32_t cev_prefix_store_put(cev_prefix_store store, const uint32_t* tokens, int32_t n, int32_t begin);
int32_t cev_prefix_store_release(cev_prefix_store store, int32_t begin);
/* Entries, their total key length and the slots in use (entries + held). */
int32_t cev_prefix_store_stats(cev_prefix_store store, int32_t* entries, int64_t* cached_tokens, int32_t* used_slots);
/* Entry i in LRU order (0 = oldest): its first slot and length. */
int32_t cev_prefix_store_entry(cev_prefix_store store, int32_t i, int32_t* begin, int32_t* len);

/* Rows of a batch (HybridEngine::rows, hybrid.rs:592-617): b rows of t
 * tokens packed row-major.  causal != 0: each row continues `past` cached
 * keys (branch_mask, qwen35.rs:471-479); causal == 0: no cache, row r has
 * lengths[r] real tokens (bidirectional_mask, qwen35.rs:483-498). */
int32_t cev_table_from_rows(int32_t b, int32_t t, int32_t past, int32_t causal, const int32_t* lengths, cev_block* blocks, int32_t max_blocks);

/* segment_mask of qwen3.rs:157-169 for contiguous segments: n new tokens
 * after `past` cached ones, seg[i] their segment ids.  A segment id that
 * reappears after another one is rejected (CEV_ERR_UNSUPPORTED). */
int32_t cev_table_from_segment_ids(const uint32_t* seg, int32_t n, int32_t past, cev_block* blocks, int32_t max_blocks, int32_t* n_out_blocks);

/* Expands a table into the dense additive mask (t, s_cache + t) of 0 and
 * -inf, for validation against the reference mask. */
int32_t cev_table_to_dense_mask(const cev_block* blocks, int32_t n_blocks, int32_t t, int32_t s_cache, float* mask);

/* Recovers a table from a dense additive mask (t, s_cache + t): row i's
 * local run is the visible run holding its own key s_cache + i (or, for a
 * padded bidirectional row, the run before it); consecutive rows with equal
 * spans and a compatible local run form one block.  Fails with
 * CEV_ERR_UNSUPPORTED on patterns a table cannot express. */
int32_t cev_table_from_dense_mask(const float* mask, int32_t t, int32_t s_cache, cev_block* blocks, int32_t max_blocks, int32_t* n_out_blocks);

/* ------------------------------------------------------------------ */
/* Runtime helpers for hosts without a HIP binding (the Rust host). */
const char* cev_last_error(void);
int32_t cev_abi_version(void);
int32_t cev_device_info(int32_t device, char* name, size_t name_len, int32_t* n_cus, int64_t* hbm_bytes, int32_t* clock_mhz);
int32_t cev_malloc(void** ptr, size_t bytes);
int32_t cev_free(void* ptr);
int32_t cev_memcpy_h2d(void* dst, const void* src, size_t bytes, cev_stream stream);
int32_t cev_memcpy_d2h(void* dst, const void* src, size_t bytes, cev_stream stream);
int32_t cev_memcpy_d2d(void* dst, const void* src, size_t bytes, cev_stream stream);
int32_t cev_stream_create(cev_stream* stream);
int32_t cev_stream_destroy(cev_stream stream);
int32_t cev_stream_synchronize(cev_stream stream);
/* Kernel timing (the FFI crate's counterpart of the harness's event timers):
 * record `start` and `end` on the stream around the launches, synchronize
 * on `end`, then read the milliseconds between the two. */
int32_t cev_event_create(cev_event* event);
int32_t cev_event_destroy(cev_event event);
int32_t cev_event_record(cev_event event, cev_stream stream);
int32_t cev_event_synchronize(cev_event event);
int32_t cev_event_elapsed_ms(cev_event start, cev_event end, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* CEV_HIP_H */
