/*
 * hga.h -- C ABI of the MI355X (gfx950) routed exact-token attention library (libhga.so).
 *
 * Each entry point replaces one step of the reference's HierarchicalGlobalAttentionRouted path
 * (vfedosov77/HierarchicalGlobalAttention, ExistingModelFineTuning/); the reference location is
 * cited on each declaration.  All data pointers are device memory owned by the caller unless a
 * comment says otherwise; no entry point allocates device memory.  Activations are laid out as
 * 4-D views [B, X, S, Dh] with the head dimension contiguous and explicit element strides for
 * (b, x, s).  Every call is asynchronous on `stream` (a hipStream_t; NULL = default stream) and
 * returns HGA_OK or a negative code; hga_last_error() then describes the failure (per thread).
 */
#ifndef HGA_H
#define HGA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { HGA_DTYPE_F32 = 0, HGA_DTYPE_BF16 = 1 };

enum {
    HGA_OK = 0,
    HGA_ERR_ARG = -1,         /* invalid argument / shape */
    HGA_ERR_UNSUPPORTED = -2, /* valid but outside what the kernels implement */
    HGA_ERR_LAUNCH = -3,      /* HIP launch / runtime error */
};

/* Router flags */
enum {
    HGA_ROUTE_CANONICAL = 1, /* score every candidate with the canonical fp32 FMA chain
                                (no MFMA pre-pass); slower, same result */
    HGA_ROUTE_SPLIT = 2,     /* bf16: separate stage-1 and stage-2 kernels instead of the fused
                                one; same result */
};

/* Layer configuration; mirrors RouterConfig + ChunkPlacementPolicy
 * (KvRouter/chunk_router.py:58-90, KvRouter/chunk_placement_policy.py:12-38). */
typedef struct hga_config {
    int32_t batch;       /* B */
    int32_t heads;       /* H, query heads */
    int32_t kv_heads;    /* KVH; heads % kv_heads == 0, query head h reads KV head h/(H/KVH) */
    int32_t head_dim;    /* Dh: 16, 32, 64 or 128 */
    int32_t chunk_size;  /* C <= 64 */
    int32_t group_size;  /* gs; C % gs == 0 */
    int32_t topk_chunks; /* 0 disables routing */
    int32_t topk_groups; /* 0 disables group opening */
    int32_t keep_first;  /* sink window, token level (first_token_level=True) */
    int32_t keep_last;   /* local window */
    int32_t cutoff_pair; /* mixed-RoPE: pairs [0, cutoff) are summed token-wise */
    int32_t dtype;       /* HGA_DTYPE_* of q/k/v and summaries */
    float scale;         /* head_dim ** -0.5 rounded to fp32 */
    float group_scale;   /* 1 / (gs + sqrt(gs)) rounded to fp32 */
} hga_config;

/* Library version (major*10000 + minor*100 + patch). */
int32_t hga_version(void);

/* Text of the last error on this thread ("" if none). */
const char* hga_last_error(void);

/* Widths of the routing outputs for a prefill block of S tokens at position 0:
 * N = ceil(S/C), Kc = min(topk_chunks, N) (0 if disabled), Kg = min(topk_groups, Kc*C/gs).
 * Replaces the size logic of vectorized.py:233-240, 304, 345, 365. */
int32_t hga_prefill_widths(const hga_config* cfg, int32_t S, int32_t* N, int32_t* Kc,
                           int32_t* Kg);

/*
 * Rotate-half RoPE:
 *   out = x*cos + cat(-x2, x1)*sin
 * flags = 0: computed in fp32 and rounded once to the activation dtype
 *   (HierarchicalGlobalAttentionRouted.py:156-157, 219-223);
 * flags = HGA_ROPE_STEPS_IN_DTYPE: each product and the sum rounded to the activation dtype,
 *   as transformers' apply_rotary_pos_emb computes it on bf16 tensors (the Qwen3 drop-in,
 *   Qwen3LongContext/qwen_routed_attention.py:176, and its DCA twin :80-84).
 * x/out: [B, nheads, S, Dh] views; cos/sin: fp32 [Bc, S, Dh] rows of the rotary table for the
 * block's positions (bf16-valued when the model's table is bf16), cos_bstride = 0 (shared) or
 * the batch stride in elements.
 */
#define HGA_ROPE_STEPS_IN_DTYPE 1
int hga_rope(const hga_config* cfg, int32_t nheads, int32_t S, const void* x, int64_t x_sb,
             int64_t x_sh, int64_t x_ss, void* out, int64_t o_sb, int64_t o_sh, int64_t o_ss,
             const float* cos, const float* sin, int64_t cos_bstride, int32_t flags,
             void* stream);

/* q and k of one block in a single launch (the two rotations of
 * HierarchicalGlobalAttentionRouted.py:156-157 / qwen_routed_attention.py:176): q [B, heads, S,
 * Dh] and k [B, kv_heads, S, Dh] views, same tables, flags and results as two hga_rope calls. */
int hga_rope_qk(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb, int64_t q_sh,
                int64_t q_ss, void* q_out, int64_t qo_sb, int64_t qo_sh, int64_t qo_ss,
                const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, void* k_out,
                int64_t ko_sb, int64_t ko_sh, int64_t ko_ss, const float* cos, const float* sin,
                int64_t cos_bstride, int32_t flags, void* stream);

/*
 * Mixed-RoPE chunk and group key summaries at KV-head granularity
 * (vectorized._rope_summary, vectorized.py:146-183, as applied at :265-287; the store twin
 * ChunkRouter._rope_summary_at, chunk_router.py:575-585, 631-652, 693-735).
 * k_raw/k_rope: [B, KVH, S, Dh] views of the block (block token 0 at absolute position pos0,
 * a multiple of C).  cos_tab/sin_tab: fp32 [*, Dh] tables indexed by absolute position
 * (pos0 + local anchor).  Writes chunk n of the block to
 *   chunk_k + b*ck_sb + h*ck_sh + n*Dh            (dtype, [.., N, Dh])
 *   group_k + b*gk_sb + h*gk_sh + (n*M + m)*Dh     (dtype, [.., N, M, Dh])
 * The optional second table/output pair (cos_b, sin_b, chunk_k_b, group_k_b; all NULL or all
 * set, same strides) receives the same summaries with a second anchor table (the reference
 * routes with the activation-dtype table and seeds its store with the fp32 one).
 */
int hga_summarize(const hga_config* cfg, int32_t S, int64_t pos0, const void* k_raw,
                  int64_t kr_sb, int64_t kr_sh, int64_t kr_ss, const void* k_rope, int64_t kp_sb,
                  int64_t kp_sh, int64_t kp_ss, const float* cos_tab, const float* sin_tab,
                  void* chunk_k, int64_t ck_sb, int64_t ck_sh, void* group_k, int64_t gk_sb,
                  int64_t gk_sh, const float* cos_b, const float* sin_b, void* chunk_k_b,
                  void* group_k_b, void* stream);

/*
 * Two-level prefill routing for a fresh block starting at position 0
 * (vectorized.py:242-396: windows, stage-1 chunk routing with per-row requests, pooled max,
 * forced previous chunk, cumsum visibility; stage-2 group routing).  Canonical semantics:
 * scores are the fp32 FMA chain over Dh times `scale`, ties go to the lower absolute index.
 * q: [B, H, S, Dh] view (RoPE applied).  chunk_k/group_k: summaries as hga_summarize writes
 * them.  Outputs (contiguous int32, ascending ids, -1 padded):
 *   sel_chunk, sel_thr [B, H, N, Kc]   routed chunk id and first query row (chunk-local) that
 *                                      sees it; n_sel [B, H, N]
 *   open_grp, open_thr [B, H, N, Kg]   opened group id (chunk*M + group) and first row;
 *                                      n_open [B, H, N]
 * Widths from hga_prefill_widths (a zero width still needs 1-element arrays).
 * stats: NULL or int32[4] device counters, incremented by the number of rows whose MFMA
 * pre-pass could not certify the selection and were re-ranked canonically
 * ([0] stage-1 rows, [1] stage-1 pooled, [2] stage-2 rows, [3] stage-2 pooled).
 */
int hga_route_prefill(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                      int64_t q_sh, int64_t q_ss, const void* chunk_k, int64_t ck_sb,
                      int64_t ck_sh, const void* group_k, int64_t gk_sb, int64_t gk_sh,
                      int32_t* sel_chunk, int32_t* sel_thr, int32_t* n_sel, int32_t* open_grp,
                      int32_t* open_thr, int32_t* n_open, int32_t flags, int32_t* stats,
                      void* stream);

/*
 * Exact attention over the routed working set of a prefill block (the assembly of
 * vectorized.py:404-490 and RoutedKV.attend, chunk_router.py:149-158, fused; nothing is
 * materialised).  Row t of query chunk n attends to: its own chunk's tokens <= t, the
 * keep_first and keep_last windows, and every opened group with open_thr <= t.
 * q/out: [B, H, S, Dh]; k/v: [B, KVH, S, Dh] (RoPE'd keys).  open_grp/open_thr as written by
 * hga_route_prefill (width Kg; Kg = 0 with 1-element arrays when routing is off).
 * lse: NULL, or fp32 [B, H, S] receiving each row's log-sum-exp of its scores times
 * scale*log2(e) (log2 units), which hga_attend_prefill_bwd can take instead of recomputing it.
 */
int hga_attend_prefill(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                       int64_t q_sh, int64_t q_ss, const void* k, int64_t k_sb, int64_t k_sh,
                       int64_t k_ss, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                       const int32_t* open_grp, const int32_t* open_thr, int32_t Kg, void* out,
                       int64_t o_sb, int64_t o_sh, int64_t o_ss, float* lse, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* Device scratch bytes hga_attend_prefill needs for a block of S tokens (16-key blocked copies
 * of K and V, 2*B*KVH*Dh*roundup(S,64) bf16 elements, for bf16 head_dim 64/128 with group and
 * chunk sizes that are multiples of 16; 0 otherwise).
 * The buffer must be 16-byte aligned and is only used during the call's kernels (stream
 * ordered).  No counterpart in the reference, whose attend materialises K/V instead. */
int32_t hga_attend_prefill_workspace(const hga_config* cfg, int32_t S, int64_t* bytes);

/*
 * Gradient of hga_attend_prefill for an upstream gradient dout (the reference trains through
 * the same attention with torch autograd, HierarchicalGlobalAttentionRouted.py:137-177 over the
 * working set of vectorized.py:404-490; routing carries no gradient).  q/out/dout/dq:
 * [B, H, S, Dh]; k/v/dk/dv: [B, KVH, S, Dh]; out is hga_attend_prefill's output for the same
 * inputs and routing, lse NULL or hga_attend_prefill's lse output for them (then the rows'
 * softmax statistics are not recomputed).  dk/dv sum the contributions of every query head of a
 * KV head.
 * chunk_size <= 64.  workspace: hga_attend_prefill_bwd_workspace bytes, 16-byte aligned (fp32
 * accumulators, cleared by the call's own kernels).
 */
int hga_attend_prefill_bwd(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                           int64_t q_sh, int64_t q_ss, const void* k, int64_t k_sb, int64_t k_sh,
                           int64_t k_ss, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                           const void* out, int64_t o_sb, int64_t o_sh, int64_t o_ss,
                           const void* dout, int64_t g_sb, int64_t g_sh, int64_t g_ss,
                           const float* lse, const int32_t* open_grp, const int32_t* open_thr,
                           int32_t Kg,
                           void* dq, int64_t dq_sb, int64_t dq_sh, int64_t dq_ss, void* dk,
                           int64_t dk_sb, int64_t dk_sh, int64_t dk_ss, void* dv, int64_t dv_sb,
                           int64_t dv_sh, int64_t dv_ss, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* Device scratch bytes hga_attend_prefill_bwd needs (2*B*KVH*S*Dh fp32).  No counterpart in the
 * reference, where autograd allocates the gradient buffers. */
int32_t hga_attend_prefill_bwd_workspace(const hga_config* cfg, int32_t S, int64_t* bytes);

/* Widths of the decode routing outputs with n_closed closed chunks: the routing pool is
 * [f_hi, l_lo) of ChunkPlacementPolicy (chunk_placement_policy.py:27-38), Kc = min(topk_chunks,
 * |pool|), Kg = min(topk_groups, Kc*C/gs)  (chunk_router.py:213-257). */
int32_t hga_decode_widths(const hga_config* cfg, int32_t n_closed, int32_t* Kc, int32_t* Kg);

/*
 * Decode routing of an L-token block inside the active chunk (ChunkRouter._route_decision,
 * chunk_router.py:187-277): canonical fp32 scores of every row against the closed-chunk
 * summaries of the routing pool; chunks pooled by the max over all L rows, top-Kc selected,
 * chunk n_closed-1 forced in when it is in the pool, each row requests its own top-Kc (first
 * requesting row = visibility threshold, 0 for the forced chunk); all M groups of the selected
 * chunks scored, top-Kg opened by the max over rows, each row requests its top-(topk_groups/2),
 * a group is visible from max(first request, parent threshold).  Ties -> lower id.
 * q: [B, H, L, Dh] view.  chunk_k element (b, kvh, c, :) at chunk_k + b*ck_sb + kvh*ck_sh +
 * c*Dh; group_k element (b, kvh, c, m, :) at group_k + b*gk_sb + kvh*gk_sh + (c*M+m)*Dh.
 * Outputs (int32, ascending ids, -1 padded, widths from hga_decode_widths, >= 1):
 *   mid, mid_thr [B, H, Kc]  routed chunks visible to some row; n_mid [B, H]
 *   open_grp, open_thr [B, H, Kg]  opened groups (chunk*M + group) visible to some row; n_open
 * workspace: hga_route_decode_workspace bytes (the pool's segments' candidate lists), 4-byte
 * aligned, used only by the call's kernels.  Pools of up to (2048 / topk_chunks) * 2048 chunks
 * (262144 chunks, 16.7M tokens at topk_chunks 16 and chunk_size 64; longer ones are refused with
 * HGA_ERR_UNSUPPORTED); L <= 64, topk_chunks <= 64.
 */
int hga_route_decode(const hga_config* cfg, int32_t L, int32_t n_closed, const void* q,
                     int64_t q_sb, int64_t q_sh, int64_t q_ss, const void* chunk_k,
                     int64_t ck_sb, int64_t ck_sh, const void* group_k, int64_t gk_sb,
                     int64_t gk_sh, int32_t* mid, int32_t* mid_thr, int32_t* n_mid,
                     int32_t* open_grp, int32_t* open_thr, int32_t* n_open, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* Device scratch bytes hga_route_decode needs for an L-row block after n_closed chunks.  No
 * counterpart in the reference, whose router keeps its scores in torch temporaries. */
int32_t hga_route_decode_workspace(const hga_config* cfg, int32_t L, int32_t n_closed,
                                   int64_t* bytes);

/*
 * Decode attention (decode_block's assembly, chunk_router.py:333-401, attended flat as in
 * RoutedKV.attend, :159-162).  Row l sits at absolute position start_pos + l in active chunk
 * n_closed and attends to the first window [0, f_hi*C), the last window [l_lo*C, n_closed*C),
 * every opened group with open_thr <= l, and active tokens [n_closed*C, start_pos + l].
 * Token sources (K and V share strides; element strides b, kv head, position):
 *   recent  positions >= l_lo*C (last window + active chunk); position p at slot p when
 *           ring_chunks == 0, else at slot (p/C % ring_chunks)*C + p%C;
 *   first   positions [0, f_hi*C) at slot p;
 *   record  the whole closed-token record at slot p, read for opened groups; device memory, or
 *           pinned host memory (hipHostMalloc / torch pin_memory) when record_on_host != 0 --
 *           the kernel then reads the opened groups across PCIe directly (zero copy).
 * q/out: [B, H, L, Dh] views.
 */
int hga_attend_decode(const hga_config* cfg, int32_t L, int32_t n_closed, int64_t start_pos,
                      const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                      const void* k_recent, const void* v_recent, int64_t r_sb, int64_t r_sh,
                      int64_t r_ss, int32_t ring_chunks, const void* k_first,
                      const void* v_first, int64_t f_sb, int64_t f_sh, int64_t f_ss,
                      const void* k_record, const void* v_record, int64_t d_sb, int64_t d_sh,
                      int64_t d_ss, int32_t record_on_host, const int32_t* open_grp,
                      const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                      int64_t o_sh, int64_t o_ss, void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * hga_attend_decode in two launches, so that the opened groups can be copied from the host
 * record while the windows are attended (the reference starts the non-blocking group copy,
 * ram_kv_cache_store.py:578-607, before the attention that needs it, chunk_router.py:251-252).
 * phase 1 attends the first window, the last window and the active chunk into the workspace
 * (open_grp/open_thr only give each head's opened-list length; the record is not read); phase 2
 * -- later on the stream, or after an event, with the same arguments and workspace except that
 * open_grp and the record may be hga_gather_decode's staging -- attends the opened groups and
 * writes out.  phase 0 is hga_attend_decode.  head_dim 64 or 128.  Same workspace size
 * (hga_attend_decode_workspace).
 */
int hga_attend_decode_phase(const hga_config* cfg, int32_t L, int32_t n_closed, int64_t start_pos,
                            const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                            const void* k_recent, const void* v_recent, int64_t r_sb,
                            int64_t r_sh, int64_t r_ss, int32_t ring_chunks, const void* k_first,
                            const void* v_first, int64_t f_sb, int64_t f_sh, int64_t f_ss,
                            const void* k_record, const void* v_record, int64_t d_sb,
                            int64_t d_sh, int64_t d_ss, int32_t record_on_host,
                            const int32_t* open_grp, const int32_t* open_thr, int32_t Kg,
                            void* out, int64_t o_sb, int64_t o_sh, int64_t o_ss, int32_t phase,
                            void* workspace, int64_t workspace_bytes, void* stream);

/*
 * hga_attend_decode without a workspace: the split partials go to a static device array of the
 * library (32 MiB on each device the library runs on, held until the process ends; the device
 * current at the call), so neither the call nor the library allocates device memory.  No
 * counterpart in the reference: for callers that cannot allocate (code under HIP graph capture,
 * serving loops that forbid allocation).  Blocks whose partials (hga_attend_decode_workspace)
 * exceed 32 MiB are refused with HGA_ERR_UNSUPPORTED.  Calls that overlap on one device (two
 * streams or threads) race on the array; nothing in it needs clearing between calls.
 */
int hga_attend_decode_noalloc(const hga_config* cfg, int32_t L, int32_t n_closed,
                              int64_t start_pos, const void* q, int64_t q_sb, int64_t q_sh,
                              int64_t q_ss, const void* k_recent, const void* v_recent,
                              int64_t r_sb, int64_t r_sh, int64_t r_ss, int32_t ring_chunks,
                              const void* k_first, const void* v_first, int64_t f_sb,
                              int64_t f_sh, int64_t f_ss, const void* k_record,
                              const void* v_record, int64_t d_sb, int64_t d_sh, int64_t d_ss,
                              int32_t record_on_host, const int32_t* open_grp,
                              const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                              int64_t o_sh, int64_t o_ss, void* stream);

/*
 * Dual Chunk Attention decode (QwenRoutedAttention._dca_attend,
 * Qwen3LongContext/qwen_routed_attention.py:244-283): the same key sequence and visibility as
 * hga_attend_decode over keys stored RoPE'd at pos % dca_chunk.  Key p is scored against
 *   q_intra  when p / dca_chunk == (start_pos + l) / dca_chunk,
 *   q_succ   when it is the DCA chunk before,
 *   q_inter  otherwise,
 * the three fp32 [B, H, L, Dh] views (shared strides) of row l RoPE'd at pos % dca_chunk,
 * min(pos % dca_chunk + dca_chunk, ceil) and ceil.  dca_chunk is a positive multiple of the
 * chunk size.  open_pos holds the opened groups' own ids when open_grp indexes a staging record
 * (hga_gather_decode's staged_grp), else NULL (open_grp's ids are the positions).  Same
 * workspace as hga_attend_decode (hga_attend_decode_workspace).  out in the activation dtype.
 */
int hga_attend_decode_dca(const hga_config* cfg, int32_t L, int32_t n_closed,
                          int64_t start_pos, const float* q_intra, const float* q_succ,
                          const float* q_inter, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                          int32_t dca_chunk, const void* k_recent, const void* v_recent,
                          int64_t r_sb, int64_t r_sh, int64_t r_ss, int32_t ring_chunks,
                          const void* k_first, const void* v_first, int64_t f_sb, int64_t f_sh,
                          int64_t f_ss, const void* k_record, const void* v_record,
                          int64_t d_sb, int64_t d_sh, int64_t d_ss, int32_t record_on_host,
                          const int32_t* open_grp, const int32_t* open_pos,
                          const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                          int64_t o_sh, int64_t o_ss, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* Device scratch bytes hga_attend_decode needs (head_dim 64 / 128: the key sequence is split
 * over workgroups of 256 keys whose fp32 partials [B*H*L, splits, head_dim+2] are merged by a
 * second kernel; 0 for other head dims).  16-byte aligned, used only by the call's kernels
 * (stream ordered).  No counterpart in the reference. */
int32_t hga_attend_decode_workspace(const hga_config* cfg, int32_t L, int32_t n_closed,
                                    int64_t start_pos, int32_t Kg, int64_t* bytes);

/*
 * Decode token ingest (chunk_router.py:317 decode_block -> _append_active, :603-614, together
 * with the store's token write): up to three row sets of [B, KVH, L, head_dim] rows of cfg's
 * dtype, each copied from src to dst in one launch: the block's RoPE'd keys and its values into
 * the token record or ring, its raw keys into the active-chunk buffer.  Each set gives element
 * strides (batch, KV head, row) with a contiguous head dim, rows 16-byte aligned; a set with both
 * pointers NULL is skipped.  Offsets are 64-bit, so the rows may lie anywhere in a record of any
 * size.
 */
int hga_write_tokens(const hga_config* cfg, int32_t L, const void* k, int64_t k_sb, int64_t k_sh,
                     int64_t k_ss, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                     const void* k_raw, int64_t r_sb, int64_t r_sh, int64_t r_ss, void* dst_k,
                     int64_t dk_sb, int64_t dk_sh, int64_t dk_ss, void* dst_v, int64_t dv_sb,
                     int64_t dv_sh, int64_t dv_ss, void* dst_raw, int64_t dr_sb, int64_t dr_sh,
                     int64_t dr_ss, void* stream);

/* Sizes for hga_gather_decode: staging capacity per (batch, KV head) in groups (rep * Kg, the
 * most distinct groups the rep query heads can open), bytes of each of the K and V staging
 * buffers ([B, KVH, stage_groups, group_size, head_dim]) and bytes of the int32 scratch. */
int32_t hga_gather_decode_sizes(const hga_config* cfg, int32_t Kg, int32_t* stage_groups,
                                int64_t* stage_bytes, int64_t* scratch_bytes);

/*
 * Decode gather (the store I/O of ram_kv_cache_store.py:_gather_record / gather_tokens,
 * :560-607, done once per KV head instead of once per query head): the groups opened by
 * hga_route_decode (open_grp/open_thr [B, H, Kg]) are deduplicated over the rep query heads of
 * each KV head and copied, in ascending group order, from the closed-token record (pinned host
 * memory read over PCIe when record_on_host != 0, else device memory; element strides b, kv
 * head, position) into stage_k / stage_v [B, KVH, stage_groups, group_size, head_dim].
 * staged_grp [B, H, Kg] receives each opened group's staging slot (-1 for padding / invisible).
 * Since a slot s occupies positions [s*gs, s*gs + gs) of the staging buffer viewed as a record,
 * hga_attend_decode with that view (d_sb = KVH*stage_groups*gs*Dh, d_sh = stage_groups*gs*Dh,
 * d_ss = Dh, record_on_host 0) and open_grp = staged_grp attends exactly as with the record.
 * scratch: int32[B*KVH*(stage_groups+1)] (slot lists and counts).
 */
int hga_gather_decode(const hga_config* cfg, int32_t n_closed, const int32_t* open_grp,
                      const int32_t* open_thr, int32_t Kg, const void* k_record,
                      const void* v_record, int64_t d_sb, int64_t d_sh, int64_t d_ss,
                      int32_t record_on_host, void* stage_k, void* stage_v, int32_t stage_groups,
                      int32_t* staged_grp, void* scratch, int64_t scratch_bytes, void* stream);

/*
 * Decode attention over a host (or page-cache) record with the opened groups' copy overlapped:
 * RoutedKV.attend for the RAM / disk tiers (chunk_router.py:139-162) with the store's
 * non-blocking group copy started before the attention that needs it
 * (ram_kv_cache_store.py:578-607, chunk_router.py:251-252), in one call: hga_gather_decode of
 * record_grp (the opened groups as ids into the record, record_chunks chunks of it) into the
 * staging runs on `stream` while hga_attend_decode_phase phase 1 attends the windows and the
 * active chunk on a side stream of the library (default priority, one per thread and device,
 * ordered after everything issued on `stream` so far); phase 2 then attends the staged groups
 * (staged_grp) on `stream` after both.  Arguments as hga_attend_decode_phase (open_grp: the
 * lists of hga_route_decode, for the list lengths) and hga_gather_decode; the result equals
 * hga_attend_decode over the record.  head_dim 64 or 128.
 */
int hga_attend_decode_overlapped(
    const hga_config* cfg, int32_t L, int32_t n_closed, int64_t start_pos, const void* q,
    int64_t q_sb, int64_t q_sh, int64_t q_ss, const void* k_recent, const void* v_recent,
    int64_t r_sb, int64_t r_sh, int64_t r_ss, int32_t ring_chunks, const void* k_first,
    const void* v_first, int64_t f_sb, int64_t f_sh, int64_t f_ss, const void* k_record,
    const void* v_record, int64_t d_sb, int64_t d_sh, int64_t d_ss, int32_t record_on_host,
    int32_t record_chunks, const int32_t* record_grp, const int32_t* open_grp,
    const int32_t* open_thr, int32_t Kg, void* stage_k, void* stage_v, int32_t stage_groups,
    int32_t* staged_grp, void* scratch, int64_t scratch_bytes, void* out, int64_t o_sb,
    int64_t o_sh, int64_t o_ss, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HGA_H */
