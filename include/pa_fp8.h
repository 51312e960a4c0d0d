/*
 * pa_fp8.h - C ABI of the MI355X (gfx950) FP8 paged-attention decode library.
 *
 * The library (libpa_fp8.so) exports hand-written HIP kernels for the
 * split-context decode of the reference's `pa_decode_ps_launch` routes and a
 * few host-side planning helpers.  Every tensor is passed as a raw device
 * pointer plus element strides; the library never allocates device memory.
 * Its only mutable global state is two per-device caches, each entry written
 * once with one value: the compute-unit count of a device and the address of
 * pa_fp8_decode_balanced_static's scratch on it.  Both are keyed on the
 * device of the stream a call is launched on (hipStreamGetDevice; the
 * current device for the null stream), so calls are re-entrant, may target
 * any device's stream, and may be captured into a HIP graph when the caller
 * preallocates every buffer.  A checked build (libpa_fp8_checked.so, see
 * pa_fp8_debug_violations) also keeps one word of violation bits per source
 * file on each device.
 *
 * Return codes: 0 on success, a positive hipError_t value when the HIP
 * runtime rejects a launch, or one of the negative PA_ERR_* codes below for
 * arguments the kernels do not support.  pa_fp8_error_string() names them.
 *
 * Tensor layouts (element strides; the innermost dimension is contiguous):
 *   query        [B * ql, Hq, D]            bf16 or f16
 *   key_cache    [NB, Hkv, D / 16, bs, 16]  fp8 e4m3fn (OCP)
 *   value_cache  trans [NB, Hkv, bs / 16, D, 16] or plain [NB, Hkv, D, bs]
 *   block_tables [B, max_blocks]            int32 physical page per logical page
 *   context_lengths [B]                     int32
 *   key/value scale  per tensor: [1] float32
 *                    per token:  [NB, Hkv, bs, 1] float32
 *   exp_sums, max_logits [B, Hkv, P, ql * gqa] float32
 *   tmp_out      [B, Hkv, P, ql * gqa, D]   bf16 or float32
 *   output       [B * ql, Hq, D]            bf16, f16 or float32
 * where gqa = Hq / Hkv and P is the number of context slots.
 *
 * Head sizes D = 64, 128, ..., 512 (every multiple of 64 up to 512) and any
 * ql * gqa are decoded by the partition, reduce and work-list entry points;
 * D = 128 with up to 64 query columns per kv head runs on the tuned
 * kernels, every other shape on generic ones (one wave per 16-column block,
 * K and V read straight into MFMA operands) with the same outputs.  The
 * balanced decode takes D = 128 and up to 64 columns only.
 */
#ifndef PA_FP8_H
#define PA_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_FP8_ABI_VERSION 1

enum pa_fp8_dtype {
  PA_DTYPE_BF16 = 0,
  PA_DTYPE_F16 = 1,
  PA_DTYPE_F32 = 2,
};

enum pa_fp8_error {
  PA_OK = 0,
  PA_ERR_NULL_ARG = -1,       /* a required pointer is NULL */
  PA_ERR_HEAD_SIZE = -2,      /* head_size not a multiple of 64 in [64, 512] (balanced decode: not 128) */
  PA_ERR_BLOCK_SIZE = -3,     /* page size not 16 or a multiple of 32 up to 1024 */
  PA_ERR_GROUP = -4,          /* ql * gqa above an entry point's limit:
                               *  - pa_fp8_decode_balanced, pa_fp8_merge_balanced,
                               *    pa_fp8_decode_balanced_static and
                               *    pa_fp8_stream_workers: above 64;
                               *  - pa_fp8_decode_partition at head_size 128 with
                               *    min(slots_per_workgroup, num_partitions) > 4
                               *    (a wave walks several slots): above 16.
                               * The partition, reduce and work-list entry points
                               * take any ql * gqa otherwise. */
  PA_ERR_DTYPE = -5,          /* unsupported query / output / partial dtype */
  PA_ERR_SHAPE = -6,          /* non-positive dimension or partition count */
  PA_ERR_ALIGN = -7,          /* a pointer or stride breaks 16-byte alignment */
  PA_ERR_ABI = -8,            /* struct abi_version mismatch */
  PA_ERR_SCRATCH = -9,        /* workspace beyond the static scratch of pa_fp8_decode_balanced_static */
};

/*
 * Split-context partition pass.
 *
 * Replaces the compiled launchers of the reference:
 *   compile_pa_decode_ps(...)["launch"]   kernels/pa_decode_fp8.py:2738-2802
 *     (page size 16 / 64 small-block route, sliding_window == 0), and
 *   compile_pa_decode_sw(...)["launch"]   kernels/pa_decode_swa.py:1644-1718
 *     (sliding_window > 0; generalised here to any supported page size).
 * Grid: one workgroup per (sequence, kv head, slot).  Slot z of a sequence
 * covers the token range of pa_fp8_plan_slot(); it stores, per query column
 * e = qi * gqa + g, exp_sums = sum exp(l - m), max_logits = m (the slot's
 * maximum scaled logit, natural-log units; -inf when empty) and the
 * normalised partial output tmp_out.  When one workgroup covers all slots
 * of its (sequence, kv head) (slots_per_workgroup >= num_partitions) it
 * also merges them by log-sum-exp (the math of pa_fp8_decode_reduce) and
 * writes the final output, so one launch completes the decode; with one
 * slot this is the reference's fused single-partition window kernel
 * (kernels/pa_decode_swa.py:1480-1620).
 */
typedef struct pa_fp8_partition_args {
  int32_t abi_version; /* = PA_FP8_ABI_VERSION */
  /* outputs */
  float* exp_sums;
  float* max_logits;
  void* tmp_out;
  /* Final output [B * ql, Hq, D], or NULL.  Written only by a launch whose
   * workgroups each cover every slot (slots_per_workgroup >=
   * num_partitions); the partial buffers may then be NULL as well. */
  void* output;
  /* inputs */
  const void* query;
  const void* key_cache;
  const void* value_cache;
  const int32_t* block_tables;
  /* Optional.  When non-NULL the page list of sequence b is the flat
   * kv_page_indices layout of the reference's persistent route:
   * block_tables + kv_indptr[b] .. block_tables + kv_indptr[b + 1]
   * (stride_bt_seq and max_blocks_per_seq are then ignored). */
  const int32_t* kv_indptr;
  const int32_t* context_lengths;
  const float* key_scale;
  const float* value_scale;
  /* element strides */
  int64_t stride_q_tok, stride_q_head;
  int64_t stride_k_block, stride_k_head;
  int64_t stride_v_block, stride_v_head;
  int64_t stride_es_seq, stride_es_head, stride_es_part;
  int64_t stride_to_seq, stride_to_head, stride_to_part, stride_to_group;
  int64_t stride_bt_seq;
  int64_t stride_ks_block, stride_ks_head; /* per-token scales only */
  int64_t stride_out_tok, stride_out_head; /* fused output only */
  /* sizes */
  int32_t num_seqs;
  int32_t num_kv_heads;
  int32_t num_partitions;
  /* Slots one workgroup walks (its waves stream them back to back):
   * 1 = one workgroup per slot (grid B * Hkv * P, merge with
   * pa_fp8_decode_reduce); >= num_partitions = one workgroup per
   * (sequence, kv head) that also merges the slots into `output`.  More
   * slots than waves per workgroup (4) needs query_length * gqa <= 16. */
  int32_t slots_per_workgroup;
  int32_t query_length;
  int32_t query_group_size;
  int32_t head_size;
  int32_t block_size;
  int32_t num_blocks;          /* pages in the cache: page indices are clamped to it */
  int32_t max_blocks_per_seq;  /* block_tables row length */
  int32_t sliding_window;      /* 0 = full causal context */
  int32_t per_token_kv;        /* 0 = per-tensor scales, 1 = [NB, Hkv, bs, 1] */
  int32_t trans_v;             /* 1 = trans value layout */
  int32_t query_dtype;         /* PA_DTYPE_BF16 / PA_DTYPE_F16 */
  int32_t tmp_dtype;           /* PA_DTYPE_BF16 / PA_DTYPE_F32 */
  int32_t output_dtype;        /* fused output only */
  float softmax_scale;
} pa_fp8_partition_args;

int pa_fp8_decode_partition(const pa_fp8_partition_args* args, void* hip_stream);

/*
 * Log-sum-exp merge of the P slot partials into the final output.
 *
 * Replaces compile_pa_decode_sw_reduce(...)["launch"]
 * (kernels/pa_decode_swa.py:1132-1177; math at :954-1130), which both
 * partitioned routes of pa_decode_ps_launch call.  For each (sequence, kv
 * head, column): M = max_p m_p, w_p = s_p e^{m_p - M} / sum_q s_q e^{m_q - M},
 * out = sum_p w_p tmp_p (zero when every slot is empty).  The output is
 * addressed through the 5-D view [B, ql, Hkv, gqa, D].
 */
typedef struct pa_fp8_reduce_args {
  int32_t abi_version;
  void* output;
  const float* exp_sums;
  const float* max_logits;
  const void* tmp_out;
  int64_t stride_out_seq, stride_out_ql, stride_out_kv_head, stride_out_group;
  int64_t stride_es_seq, stride_es_head, stride_es_part;
  int64_t stride_to_seq, stride_to_head, stride_to_part, stride_to_group;
  int32_t num_seqs;
  int32_t num_kv_heads;
  int32_t num_partitions;
  int32_t query_length;
  int32_t query_group_size;
  int32_t head_size;
  int32_t output_dtype;
  int32_t tmp_dtype;
} pa_fp8_reduce_args;

int pa_fp8_decode_reduce(const pa_fp8_reduce_args* args, void* hip_stream);

/*
 * Per-wave streaming decode.  Every wave of the launch walks a list of
 * pieces -- (sequence, kv head, run of 32-token chunks) -- back to back
 * through one LDS pipeline, and writes each piece either straight into
 * `output` (the piece is the whole (sequence, kv head)) or as a float32
 * partial (normalised output row plus its log-sum-exp) for a merge pass.
 * Up to 16 query columns per kv head (query_length * gqa) every wave walks
 * its own pieces; 17..64 columns run cooperatively: a workgroup has one
 * wave per 16-column block, the waves share each chunk through LDS and the
 * workgroup walks the pieces (num_workers then counts workgroups).
 *
 * pa_fp8_decode_worklist: pieces come from the work list of
 * pa_fp8_plan_worklist, one workgroup per bin (num_workers = bins, the
 * reference's CU * 3): up to 16 columns its three waves split the bin's
 * chunks into equal runs and merge works cut between them in LDS; 17..64
 * columns the cooperative workgroup walks the bin's works.  Replaces
 * compile_pa_decode_metadata(...)["launch"] (kernels/pa_decode_fp8.py:
 * 1030-1721, launched at :3144-3184): a work with partial_qo_loc < 0 writes
 * output rows qo_start + qi; otherwise partial rows ploc + query_length + qi
 * of partial_output [rows, Hq, D] / partial_lse [rows, Hq], lse = max
 * logit + ln(sum), natural-log units.  Merge with pa_fp8_reduce_worklist.
 *
 * pa_fp8_decode_balanced: no work list; the kernel cuts the chunks of all
 * (sequence, kv head) pairs into num_workers equal runs itself (stream-K),
 * so ragged batches load every wave equally without a host round trip.
 * With up to 16 columns the runs are per wave and, when 4 (or 2) divides
 * both num_kv_heads and num_workers, cover groups of that many adjacent kv
 * heads walked by the waves of one workgroup in step.
 * Pairs a single wave holds whole go straight to `output`; then
 * pa_fp8_merge_balanced, on the same stream and with the same arguments
 * and workspace, merges the pieces of the pairs that were cut (and writes
 * zeros for pairs with no visible key).  The workspace
 * (pa_fp8_balanced_workspace_bytes bytes, 256-byte aligned) holds the
 * pieces' partials (pair descriptors, float32 lse, bf16 normalised rows:
 * internal to the call); it needs no initialisation.  num_seqs <= 1024.  No
 * reference counterpart: it serves the small-block and flat-page routes of
 * pa_decode_ps_launch when the caller does not ask for the slot partials.
 */
typedef struct pa_fp8_stream_args {
  int32_t abi_version;
  void* output; /* [B * ql, Hq, D] */
  const void* query;
  const void* key_cache;
  const void* value_cache;
  const int32_t* block_tables; /* [B, max_blocks], or the flat page list when kv_indptr != NULL */
  const int32_t* kv_indptr;    /* optional [B + 1] offsets into the flat page list */
  const int32_t* context_lengths;
  const float* key_scale;
  const float* value_scale;
  /* work list (pa_fp8_decode_worklist only) */
  const int32_t* work_indptr;      /* [num_workers + 1] */
  const int32_t* work_info;        /* [works, 8] */
  const int32_t* partition_indptr; /* [B + 1] cumulative 256-token partitions */
  float* partial_output;           /* [rows, Hq, D] float32 */
  float* partial_lse;              /* [rows, Hq] float32 */
  /* element strides */
  int64_t stride_q_tok, stride_q_head;
  int64_t stride_k_block, stride_k_head;
  int64_t stride_v_block, stride_v_head;
  int64_t stride_bt_seq;
  int64_t stride_ks_block, stride_ks_head;
  int64_t stride_out_tok, stride_out_head;
  int64_t stride_po_row, stride_pl_row; /* work list partial rows */
  /* sizes */
  int32_t num_seqs;
  int32_t num_kv_heads;
  int32_t query_length;
  int32_t query_group_size;
  int32_t head_size;
  int32_t block_size;
  int32_t num_blocks;
  int32_t max_blocks_per_seq;
  int32_t sliding_window;
  int32_t per_token_kv;
  int32_t trans_v;
  int32_t query_dtype;
  int32_t output_dtype;
  int32_t num_workers; /* balanced: runs (waves <= 16 columns, else workgroups); work list: bins */
  float softmax_scale;
} pa_fp8_stream_args;

int pa_fp8_decode_worklist(const pa_fp8_stream_args* args, void* hip_stream);
int pa_fp8_decode_balanced(const pa_fp8_stream_args* args, void* workspace, int64_t workspace_bytes,
                           void* hip_stream);
int pa_fp8_merge_balanced(const pa_fp8_stream_args* args, const void* workspace, int64_t workspace_bytes,
                          void* hip_stream);
int64_t pa_fp8_balanced_workspace_bytes(int num_seqs, int num_kv_heads, int query_length, int query_group_size,
                                        int num_workers);
/*
 * pa_fp8_decode_balanced_static: pa_fp8_decode_balanced followed by
 * pa_fp8_merge_balanced (same kernels, same results), with the workspace
 * taken from a static device array of the library instead of an argument,
 * so the call allocates nothing (no hipMalloc, no allocating library call).
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  The array holds pa_fp8_static_scratch_bytes() = 64 MiB per
 * device, for the life of the process; a call whose workspace
 * (pa_fp8_balanced_workspace_bytes) exceeds it returns PA_ERR_SCRATCH.
 * Every call on a device shares that device's array: calls that overlap on
 * one device (other streams, other host threads) race and must be
 * serialised by the caller.  The workspace needs no initialisation, so
 * nothing is cleared between calls.
 */
int pa_fp8_decode_balanced_static(const pa_fp8_stream_args* args, void* hip_stream);
int64_t pa_fp8_static_scratch_bytes(void);

/* Runs a streaming launch keeps resident on num_cu CUs: waves for up to 16
 * query columns (4 per workgroup; two workgroups per CU when their LDS
 * fits, else one), cooperative workgroups for 17..64 columns. */
int pa_fp8_stream_workers(int num_cu, int query_length, int query_group_size, int per_token_kv);

/*
 * Log-sum-exp merge of work-list partials.  Replaces aiter's pa_reduce_v1
 * as called at kernels/pa_decode_fp8.py:3189-3200: partial_output and
 * partial_lse point at row query_length of the buffers the decode wrote
 * (the reference passes partial_output[query_length:]).  Group g merges the
 * partial rows reduce_partial_map[reduce_indptr[g] .. reduce_indptr[g+1]) + qi
 * into output rows reduce_final_map[g][0] + qi, for qi <
 * reduce_final_map[g][1] - reduce_final_map[g][0] and every query head.
 */
typedef struct pa_fp8_worklist_reduce_args {
  int32_t abi_version;
  void* output;
  const float* partial_output;
  const float* partial_lse;
  const int32_t* reduce_indptr;      /* [num_groups + 1] */
  const int32_t* reduce_final_map;   /* [num_groups, 2] */
  const int32_t* reduce_partial_map;
  int64_t stride_out_tok, stride_out_head;
  int64_t stride_po_row, stride_pl_row;
  int32_t num_groups; /* entries of reduce_indptr minus one (the batch size) */
  int32_t num_query_heads;
  int32_t head_size;
  int32_t max_query_length;
  int32_t output_dtype;
} pa_fp8_worklist_reduce_args;

int pa_fp8_reduce_worklist(const pa_fp8_worklist_reduce_args* args, void* hip_stream);

/*
 * Host-only planning helpers (no GPU needed).
 *
 * pa_fp8_recommended_splits replaces get_recommended_splits
 * (kernels/pa_decode_fp8.py:1922-1949) with the CU count passed in;
 * pa_fp8_plan_slot returns the logical token range [*t0, *t1) that slot
 * `slot` reads (kernels/pa_decode_fp8.py:2311-2320 and
 * kernels/pa_decode_swa.py:1356-1368); pa_fp8_plan_visible returns the key
 * range query qi may attend (kernels/pa_decode_swa.py:1597-1620).
 */
int pa_fp8_recommended_splits(int num_seqs, int num_kv_heads, int split_kv_blocks, int sliding_window,
                              int partition_tokens, int query_length, int num_cu);
int pa_fp8_plan_slot(int context_length, int num_partitions, int slot, int sliding_window, int query_length,
                     int* t0, int* t1);
int pa_fp8_plan_visible(int context_length, int qi, int query_length, int sliding_window, int* lo, int* hi);

/*
 * Work list of the persistent route, on the host (host pointers in and
 * out).  Replaces get_pa_metadata_v1 (kernels/pa_metadata.py:450-524, the
 * scheduler kernel :145-420) and get_pa_metadata_info_v1 (:53-79) for
 * causal decode with uniform query length: the ceil(ctx / kv_granularity)
 * partitions of each sequence are dealt, per kv head, to num_cu /
 * num_kv_heads bins.  Buffers: work_indptr [num_cu + 1], work_info
 * [max_works * 8], reduce_indptr [num_seqs + 1], reduce_final_map
 * [num_seqs * 2], reduce_partial_map [max_split_tiles]; unused entries are
 * zeroed.  Returns the number of works (>= 0) or a PA_ERR_* code.
 */
int pa_fp8_worklist_sizes(int num_seqs, int num_kv_heads, int num_cu, int* max_works, int* max_split_tiles);
int pa_fp8_plan_worklist(const int32_t* context_lengths, int num_seqs, int num_kv_heads, int query_group_size,
                         int query_length, int num_cu, int kv_granularity, int32_t* work_indptr, int32_t* work_info,
                         int32_t* reduce_indptr, int32_t* reduce_final_map, int32_t* reduce_partial_map);

/*
 * KV-cache writer: NeoX RoPE on the new tokens' Q and K, K and V written into
 * the paged cache.  Replaces the launch function built by
 * build_fused_rope_cache_module (kernels/fused_rope_cache_kernel.py:49-512:
 * kernel :105-412, launch :460-512), which fuses the same three steps.
 *
 *   q, q_out          [T, QH, D]  bf16 or f16 (token / head strides)
 *   k, v, k_out       [T, KH, D]  same dtype
 *   positions, slot_mapping [T]   int32, or int64 read as their low words
 *                                 (index_i64 = 1); slot < 0 skips the cache
 *   cos_cache, sin_cache [max_pos, D / 2] (reuse_freqs_front_part = 1) or
 *                        [max_pos, D], same dtype as q (row strides)
 *   key_cache, value_cache, contiguous, by cache_layout:
 *     PA_CACHE_FLASH         K, V [NB, bs, KH, D]
 *     PA_CACHE_ATOM          K [NB, KH, D / 16, bs, 16], V [NB, KH, D, bs]
 *     PA_CACHE_ATOM_TRANS_V  K as ATOM, V [NB, KH, bs / 16, D, 16] (the
 *                            layout the decode kernels read fastest; no
 *                            counterpart in the reference writer)
 *     element: the input dtype, or fp8 e4m3fn when apply_scale = 1 (value *
 *     1 / k_scale[0] or 1 / v_scale[0], saturated at +-448)
 * D a multiple of 16 from 16 to 512 (D = 96, for one, runs 5 rows of 12
 * lanes per wave).
 */
enum pa_fp8_cache_layout {
  PA_CACHE_FLASH = 0,
  PA_CACHE_ATOM = 1,
  PA_CACHE_ATOM_TRANS_V = 2,
};

typedef struct {
  int32_t abi_version; /* = PA_FP8_ABI_VERSION */
  const void* q;
  const void* k;
  const void* v;
  const void* positions;
  const void* cos_cache;
  const void* sin_cache;
  const void* slot_mapping;
  void* key_cache;
  void* value_cache;
  void* q_out;
  void* k_out;
  const float* k_scale;
  const float* v_scale;
  int64_t stride_q_tok, stride_q_head;
  int64_t stride_k_tok, stride_k_head;
  int64_t stride_v_tok, stride_v_head;
  int64_t stride_qo_tok, stride_qo_head;
  int64_t stride_ko_tok, stride_ko_head;
  int64_t stride_cos_pos, stride_sin_pos;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t num_blocks;  /* slots past the cache are not written */
  int32_t max_pos;     /* rows of cos/sin; positions are clamped into them */
  int32_t dtype;       /* PA_DTYPE_BF16 / PA_DTYPE_F16 */
  int32_t cache_layout;
  int32_t apply_scale;
  int32_t reuse_freqs_front_part;
  int32_t index_i64;
} pa_fp8_rope_cache_args;

int pa_fp8_rope_cache(const pa_fp8_rope_cache_args* args, void* hip_stream);

/*
 * Fused per-token RMSNorm + GPT-J RoPE + optional fp8 quantisation of the
 * query heads and the single KV row of each token.  Replaces the launcher
 * compiled by compile_flydsl_qk_norm_rope_quant
 * (kernels/qk_norm_rope_quant.py:709-736; kernel :259-640, launch :650-686)
 * as flydsl_qk_norm_rope_quant (:739-955) calls it.
 *
 *   q          [T, H, D]  bf16, token stride stride_q_tok, heads dense
 *   kv         [T, D]     bf16, token stride stride_kv_tok
 *   q_weight   [D] bf16 or NULL (unweighted Q); kv_weight [D] bf16
 *   cos_cache, sin_cache [max_pos, RD / 2] bf16, contiguous
 *   positions  [T] int64, read as their low 32-bit words; outside
 *              [0, max_pos) the rotation reads zeros
 *   q_out [T, H, D], kv_out [T, D], dense: bf16, or fp8 e4m3fn when quant
 *   q_scale [T, H, NG], kv_scale [T, NG], NG = D / group_size: float32, or
 *              uint8 e8m0 exponents when scale_e8m0 (quant only)
 * Row statistic rstd = rsqrt(mean(x^2) + 1e-6) over the unweighted row; the
 * last RD elements are rotated in pairs (2k, 2k + 1) by cos/sin[pos, k].
 * D in {128, 256, 512}; RD even, a multiple of D / 64, at most D;
 * group_size a multiple of D / 64 dividing D, D / 64 lanes per group a
 * power of two.  T * (H + 1) < 2^31.
 */
typedef struct {
  int32_t abi_version; /* = PA_FP8_ABI_VERSION */
  const void* q;
  const void* kv;
  const void* q_weight;
  const void* kv_weight;
  const void* cos_cache;
  const void* sin_cache;
  const int64_t* positions;
  void* q_out;
  void* kv_out;
  void* q_scale;
  void* kv_scale;
  int64_t stride_q_tok;
  int64_t stride_kv_tok;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t head_dim;
  int32_t rope_head_dim;
  int32_t max_pos;
  int32_t quant;
  int32_t group_size;
  int32_t scale_e8m0;
} pa_qk_norm_rope_args;

int pa_fp8_qk_norm_rope_quant(const pa_qk_norm_rope_args* args, void* hip_stream);

/*
 * MLA (multi-head latent attention, DeepSeek-V3 shape) fp8 decode.
 * Replaces launch_mla_fwd_decode_m16x8_fp8_fp8
 * (kernels/mla_fwd_decode_m16x8_fp8_fp8.py:2069-2104; kernel :310-2066) as
 * flydsl_mla_fwd_decode (kernels/mla_fwd_decode.py:57-167) calls it.
 *
 *   query        [num_rows, 128, 576] fp8 e4m3fn, dense (576 = 512 latent
 *                + 64 rope dims)
 *   kv_buffer    [num_pages, 576] fp8 e4m3fn, dense: page size 1, one kv
 *                head; the value of a token is the first 512 bytes of its row
 *   kv_page_indices [num_page_indices] int32
 *   work_indptr  [num_workers + 1] int32: works of worker w are
 *                work_indptr[w] .. work_indptr[w+1]
 *   work_info    [num_works][8] int32: (batch, partial row or -1, query row,
 *                query row + 1, first position, end position in
 *                kv_page_indices, 0, heads)
 *   final_output [num_rows, 128, 512] bf16, written for partial row -1
 *   split_output [num_partial, 128, 512] float32 and split_lse
 *                [num_partial, 128] float32, written for partial rows >= 0:
 *                the normalised partial output and its log-sum-exp
 *                (natural log of the scaled logits)
 * Logits are softmax_scale * q.k over all 576 dims; p is rounded to fp8
 * for the value product (the reference's arithmetic), or split into two
 * fp8 terms when precise_p is non-zero.  Work fields and page indices out
 * of range are clamped into range (memory safety, not a result contract).
 * A work with an empty range writes zeros (and lse -inf).
 */
typedef struct {
  int32_t abi_version; /* = PA_FP8_ABI_VERSION */
  const void* query;
  const void* kv_buffer;
  const int32_t* kv_page_indices;
  const int32_t* work_indptr;
  const int32_t* work_info;
  void* final_output;
  float* split_output;
  float* split_lse;
  int64_t num_pages;
  int32_t num_page_indices;
  int32_t num_rows;
  int32_t num_workers;
  int32_t num_works;
  int32_t num_partial;
  float softmax_scale;
  int32_t precise_p;
} pa_mla_decode_args;

int pa_fp8_mla_decode(const pa_mla_decode_args* args, void* hip_stream);

/*
 * Log-sum-exp merge of the split MLA outputs (replaces aiter's
 * mla_reduce_v1, called at tests/kernels/test_mla_decode.py:356-365; not
 * part of the reference).  Group g (0 <= g < num_groups) merges, for each
 * query row r of reduce_final_map[g] = (row0, row1), the partial rows
 * reduce_partial_map[i] + (r - row0), i in reduce_indptr[g] ..
 * reduce_indptr[g+1]; empty groups are skipped.
 *   out = sum_i w_i o_i / sum_i w_i, w_i = exp(lse_i - max lse)
 * into final_output [num_rows, 128, 512] bf16 and, when not NULL,
 * final_lse [num_rows, 128] float32.  Rows and partial rows out of range
 * are skipped.
 */
typedef struct {
  int32_t abi_version; /* = PA_FP8_ABI_VERSION */
  const float* split_output;
  const float* split_lse;
  const int32_t* reduce_indptr;
  const int32_t* reduce_final_map;
  const int32_t* reduce_partial_map;
  void* final_output;
  float* final_lse;
  int32_t num_groups;
  int32_t num_partial;
  int32_t num_partial_map;
  int32_t num_rows;
} pa_mla_reduce_args;

int pa_fp8_mla_reduce(const pa_mla_reduce_args* args, void* hip_stream);

/*
 * Host planner of the MLA work list (our own; aiter's get_mla_metadata_v1,
 * tests/kernels/test_mla_decode.py:274-295, is not part of the reference):
 * 128-token blocks of every query row dealt to num_workers workers in
 * contiguous balanced runs.  qo_indptr, kv_indptr [num_seqs + 1] host int32.
 * Output buffers sized by pa_fp8_mla_plan_sizes (num_rows =
 * qo_indptr[num_seqs] - qo_indptr[0]); reduce_indptr [num_rows + 1],
 * reduce_final_map [num_rows][2].  Returns the number of works or a
 * PA_ERR_* code; *num_groups / *num_partials receive the reduce group and
 * partial row counts.
 */
int pa_fp8_mla_plan_sizes(int num_rows, int num_workers, int* max_works, int* max_partials);
int pa_fp8_mla_plan(const int32_t* qo_indptr, const int32_t* kv_indptr, int num_seqs, int num_workers,
                    int max_works, int max_partials, int32_t* work_indptr, int32_t* work_info,
                    int32_t* reduce_indptr, int32_t* reduce_final_map, int32_t* reduce_partial_map,
                    int* num_groups, int* num_partials);

/*
 * float8_e4m3fnuz rows to float8_e4m3fn by value, gathered.  No counterpart
 * in the reference (its gfx942 kernels read fnuz directly); it serves
 * flydsl_mla_fwd_decode's fnuz inputs (kernels/mla_fwd_decode.py:52-53) on
 * gfx950, whose matrix cores read e4m3fn only.  dst row i (row_bytes bytes)
 * = convert(src row rows[i]) for i < num_rows; rows == NULL means row i.
 * Row indices are clamped into [0, num_src_rows).  Conversion per byte:
 * magnitudes >= 2^-6 exactly (exponent - 1), smaller ones rounded to the
 * nearest multiple of 2^-9 (ties to even), fnuz NaN (0x80) -> e4m3fn NaN.
 * row_bytes must be a multiple of 16 and src/dst 16-byte aligned.
 */
int pa_fp8_fnuz_to_fn(const void* src, const int32_t* rows, int64_t num_rows, int64_t num_src_rows,
                      int64_t row_bytes, void* dst, void* hip_stream);

/*
 * Checked builds.  libpa_fp8_checked.so is built from the same sources with
 * -DPA_FP8_CHECKED.  Like the release library it clamps every index it reads
 * from caller data into range before using it as an address; it also
 * records each value it had to clamp as one of these bits (no trap, no
 * wait; the results are those of the release library):
 */
enum {
  PA_VIOLATION_PAGE = 1,     /* block_tables / kv_page_indices entry, or fnuz row index, outside the cache */
  PA_VIOLATION_WORK = 2,     /* MLA work record: query row, partial row or kv range outside its buffer */
  PA_VIOLATION_POSITION = 4, /* rope position outside [0, max_pos) */
  PA_VIOLATION_SLOT = 8      /* KV-cache slot past the last cache block */
};
/* ORs the bits recorded on the current device since the last call into
 * *bits and clears them (always 0 in a release build; each device keeps its
 * own bits).  Synchronises the current device; returns PA_OK or a HIP error
 * code.  No counterpart in the reference: a debug aid for callers chasing a
 * bad page table or slot mapping. */
int pa_fp8_debug_violations(unsigned int* bits);
/* 1 in a checked build, 0 in a release build. */
int pa_fp8_checked_build(void);

/* Library identification and error names. */
const char* pa_fp8_version(void);
const char* pa_fp8_error_string(int code);

#ifdef __cplusplus
}
#endif

#endif /* PA_FP8_H */
