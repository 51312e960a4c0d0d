// Integer planning of the split-context FP8 paged decode, shared by the host
// entry points and the device kernels so both index the same way.
//
//   pa_plan_splits        kernels/pa_decode_fp8.py:1922-1949
//   pa_plan_slot_tokens   kernels/pa_decode_fp8.py:2311-2320 (slot = run of
//                         256-token sub-partitions) and
//                         kernels/pa_decode_swa.py:1356-1368 (window route:
//                         slot = one 256-token tile of the logical sequence,
//                         for any page size; a single slot walks all visible
//                         tiles, as the fused window kernel does)
//   pa_plan_visible       kernels/pa_decode_swa.py:1597-1620 masks
#pragma once

#ifdef __HIPCC__
#define PA_HD __host__ __device__ __forceinline__
#else
#define PA_HD static inline
#endif

#define PA_PARTITION_TOKENS 256

PA_HD int pa_cdiv(int a, int b) { return (a + b - 1) / b; }
PA_HD int pa_min(int a, int b) { return a < b ? a : b; }
PA_HD int pa_max(int a, int b) { return a > b ? a : b; }

// Slots per (sequence, kv head).  Window: tiles covering W + ql - 1 tokens
// at any alignment.  Otherwise two workgroups per CU over B*Hkv*s units,
// rounded up to a multiple of s (pages per 256-token partition), in [4, 8].
PA_HD int pa_plan_splits(int num_seqs, int num_kv_heads, int split_kv_blocks, int sliding_window,
                         int partition_tokens, int query_length, int num_cu) {
  if (sliding_window > 0) return pa_cdiv(sliding_window + query_length - 1, partition_tokens) + 1;
  int target = num_cu * 2;
  long long d = (long long)num_seqs * num_kv_heads * split_kv_blocks;
  int denom = d < 1 ? 1 : (d > 0x7fffffff ? 0x7fffffff : (int)d);
  int n = pa_cdiv(target, denom) * split_kv_blocks;
  return pa_max(4, pa_min(n, 8));
}

// Logical token range [*t0, *t1) that slot `slot` of a sequence reads.
PA_HD void pa_plan_slot_tokens(int ctx, int num_slots, int slot, int sliding_window, int query_length,
                               int* t0, int* t1) {
  int nt = pa_cdiv(ctx, PA_PARTITION_TOKENS);
  if (sliding_window > 0) {
    int start = pa_max(ctx - query_length - sliding_window, 0);
    int tile = start / PA_PARTITION_TOKENS + slot;
    if (tile >= nt) { *t0 = 0; *t1 = 0; return; }
    if (num_slots == 1) {  // fused: one workgroup walks every visible tile
      *t0 = tile * PA_PARTITION_TOKENS;
      *t1 = ctx;
      return;
    }
    *t0 = tile * PA_PARTITION_TOKENS;
    *t1 = pa_min((tile + 1) * PA_PARTITION_TOKENS, ctx);
    return;
  }
  int pps = nt > 0 ? pa_cdiv(nt, num_slots) : 0;
  int first = slot * pps;
  int end = pa_min((slot + 1) * pps, nt);
  if (end <= first) { *t0 = 0; *t1 = 0; return; }
  *t0 = first * PA_PARTITION_TOKENS;
  *t1 = pa_min(end * PA_PARTITION_TOKENS, ctx);
}

// Keys that query qi (0-based among the ql new tokens) may attend: the query
// sits at ctx - ql + qi; causal keeps keys up to it, a window W the W + 1
// most recent of those.
PA_HD void pa_plan_visible(int ctx, int qi, int query_length, int sliding_window, int* lo, int* hi) {
  int h = ctx - query_length + 1 + qi;
  int l = sliding_window > 0 ? ctx - query_length - sliding_window + qi : 0;
  h = pa_min(h, ctx);
  *lo = pa_max(l, 0);
  *hi = pa_max(h, 0);
}

// 32-token chunks a sequence attends, counted from its first visible token
// rounded down to a multiple of 32 (the union of every query's keys).
#define PA_CHUNK_TOKENS 32
PA_HD int pa_plan_seq_chunks(int ctx, int query_length, int sliding_window) {
  int lo, hi, unused;
  pa_plan_visible(ctx, 0, query_length, sliding_window, &lo, &unused);
  pa_plan_visible(ctx, query_length - 1, query_length, sliding_window, &unused, &hi);
  if (hi <= lo) return 0;
  return pa_cdiv(hi - (lo & ~(PA_CHUNK_TOKENS - 1)), PA_CHUNK_TOKENS);
}

// Balanced split: the T chunks of all (sequence, kv head) segments, laid
// end to end, are cut into nw runs; run w is [floor(w T / nw),
// floor((w + 1) T / nw)).  Returns the run holding chunk g (0 <= g < T).
PA_HD int pa_plan_run_of_chunk(long long g, long long T, int nw) {
  return (int)(((g + 1) * nw + T - 1) / T) - 1;
}
PA_HD long long pa_plan_run_begin(int w, long long T, int nw) { return (long long)w * T / nw; }
