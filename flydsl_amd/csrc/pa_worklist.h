// Host-side work-list planner of the persistent decode route.
//
// Restates the CU-major greedy scheduler of kernels/pa_metadata.py:145-420
// (the reference's single-wave port of aiter's get_pa_metadata_v1) as plain
// serial C: per kv head, the cumulative 256-token partitions of every
// sequence are dealt to `num_cu / num_kv_heads` bins in order, each bin
// taking `average` partitions (+1 for the first `remainder` bins).  A
// sequence cut across bins produces one partial work per bin piece and one
// reduce group.  Output formats are the reference's:
//
//   work_indptr [num_cu + 1]             works of bin c: [work_indptr[c], work_indptr[c+1])
//   work_info   [max_works][8]           batch, partial_qo_loc (-1: direct), qo_start, qo_end,
//                                        kv_start, kv_end (cumulative partitions), 0,
//                                        (qhead_end << 16) | qhead_start
//   reduce_indptr [B + 1]                partials of group g: [reduce_indptr[g], reduce_indptr[g+1])
//   reduce_final_map [B][2]              output rows (qo_start, qo_end) of group g
//   reduce_partial_map [max_split_tiles] partial row of each piece
//
// The reference writes the reduce maps once per kv head (its structure is
// the same for every head) and leaves unused entries uninitialised; here
// unused entries are zero.
#pragma once

#include <stdint.h>
#include <string.h>

static inline void pa_worklist_sizes(int num_seqs, int num_kv_heads, int num_cu, int* max_works,
                                     int* max_split_tiles) {
  // kernels/pa_metadata.py:53-79
  *max_works = (num_seqs + num_cu - 1) * num_kv_heads;
  const int a = num_seqs + num_cu - 1, b = (num_cu - 1) * 2;
  *max_split_tiles = a < b ? a : b;
}

// Returns the number of works, or -1 when a buffer would overflow (cannot
// happen with buffers sized by pa_worklist_sizes()).
static inline int pa_worklist_plan(const int32_t* ctx, int B, int Hkv, int gqa, int ql, int num_cu, int gran,
                                   int32_t* work_indptr, int32_t* work_info, int32_t* reduce_indptr,
                                   int32_t* reduce_final_map, int32_t* reduce_partial_map) {
  int max_works, max_split;
  pa_worklist_sizes(B, Hkv, num_cu, &max_works, &max_split);
  memset(work_indptr, 0, sizeof(int32_t) * (size_t)(num_cu + 1));
  if (max_works > 0) memset(work_info, 0, sizeof(int32_t) * 8 * (size_t)max_works);
  memset(reduce_indptr, 0, sizeof(int32_t) * (size_t)(B + 1));
  if (B > 0) memset(reduce_final_map, 0, sizeof(int32_t) * 2 * (size_t)B);
  if (max_split > 0) memset(reduce_partial_map, 0, sizeof(int32_t) * (size_t)max_split);
  if (B == 0) return 0;

  const int nspk = num_cu / Hkv;  // bins per kv head
#define PA_NPART(b) (((ctx[(b)] < 0 ? 0 : ctx[(b)]) + gran - 1) / gran)
  int64_t sum_blocks = 0;
  for (int b = 0; b < B; ++b) sum_blocks += PA_NPART(b);
  const int average = (int)(sum_blocks / nspk);
  const int reminder = (int)(sum_blocks % nspk);
#define PA_REMAIN(c) (average + (((c) % nspk) < reminder ? 1 : 0))

  int cid = 0, num_works = 0, lri = 0, grt = 0;
  for (int kh = 0; kh < Hkv; ++kh) {
    const int32_t qhr = (int32_t)((((uint32_t)((kh + 1) * gqa)) << 16) | ((uint32_t)(kh * gqa) & 0xffffu));
    int batch = 0, kvblk = 0, nsplit = 0, pidx = 0, kvbeg = 0;
    int kvend = PA_NPART(0);
    int remain = PA_REMAIN(cid);
    lri = 0;
    grt = 0;
    while (cid < num_cu && batch < B) {
      const int remain_kv = (kvend - kvbeg) - kvblk;
      const bool finish = remain >= remain_kv;
      const int qo_start = batch * ql, qo_end = (batch + 1) * ql;
      const int kv_start = kvbeg + kvblk;
      const bool emit = finish || remain > 0;
      if (emit) {
        if (num_works >= max_works) return -1;
        int32_t* w = work_info + 8 * (size_t)num_works;
        w[0] = batch;
        w[1] = finish ? (nsplit > 0 ? pidx : -1) : pidx;
        w[2] = qo_start;
        w[3] = qo_end;
        w[4] = kv_start;
        w[5] = finish ? kvend : (kv_start + remain < kvend ? kv_start + remain : kvend);
        w[6] = 0;
        w[7] = qhr;
      }
      if (finish && nsplit > 0) {
        // This bin closes a sequence cut into nsplit + 1 pieces: one group.
        const int n = nsplit + 1;
        if (lri + n > max_split || grt >= B) return -1;
        reduce_indptr[grt + 1] = lri + n;
        reduce_final_map[2 * grt] = qo_start;
        reduce_final_map[2 * grt + 1] = qo_end;
        for (int s = 0; s < n; ++s) reduce_partial_map[lri + s] = pidx - (nsplit - s) * ql;
        lri += n;
        grt += 1;
      }
      const int cid_now = cid;
      if (finish) {
        if (nsplit > 0) pidx += ql;
        num_works += 1;
        remain -= remain_kv;
        batch += 1;
        kvbeg = kvend;
        kvend += batch < B ? PA_NPART(batch) : 0;
        kvblk = 0;
        nsplit = 0;
      } else {
        if (remain > 0) {
          num_works += 1;
          pidx += ql;
          kvblk += remain;
          nsplit += 1;
        }
        cid += 1;
        remain = PA_REMAIN(cid);
      }
      work_indptr[cid_now + 1] = num_works;
    }
    if (cid < num_cu) cid += 1;
  }
  for (int i = cid; i <= num_cu; ++i) work_indptr[i] = num_works;
  for (int i = grt; i <= B; ++i) reduce_indptr[i] = lri;
#undef PA_NPART
#undef PA_REMAIN
  return num_works;
}
