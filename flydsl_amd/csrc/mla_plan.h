// Host-side work-list planner of the MLA decode (serial C, no device code).
//
// The reference kernel (kernels/mla_fwd_decode_m16x8_fp8_fp8.py:1616-1636)
// consumes aiter's MLA work list: work_indptr[num_workers + 1] and 8-dword
// work records whose dword 1 is the partial row (or -1), dword 2/3 the query
// row range and dwords 4/5 the range of positions in kv_page_indices.  The
// planner that fills them (aiter get_mla_metadata_v1) is not part of the
// reference, so this is a planner of our own that emits the same format:
//
//   * every query row r of sequence b attends the pages
//     kv_indptr[b] .. kv_indptr[b+1]; its cost is the number of 128-token
//     blocks (at least 1, so an empty row still gets a work that writes
//     zeros);
//   * the blocks of all rows, in row order, are dealt to the workers in
//     contiguous runs of `average` blocks (+1 for the first `remainder`
//     workers), cutting rows at worker boundaries;
//   * a row that stays whole is written straight to the final output
//     (partial row -1); a row cut into k pieces gets k consecutive partial
//     rows and one reduce group: reduce_indptr[g] .. reduce_indptr[g+1]
//     index reduce_partial_map (the partial rows), reduce_final_map[g] =
//     (row, row + 1).
//
// Unused reduce groups are empty (reduce_indptr repeats its last value) and
// unused entries are zero, so a reduce launched over every group slot is
// correct without knowing the group count.
#pragma once

#include <stdint.h>
#include <string.h>

#define MLA_PLAN_BLOCK 128

static inline void mla_plan_sizes(int num_rows, int num_workers, int* max_works, int* max_partials) {
  // Each worker boundary inside a row adds one piece; every cut row has at
  // least two pieces and at most (boundaries inside it) + 1.
  const long w = (long)num_rows + (num_workers > 0 ? num_workers - 1 : 0);
  const long p = 2L * (num_workers > 0 ? num_workers - 1 : 0);
  *max_works = (int)(w < 0x7fffffffL ? w : 0x7fffffffL);
  *max_partials = (int)(w < p ? w : p);
}

// Returns the number of works, or -1 when the inputs are inconsistent
// (decreasing indptr) or a buffer would overflow (not possible with buffers
// sized by mla_plan_sizes()).
static inline int mla_plan(const int32_t* qo_indptr, const int32_t* kv_indptr, int num_seqs, int num_workers,
                           int max_works, int max_partials, int32_t* work_indptr, int32_t* work_info,
                           int32_t* reduce_indptr, int32_t* reduce_final_map, int32_t* reduce_partial_map,
                           int* num_groups_out, int* num_partials_out) {
  if (num_seqs < 0 || num_workers <= 0) return -1;
  const int num_rows = qo_indptr[num_seqs] - qo_indptr[0];
  if (num_rows < 0) return -1;
  memset(work_indptr, 0, sizeof(int32_t) * (size_t)(num_workers + 1));
  if (max_works > 0) memset(work_info, 0, sizeof(int32_t) * 8 * (size_t)max_works);
  memset(reduce_indptr, 0, sizeof(int32_t) * (size_t)(num_rows + 1));
  if (num_rows > 0) memset(reduce_final_map, 0, sizeof(int32_t) * 2 * (size_t)num_rows);
  if (max_partials > 0) memset(reduce_partial_map, 0, sizeof(int32_t) * (size_t)max_partials);
  *num_groups_out = 0;
  *num_partials_out = 0;

  int64_t total = 0;
  for (int b = 0; b < num_seqs; ++b) {
    const int rows = qo_indptr[b + 1] - qo_indptr[b];
    const int len = kv_indptr[b + 1] - kv_indptr[b];
    if (rows < 0 || len < 0) return -1;
    const int64_t cost = len > 0 ? (len + MLA_PLAN_BLOCK - 1) / MLA_PLAN_BLOCK : 1;
    total += cost * rows;
  }
  const int64_t average = total / num_workers;
  const int64_t remainder = total % num_workers;

  int worker = 0, works = 0, groups = 0, partials = 0;
  int64_t left = average + (0 < remainder ? 1 : 0);  // blocks the current worker still takes
  for (int b = 0; b < num_seqs; ++b) {
    const int len = kv_indptr[b + 1] - kv_indptr[b];
    const int64_t cost = len > 0 ? (len + MLA_PLAN_BLOCK - 1) / MLA_PLAN_BLOCK : 1;
    for (int row = qo_indptr[b]; row < qo_indptr[b + 1]; ++row) {
      int64_t done = 0;
      const int first = works;
      while (done < cost) {
        while (left <= 0 && worker + 1 < num_workers) {
          work_indptr[worker + 1] = works;
          ++worker;
          left = average + (worker < remainder ? 1 : 0);
        }
        int64_t take = cost - done;
        if (worker + 1 < num_workers && take > left) take = left;  // the last worker takes the rest
        if (works >= max_works) return -1;
        int32_t* w = work_info + 8 * (size_t)works;
        const int64_t t0 = done * MLA_PLAN_BLOCK;
        int64_t t1 = (done + take) * MLA_PLAN_BLOCK;
        if (t1 > len) t1 = len;
        w[0] = b;
        w[1] = -1;
        w[2] = row;
        w[3] = row + 1;
        w[4] = kv_indptr[b] + (int32_t)t0;
        w[5] = kv_indptr[b] + (int32_t)t1;
        w[6] = 0;
        w[7] = (int32_t)(128u << 16);  // query heads [0, 128)
        ++works;
        done += take;
        left -= take;
      }
      const int pieces = works - first;
      if (pieces > 1) {
        if (partials + pieces > max_partials) return -1;
        for (int i = 0; i < pieces; ++i) {
          work_info[8 * (size_t)(first + i) + 1] = partials + i;
          reduce_partial_map[partials + i] = partials + i;
        }
        reduce_final_map[2 * groups] = row;
        reduce_final_map[2 * groups + 1] = row + 1;
        partials += pieces;
        reduce_indptr[groups + 1] = partials;
        ++groups;
      }
    }
  }
  for (int c = worker + 1; c <= num_workers; ++c) work_indptr[c] = works;
  for (int g = groups + 1; g <= num_rows; ++g) reduce_indptr[g] = partials;
  *num_groups_out = groups;
  *num_partials_out = partials;
  return works;
}
