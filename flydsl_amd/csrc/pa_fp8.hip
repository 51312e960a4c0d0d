// FP8 paged-attention decode for MI355X (gfx950): split-context partition
// kernel, log-sum-exp reduce kernel and the C ABI declared in pa_fp8.h.
//
// Work decomposition.  One 256-thread workgroup per (sequence, kv head,
// slot); the slot's token range comes from pa_plan.h, so the partial
// outputs land in the same [B, Hkv, P, ql*gqa] cells as the reference's
// partition kernel (kernels/pa_decode_fp8.py:2127-2320).  Inside the slot,
// the four waves deal 32-token chunks round robin.  Each wave streams its
// chunks through a private LDS ring with gfx950 direct-to-LDS 16-byte loads
// (global_load_lds_dwordx4): the loads of the next chunk are in flight
// while the current one is computed, and no VGPRs hold data in flight.
//
// Arithmetic.  QK^T and PV run on v_mfma_f32_16x16x32_fp8_fp8.  The A
// operand is the fp8 cache itself (keys: 16 tokens x 32 head dims; values:
// 16 head dims x 32 tokens); the B operand is a 16-column block of query
// columns (e = qi * gqa + g).  Queries and probabilities are split into a
// high and a low fp8 term (x = hi + lo, both e4m3fn) and both terms go
// through the MFMA into one fp32 accumulator, which keeps ~8 significant
// bits -- the accuracy of bf16 -- while the cache is consumed in fp8
// without conversion.  Softmax runs in base 2 with the softmax scale,
// log2(e), the query scale and per-tensor key scale folded into one column
// factor; per-token key scales multiply the logits, per-token value scales
// fold into the probabilities (normalised by the running maximum of the
// value scales, so the fp8 range is used in full).
//
// Operand layouts of v_mfma_f32_16x16x32_fp8_fp8 (lane l, grp = l / 16,
// c = l % 16): A row c, k = 8*grp .. 8*grp+7; B column c, same k; result
// rows 4*grp .. 4*grp+3 of column c.  The k order of QK is a permutation
// of the head dimension shared by K and Q; the 32 tokens of a chunk are
// ordered so that the QK result a lane holds (rows 4*grp+i of two 16-row
// tiles) is exactly the 8 tokens 8*grp .. 8*grp+7 that the same lane must
// supply as the PV B operand.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "pa_fp8.h"
#include "pa_plan.h"
#include "pa_worklist.h"
#include "pa_check.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))

// LDS ring depth per wave (chunks); each stage holds one chunk's K and V.
#ifndef PA_FP8_STAGES
#define PA_FP8_STAGES 2
#endif
constexpr int kStages = PA_FP8_STAGES;
// Waves per workgroup (each streams its own chunks of the slot).
#ifndef PA_FP8_WAVES
#define PA_FP8_WAVES 4
#endif
constexpr int kWaves = PA_FP8_WAVES;
// Waves per workgroup of the per-wave streaming decode with one query image
// of up to 4 columns per wave (larger images: 4 waves, for LDS).
#ifndef PA_FP8_STREAM_WAVES
#define PA_FP8_STREAM_WAVES 4
#endif
__host__ __device__ constexpr int stream_waves(int nq) { return nq == 1 ? PA_FP8_STREAM_WAVES : 4; }
// Query images (of 4 columns) per wave of the streaming decode for eq columns.
__host__ __device__ constexpr int stream_nq(int eq) { return eq <= 4 ? 1 : (eq <= 8 ? 2 : 4); }
constexpr int kHead = 128;
constexpr int kChunk = 32;                  // tokens per wave step
// Key image of one chunk in LDS: two 16-token halves, each [8 dim chunks]
// [16 tokens][16 B]; the second half sits 64 B past a 2 KiB boundary so the
// two halves map to different LDS banks.
constexpr int kKHalf = 2048 + 64;
constexpr int kKBytes = 2 * kKHalf;         // fp8 keys of one chunk (+ pad)
constexpr int kVBytes = kChunk * kHead;     // fp8 values of one chunk
constexpr int kScaleBytes = 2 * kChunk * 4; // per-token K and V scales
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h;
  uint16_t s = (uint16_t)bits16;
  __builtin_memcpy(&h, &s, 2);
  return (float)h;
}

// Round to nearest even; inputs here are finite.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  uint16_t s;
  __builtin_memcpy(&s, &h, 2);
  return s;
}

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

// Four floats -> four e4m3fn bytes (round to nearest even).
__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

// pack4_fp8 without the zeroing move: the first conversion writes the low
// half of a fresh register whose old high half the second one overwrites.
// The statement is outside the compiler's hazard tracking, so a and b must
// not come straight from a transcendental instruction (which needs a wait
// state before another VALU reads its result).
__device__ __forceinline__ uint32_t pack4_fp8_fresh(float a, float b, float c, float d) {
  int r;
  asm("v_cvt_pk_fp8_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

// x[0..7] -> (hi, lo) with x ~= hi + lo, both packed e4m3fn, byte i = x[i].
// kFresh: x was not written by a transcendental instruction directly (the
// residuals never are), so the high part packs without zeroing moves too.
template <bool kFresh = false>
__device__ __forceinline__ void split8_fp8(const float* x, long& hi, long& lo) {
  uint32_t h0, h1;
  if constexpr (kFresh) {
    h0 = pack4_fp8_fresh(x[0], x[1], x[2], x[3]);
    h1 = pack4_fp8_fresh(x[4], x[5], x[6], x[7]);
  } else {
    h0 = pack4_fp8(x[0], x[1], x[2], x[3]);
    h1 = pack4_fp8(x[4], x[5], x[6], x[7]);
  }
  f32x2 b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, false);
  f32x2 b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, true);
  f32x2 b2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, false);
  f32x2 b3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, true);
  uint32_t l0 = pack4_fp8_fresh(x[0] - b0[0], x[1] - b0[1], x[2] - b1[0], x[3] - b1[1]);
  uint32_t l1 = pack4_fp8_fresh(x[4] - b2[0], x[5] - b2[1], x[6] - b3[0], x[7] - b3[1]);
  hi = (long)((uint64_t)h0 | ((uint64_t)h1 << 32));
  lo = (long)((uint64_t)l0 | ((uint64_t)l1 << 32));
}

// Wait states between an MFMA that an inline statement issued (the
// compiler's hazard tracking does not see it) and the next VALU access of
// its result: 20, more than the longest MFMA used here needs.
#define PA_MFMA_DRAIN "s_nop 7\n\ts_nop 7\n\ts_nop 3\n\t"

// acc *= f in place (tied operands): a conditional rescale then keeps the
// accumulators in their registers on both paths (no copies on the path
// that skips it).  Its input may come from mfma_k128_pair, whose MFMAs it
// waits out first (mfma_drain).
__device__ __forceinline__ void mfma_drain(f32x4 (&acc)[8]);
__device__ __forceinline__ void scale_inplace(f32x4 (&acc)[8], float f) {
  mfma_drain(acc);
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(acc[j][i]) : "v"(f));
}

__device__ __forceinline__ f32x4 mfma_fp8(long a, long b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

// acc += A B0, then acc += A B1 (v_mfma_f32_16x16x128_f8f6f4, fp8 e4m3fn
// operands), the accumulator tied in place (the accumulate chain needs no
// moves).  The compiler does not see inside the statement, so the hazards
// it would cover are covered here: s_nop 1 gives the two wait states a
// VALU write of an operand needs before an MFMA reads it; the second
// product reads the first's result as srcC with the same registers and
// opcode (no wait).  Any other access of acc first waits out the MFMA
// (mfma_drain, scale_inplace).  Not volatile: the operands order it, and
// the next tile's LDS reads may then be scheduled ahead of it.
__device__ __forceinline__ void mfma_k128_pair(f32x4& acc, const i32x8& a, const i32x8& b0, const i32x8& b1) {
  asm(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0\n\t"
      "v_mfma_f32_16x16x128_f8f6f4 %0, %1, %3, %0"
      : "+v"(acc)
      : "v"(a), "v"(b0), "v"(b1));
}

// Waits out mfma_k128_pair before acc is read or written by anything else;
// the tied operands keep every later access of acc after it.
__device__ __forceinline__ void mfma_drain(f32x4 (&acc)[8]) {
  asm volatile(PA_MFMA_DRAIN
               : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]), "+v"(acc[6]),
                 "+v"(acc[7]));
}

// v_mfma_f32_16x16x128_f8f6f4 with both operands e4m3fn and unit scales:
// lane l holds 32 k-values of row (A) / column (B) l % 16.
__device__ __forceinline__ f32x4 mfma_fp8_k128(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Reductions over the four lanes l, l^16, l^32, l^48 (one query column
// across the four 16-lane groups) with gfx950 permlane swaps (VALU only).
__device__ __forceinline__ float max_over_groups(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_over_groups(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 16 bytes per lane from global memory straight into LDS (lane l fills
// bytes 16l .. 16l+15 of ldst).  KV-cache pages are read once per decode
// step: the loads carry the non-temporal hint (nt), which streams them past
// the caches -- about 15% more HBM throughput for random 2 KiB pages on
// MI355X than loads with the default policy.
__device__ __forceinline__ void lds_dma16(const void* gsrc, LDS_AS void* ldst) {
  __builtin_amdgcn_global_load_lds(gsrc, ldst, 16, 0, 2);
}
// Default cache policy: query rows, which several workgroups of one launch
// may read, and per-token scales (at page size 16 a page-head's 64 bytes of
// scales share a 128-byte line with the next kv head's, which another wave
// reads; cached loads let that read hit).
__device__ __forceinline__ void lds_dma16_cached(const void* gsrc, LDS_AS void* ldst) {
  __builtin_amdgcn_global_load_lds(gsrc, ldst, 16, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= n only:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt and lgkmcnt at
// their maxima (7 and 15) so they are not waited on.
constexpr int vmcnt_only(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

// Store 8 head dims of the final output row (sequence b, query column e of
// kv head h) in the output dtype.
__device__ __forceinline__ void store_output8(const pa_fp8_partition_args& a, int b, int h, int e, int d0,
                                              const float* v) {
  const int gqa = a.query_group_size;
  const int qi = e / gqa, g = e - qi * gqa;
  const int64_t off = (int64_t)(b * a.query_length + qi) * a.stride_out_tok + (int64_t)(h * gqa + g) * a.stride_out_head + d0;
  if (a.output_dtype == PA_DTYPE_F32) {
    f32x4* p = (f32x4*)((float*)a.output + off);
    p[0] = f32x4{v[0], v[1], v[2], v[3]};
    p[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    const bool bf = a.output_dtype == PA_DTYPE_BF16;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo16 = bf ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
      const uint32_t hi16 = bf ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
      w[i] = lo16 | (hi16 << 16);
    }
    *(i32x4*)((uint16_t*)a.output + off) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

// Write one slot's outputs for query column e (8 head dims per thread call).
__device__ __forceinline__ void store_partial8(const pa_fp8_partition_args& a, int b, int h, int slot, int e,
                                               int d0, const float* v) {
  const int64_t off = (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head +
                      (int64_t)slot * a.stride_to_part + (int64_t)e * a.stride_to_group + d0;
  if (a.tmp_dtype == PA_DTYPE_F32) {
    float* p = (float*)a.tmp_out + off;
    ((f32x4*)p)[0] = f32x4{v[0], v[1], v[2], v[3]};
    ((f32x4*)p)[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_bf16_bits(v[2 * i]) | (f32_to_bf16_bits(v[2 * i + 1]) << 16);
    *(i32x4*)((uint16_t*)a.tmp_out + off) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

// 4 consecutive head dims (d0 multiple of 4) of a slot partial row.
__device__ __forceinline__ void store_partial4(const pa_fp8_partition_args& a, int b, int h, int slot, int e,
                                               int d0, f32x4 v) {
  const int64_t off = (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head +
                      (int64_t)slot * a.stride_to_part + (int64_t)e * a.stride_to_group + d0;
  if (a.tmp_dtype == PA_DTYPE_F32) {
    *(f32x4*)((float*)a.tmp_out + off) = v;
  } else {
    const uint32_t w0 = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
    const uint32_t w1 = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
    *(i32x2*)((uint16_t*)a.tmp_out + off) = i32x2{(int)w0, (int)w1};
  }
}

__device__ __forceinline__ void store_stats(const pa_fp8_partition_args& a, int b, int h, int slot, int e,
                                            float exp_sum, float max_logit) {
  const int64_t off = (int64_t)b * a.stride_es_seq + (int64_t)h * a.stride_es_head +
                      (int64_t)slot * a.stride_es_part + e;
  a.exp_sums[off] = exp_sum;
  a.max_logits[off] = max_logit;
}

// Online-softmax state of one wave over NCG 16-column query blocks: base-2
// running maximum m2, lane-partial sum lsum of 256 * 2^(l - m2), and the PV
// accumulator (acc[cg][j][i] = head dim 16j + 4*grp + i of column c16);
// vsmax is the running maximum of the per-token value scales.
template <int NCG>
struct WaveState {
  float m2[NCG];
  float lsum[NCG];
  f32x4 acc[NCG][8];
  float vsmax;
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      m2[cg] = kNegInf;
      lsum[cg] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[cg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    vsmax = 0.0f;
  }
};

// Query columns of one (sequence, kv head) as MFMA B operands, with the
// keys each column may see.  lo_all/hi_all bound the union of the columns'
// visible ranges, lo_max/hi_min their intersection (no masking needed).
template <int NCG>
struct QueryTile {
  i32x8 hi[NCG], lo[NCG];
  float fac[NCG];  // base-2 logit factor per column
  int vis_lo[NCG], vis_hi[NCG];
  int lo_all, hi_all, lo_max, hi_min;
};

// Raw query rows (bf16 or f16 bits) -> fp8 hi + lo B operands.  Lane
// (grp, c16) holds, for column col0 + cg * 16 + c16, the 32 head dims of
// 16-dim chunks grp and grp + 4 in qraw[cg][0..3] (8 dims each).  The column
// is scaled by a power of two putting its amax into [128, 256), which is
// exact.  The column's query index sets its causal / window bounds.
template <int NCG>
__device__ __forceinline__ void prepare_query(QueryTile<NCG>& q, const i32x4 (&qraw)[NCG][4], int query_dtype,
                                              float logit_scale, int ctx, int ql, int gqa, int W, int c16,
                                              int col0 = 0) {
  const int eq = ql * gqa;
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    const int e = col0 + cg * 16 + c16;
    const bool valid = e < eq;
    const int qi = valid ? e / gqa : 0;
    float v[32];
    if (query_dtype == PA_DTYPE_F16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t w = (uint32_t)qraw[cg][i >> 2][i & 3];
        v[2 * i] = f16_bits_to_f32(w & 0xffffu);
        v[2 * i + 1] = f16_bits_to_f32(w >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t w = (uint32_t)qraw[cg][i >> 2][i & 3];
        v[2 * i] = bf16_bits_to_f32(w & 0xffffu);
        v[2 * i + 1] = bf16_bits_to_f32(w >> 16);
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = max_over_groups(amax);
    int sexp = 261 - (int)((__float_as_uint(amax) >> 23) & 0xffu);
    sexp = sexp < 1 ? 1 : (sexp > 254 ? 254 : sexp);
    // The logit factor's sign (a launch constant: softmax scale times the
    // per-tensor key scale) goes into the query, so the column factor is
    // positive and the softmax takes its maxima on raw logits.
    const float sq0 = amax > 0.0f ? __uint_as_float((uint32_t)sexp << 23) : 1.0f;
    const float sq = logit_scale < 0.0f ? -sq0 : sq0;
#pragma unroll
    for (int sI = 0; sI < 4; ++sI) {
      float xs[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xs[i] = v[8 * sI + i] * sq;
      long hi, lo;
      split8_fp8(xs, hi, lo);
      q.hi[cg][2 * sI] = (int)(uint32_t)hi;
      q.hi[cg][2 * sI + 1] = (int)(uint32_t)((uint64_t)hi >> 32);
      q.lo[cg][2 * sI] = (int)(uint32_t)lo;
      q.lo[cg][2 * sI + 1] = (int)(uint32_t)((uint64_t)lo >> 32);
    }
    // > 0; a zero scale gives a tiny factor (all logits ~0, masked -inf
    // stays -inf rather than 0 * -inf)
    q.fac[cg] = fmaxf(logit_scale / sq, 1e-30f);
    int lo = 0, hi = 0;
    if (valid) pa_plan_visible(ctx, qi, ql, W, &lo, &hi);
    q.vis_lo[cg] = lo;
    q.vis_hi[cg] = hi;
  }
  // lo and hi grow with qi: the extremes come from the first and last query.
  // They are wave-uniform (readfirstlane states it), so the per-chunk
  // interior / edge tests are scalar compares and scalar branches.
  int lo_all, hi_min, lo_max, hi_all;
  pa_plan_visible(ctx, 0, ql, W, &lo_all, &hi_min);
  pa_plan_visible(ctx, ql - 1, ql, W, &lo_max, &hi_all);
  q.lo_all = __builtin_amdgcn_readfirstlane(lo_all);
  q.hi_min = __builtin_amdgcn_readfirstlane(hi_min);
  q.lo_max = __builtin_amdgcn_readfirstlane(lo_max);
  q.hi_all = __builtin_amdgcn_readfirstlane(hi_all);
}

// QK^T of one chunk: raw logits of the lane's 8 tokens (two 16-token
// tiles) for each column block, Q's hi and lo terms accumulated.
template <int NCG>
__device__ __forceinline__ void chunk_logits(const QueryTile<NCG>& q, const LDS_AS unsigned char* sk, int krow,
                                             int grp, f32x4 (&la)[NCG], f32x4 (&lb)[NCG]) {
  const i32x4 ka0 = *(const LDS_AS i32x4*)(sk + krow + grp * 256);
  const i32x4 ka1 = *(const LDS_AS i32x4*)(sk + krow + (grp + 4) * 256);
  const i32x4 kb0 = *(const LDS_AS i32x4*)(sk + krow + 64 + grp * 256);
  const i32x4 kb1 = *(const LDS_AS i32x4*)(sk + krow + 64 + (grp + 4) * 256);
  const i32x8 KA = {ka0[0], ka0[1], ka0[2], ka0[3], ka1[0], ka1[1], ka1[2], ka1[3]};
  const i32x8 KB = {kb0[0], kb0[1], kb0[2], kb0[3], kb1[0], kb1[1], kb1[2], kb1[3]};
  const f32x4 zz = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    la[cg] = mfma_fp8_k128(KA, q.hi[cg], zz);
    lb[cg] = mfma_fp8_k128(KB, q.hi[cg], zz);
    la[cg] = mfma_fp8_k128(KA, q.lo[cg], la[cg]);
    lb[cg] = mfma_fp8_k128(KB, q.lo[cg], lb[cg]);
  }
}

// Softmax and PV of NCH chunks (raw logits la/lb, stages sk, per-token K
// scales at ssc and V scales 32 floats later, first tokens tb) folded into the online softmax as one step: one running-maximum
// update, one accumulator rescale and one value-scale update for all of
// them.  A chunk whose first token lies past every visible range is fully
// masked (its value bytes are zeroed, so its LDS content does not matter).
// Per-chunk operands are read from LDS where they are used, which keeps the
// live registers of several chunks few.
template <int NCG, bool PER_TOKEN, int NCH>
__device__ __forceinline__ void chunk_softmax_pv(WaveState<NCG>& s, const QueryTile<NCG>& q,
                                                 const f32x4 (&la)[NCH][NCG], const f32x4 (&lb)[NCH][NCG],
                                                 const LDS_AS unsigned char* const (&sk)[NCH],
                                                 const LDS_AS float* const (&ssc)[NCH], int grp, int c16,
                                                 const int (&tb)[NCH]) {
  // Tokens j in [jlo, jhi) of this lane's 8 (tb + 8*grp + j) are visible to
  // some column; edge chunks zero the value bytes and scales of the others,
  // since stale page tails must not inject NaN.
  bool edge[NCH];
  int jlo[NCH], jhi[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    edge[ch] = tb[ch] < q.lo_all || tb[ch] + kChunk > q.hi_all;
    const int tok0 = tb[ch] + 8 * grp;
    jlo[ch] = pa_min(pa_max(q.lo_all - tok0, 0), 8);
    jhi[ch] = pa_min(pa_max(q.hi_all - tok0, jlo[ch]), 8);
  }
  auto scales = [&](int ch, int off, float (&x)[8]) {
    const LDS_AS float* ss = ssc[ch] + off + 8 * grp;
    const f32x4 x0 = *(const LDS_AS f32x4*)ss;
    const f32x4 x1 = *(const LDS_AS f32x4*)(ss + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = x0[j];
      x[4 + j] = x1[j];
    }
  };

  // vratio rescales the accumulator when the running maximum of the value
  // scales grows; vmul is that maximum (1 while it is still 0) and vlog its
  // base-2 logarithm, which the exponent subtracts so that the
  // probabilities come out already divided by it.
  float vsc[NCH][8];
  float vratio = 1.0f, vmul = 1.0f, vlog = 0.0f;
  if (PER_TOKEN) {
    float cmax = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      scales(ch, 32, vsc[ch]);
      if (__builtin_expect(edge[ch], 0)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) vsc[ch][j] = (j >= jlo[ch] && j < jhi[ch]) ? vsc[ch][j] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) cmax = fmaxf(cmax, vsc[ch][j]);
    }
    cmax = max_over_groups(cmax);
    const float vnew = fmaxf(s.vsmax, cmax);
    // The probabilities and the accumulator are both taken relative to the
    // same running maximum; the final output multiplies by it again.
    vratio = vnew > 0.0f ? s.vsmax * __builtin_amdgcn_rcpf(vnew) : 1.0f;
    vmul = vnew > 0.0f ? vnew : 1.0f;
    vlog = __builtin_amdgcn_logf(vmul);
    s.vsmax = vnew;
  }

#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    // Base-2 logits l = raw * fac (* per-token key scale).  The column
    // factor is positive (prepare_query), so the maximum is taken on the
    // raw products, which orders them the same way, and the factor goes
    // into the exponent's FMA.
    const float post = q.fac[cg];
    float lg[NCH][8];
    float cmax = kNegInf;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lg[ch][i] = la[ch][cg][i];
        lg[ch][4 + i] = lb[ch][cg][i];
      }
      if (PER_TOKEN) {
        float ksc[8];
        scales(ch, 0, ksc);
#pragma unroll
        for (int j = 0; j < 8; ++j) lg[ch][j] *= ksc[j];
      }
      const bool interior = tb[ch] >= q.lo_max && tb[ch] + kChunk <= q.hi_min;
      if (__builtin_expect(!interior, 0)) {
        const int tok0 = tb[ch] + 8 * grp;
        const int jl = q.vis_lo[cg] - tok0, jh = q.vis_hi[cg] - tok0;
#pragma unroll
        for (int j = 0; j < 8; ++j) lg[ch][j] = (j >= jl && j < jh) ? lg[ch][j] : kNegInf;
      }
      // a linear chain, which the compiler folds into v_max3_f32
#pragma unroll
      for (int j = 0; j < 8; ++j) cmax = fmaxf(cmax, lg[ch][j]);
    }
    cmax = max_over_groups(cmax) * post;  // post > 0: -inf stays -inf
    const float mnew = fmaxf(s.m2[cg], cmax);
    const float muse = mnew == kNegInf ? 0.0f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(s.m2[cg] - muse);
    s.m2[cg] = mnew;
    const float f = alpha * vratio;
    if (__ballot(f != 1.0f)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s.acc[cg][j] *= f;
    }
    // ev = 256 * exp(l - m) (/ vmul with per-token scales, where the
    // probability fed to PV is ev * vsc).
    const float bias = 8.0f - muse - vlog;
    float psum = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      float pr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(lg[ch][j], post, bias));
        psum += ev;
        pr[j] = PER_TOKEN ? ev * vsc[ch][j] : ev;
      }
      long phi, plo;
      split8_fp8(pr, phi, plo);
      // value operands: head dim 16j + c16, tokens 8*grp .. 8*grp+7
      const LDS_AS unsigned char* sv = sk[ch] + kKBytes;
      long V[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        V[j] = *(const LDS_AS long*)(sv + (grp >> 1) * 2048 + (16 * j + c16) * 16 + 8 * (grp & 1));
      if (__builtin_expect(edge[ch], 0)) {
        const uint64_t below_hi = jhi[ch] >= 8 ? ~0ull : (1ull << (8 * jhi[ch])) - 1;
        const uint64_t below_lo = jlo[ch] >= 8 ? ~0ull : (1ull << (8 * jlo[ch])) - 1;
        const uint64_t keep = below_hi & ~below_lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) V[j] = (long)((uint64_t)V[j] & keep);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        s.acc[cg][j] = mfma_fp8(V[j], phi, s.acc[cg][j]);
        s.acc[cg][j] = mfma_fp8(V[j], plo, s.acc[cg][j]);
      }
    }
    s.lsum[cg] = s.lsum[cg] * alpha + psum * vmul;
  }
}

// Softmax and value product of a unit of NCH = 4 (128 tokens) or 2 chunks
// (raw logits la/lb, stages sk, per-token K scales at ssc and V scales 32
// floats later, first tokens tb) of one 16-column block, as one
// online-softmax step.
//
// The value product runs on v_mfma_f32_16x16x128_f8f6f4 with the unit's
// tokens along K: for k-bytes 8 ch .. 8 ch + 7, lane (grp, c16) supplies
// tokens 8 grp .. 8 grp + 7 of chunk ch -- the probabilities its QK results
// hold (B operand, column c16) and the values of head dim 16 j + c16 of the
// same tokens (A operand, one 8-byte LDS read per chunk); a 2-chunk unit
// leaves k-bytes 16 .. 31 zero.  So one MFMA per 16 head dims and fp8 term
// covers the unit: 16 per four chunks instead of 64 of the K = 32 form.
//
// The reference maximum moves lazily: only when the unit's column maximum
// passes it by more than kLazyMax (base 2); the value-scale reference only
// when the unit's largest value scale is more than twice it.  Probabilities
// are 2^(kPBias + l - m) * (value scale / reference) <= 2^(4 + 3) * 2 = 256,
// inside e4m3fn, and the accumulator rescale is skipped unless a reference
// moved -- for smooth logits, after a piece's first unit almost never.
constexpr float kPBias = 4.0f;
constexpr float kLazyMax = 3.0f;

template <bool PER_TOKEN, int NCH>
__device__ __forceinline__ void unit_softmax_pv(WaveState<1>& s, const QueryTile<1>& q, const f32x4 (&la)[NCH][1],
                                                const f32x4 (&lb)[NCH][1],
                                                const LDS_AS unsigned char* const (&sk)[NCH],
                                                const LDS_AS float* const (&ssc)[NCH], int grp, int c16,
                                                const int (&tb)[NCH]) {
  static_assert(NCH == 2 || NCH == 4, "units of two or four chunks");
  auto scales = [&](int ch, int off, float (&x)[8]) {
    const LDS_AS float* ss = ssc[ch] + off + 8 * grp;
    const f32x4 x0 = *(const LDS_AS f32x4*)ss;
    const f32x4 x1 = *(const LDS_AS f32x4*)(ss + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = x0[j];
      x[4 + j] = x1[j];
    }
  };

  // Value scales are read where they are used: the loading wave zeroed the
  // scales of keys no column sees, so no mask applies to them.
  float vratio = 1.0f, vmul = 1.0f, vlog = 0.0f;
  if (PER_TOKEN) {
    float cmax = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      float vs[8];
      scales(ch, 32, vs);
#pragma unroll
      for (int j = 0; j < 8; ++j) cmax = fmaxf(cmax, vs[j]);
    }
    cmax = max_over_groups(cmax);
    const float vnew = cmax > 2.0f * s.vsmax ? cmax : s.vsmax;
    vratio = vnew > s.vsmax && s.vsmax > 0.0f ? s.vsmax * __builtin_amdgcn_rcpf(vnew) : 1.0f;
    vmul = vnew > 0.0f ? vnew : 1.0f;
    vlog = __builtin_amdgcn_logf(vmul);
    s.vsmax = vnew;
  }

  const float post = q.fac[0];  // > 0 (prepare_query)
  float lg[NCH][8];
  float cmax = kNegInf;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lg[ch][i] = la[ch][0][i];
      lg[ch][4 + i] = lb[ch][0][i];
    }
    if (PER_TOKEN) {
      float ksc[8];
      scales(ch, 0, ksc);
#pragma unroll
      for (int j = 0; j < 8; ++j) lg[ch][j] *= ksc[j];
    }
    const bool interior = tb[ch] >= q.lo_max && tb[ch] + kChunk <= q.hi_min;
    if (__builtin_expect(!interior, 0)) {
      const int tok0 = tb[ch] + 8 * grp;
      const int jl = q.vis_lo[0] - tok0, jh = q.vis_hi[0] - tok0;
#pragma unroll
      for (int j = 0; j < 8; ++j) lg[ch][j] = (j >= jl && j < jh) ? lg[ch][j] : kNegInf;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) cmax = fmaxf(cmax, lg[ch][j]);
  }
  cmax = max_over_groups(cmax) * post;
  const bool move = cmax > s.m2[0] + kLazyMax;  // also: the first visible key of the piece
  const float mnew = move ? cmax : s.m2[0];
  const float muse = mnew == kNegInf ? 0.0f : mnew;
  const float alpha = move ? __builtin_amdgcn_exp2f(s.m2[0] - muse) : 1.0f;
  s.m2[0] = mnew;
  const float f = alpha * vratio;
  if (__ballot(f != 1.0f)) scale_inplace(s.acc[0], f);
  const float bias = kPBias - muse - vlog;
  float psum = 0.0f;
  i32x8 PH = {0, 0, 0, 0, 0, 0, 0, 0}, PL = PH;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    float pr[8], vs[8];
    if (PER_TOKEN) scales(ch, 32, vs);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(lg[ch][j], post, bias));
      psum += ev;
      pr[j] = PER_TOKEN ? ev * vs[j] : ev;
    }
    long phi, plo;
    split8_fp8(pr, phi, plo);
    PH[2 * ch] = (int)(uint32_t)phi;
    PH[2 * ch + 1] = (int)(uint32_t)((uint64_t)phi >> 32);
    PL[2 * ch] = (int)(uint32_t)plo;
    PL[2 * ch + 1] = (int)(uint32_t)((uint64_t)plo >> 32);
  }
  // value operands: head dim 16 j + c16, tokens 8 grp .. 8 grp + 7 of each
  // chunk (stale bytes of edge chunks were zeroed in LDS), the next tile's
  // read ahead of this tile's products
  auto value_tile = [&](int j) {
    i32x8 V = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      const LDS_AS unsigned char* sv = sk[ch] + kKBytes;
      const uint64_t v = *(const LDS_AS uint64_t*)(sv + (grp >> 1) * 2048 + (16 * j + c16) * 16 + 8 * (grp & 1));
      V[2 * ch] = (int)(uint32_t)v;
      V[2 * ch + 1] = (int)(uint32_t)(v >> 32);
    }
    return V;
  };
  i32x8 VA[2];
  VA[0] = value_tile(0);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j + 1 < 8) VA[(j + 1) & 1] = value_tile(j + 1);
    mfma_k128_pair(s.acc[0][j], VA[j & 1], PH, PL);
  }
  __builtin_amdgcn_s_setprio(0);
  s.lsum[0] = s.lsum[0] * alpha + psum * vmul;
}

// Maximum of two non-negative floats over the wave, on their bits as
// integers (the same order for non-negative floats; no NaN canonicalisation
// as for float maxima): within each row of 16 lanes by DPP (quad swaps, then
// the 8- and 16-lane mirrors), then across the four rows.
__device__ __forceinline__ float wave_max_nonneg(float a, float b) {
  int v = pa_max(__float_as_int(a), __float_as_int(b));
  v = pa_max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
  v = pa_max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
  v = pa_max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
  v = pa_max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
  auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = pa_max((int)r[0], (int)r[1]);
  r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return __int_as_float(pa_max((int)r[0], (int)r[1]));
}

// QK, softmax and value product of a 128-token unit of four chunks for one
// 16-column block (the cooperative kernel's four-chunk units), as one
// online-softmax step, with lane group g holding chunk g:
//   * QK tile t (t = 0 .. 7) takes key rows 4 c + i = token 4 t + i of
//     chunk c, so the result rows 4 g .. 4 g + 3 of lane group g are tokens
//     4 t .. 4 t + 3 of chunk g: after the eight tiles a lane holds its
//     column's logits for all 32 tokens of chunk g, in order;
//   * the value product (v_mfma_f32_16x16x128_f8f6f4, tokens along K) then
//     takes k-bytes 0 .. 31 of lane (g, c) = tokens 0 .. 31 of chunk g: the
//     probabilities the lane holds (B operand) and, for head dim 16 j + c,
//     the two 16-byte rows [half][dim][16 tokens] of the chunk's value image
//     (A operand: two ds_read_b128 straight into the operand registers).
// Per logit the softmax costs a multiply and an FMA (x = logit * key scale
// * column factor + C, with C = kPBias - m - log2(value reference) per
// column), a share of the maximum,
// one exponential, the sum and the value-scale product with the fp8 split;
// masks run only on units with keys some column does not see.  The
// value-scale reference moves on the unit's largest value scale, which each
// wave reads with two loads per lane (the keys nobody sees have their
// scales zeroed in LDS by the wave that loaded them).  Chunk c sits in ring
// slot (cslot + c) mod S (a missing chunk, c >= nch, reads chunk 0's and is
// masked); tb0 is the unit's first token.  References move lazily, as
// unit_softmax_pv describes.
template <bool PER_TOKEN, int S, int kSlotBytes>
__device__ __forceinline__ void unit4_softmax_pv(WaveState<1>& s, const QueryTile<1>& q,
                                                 const LDS_AS unsigned char* ring, int cslot, int nch, int tb0,
                                                 int grp, int c16) {
  // Per-lane bases: the key row's chunk (c16 / 4) and the lane's own chunk
  // (grp), chunk c sitting in ring slot (cslot + c) mod S (a missing chunk
  // reads chunk 0's slot).
  auto slot_of = [&](int c) {
    int sl = cslot + (c < nch ? c : 0);
    sl = sl >= S ? sl - S : sl;
    return ring + sl * kSlotBytes;
  };
  const int kc = c16 >> 2;  // the chunk whose key rows this lane supplies
  const LDS_AS unsigned char* kb = slot_of(kc) + (c16 & 3) * 16 + grp * 256;
  const LDS_AS unsigned char* own = slot_of(grp);
  const LDS_AS unsigned char* vb = own + kKBytes + c16 * 16;
  const LDS_AS float* sb = (const LDS_AS float*)(own + kKBytes + kVBytes);
  // key products, the next tile's operand read ahead of this tile's MFMAs;
  // token 4 t + i of chunk kc sits in row (4 t + i) ^ 4 kc of its half (the
  // loads' swizzle)
  auto key_tile = [&](int t) {
    const int off = (t >> 2) * kKHalf + (((t & 3) ^ kc) << 6);
    const i32x4 k0 = *(const LDS_AS i32x4*)(kb + off);
    const i32x4 k1 = *(const LDS_AS i32x4*)(kb + off + 1024);
    return i32x8{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
  };
  // Tokens of the lane's chunk: tok0 + k.  full: every token of the unit
  // is visible to every column (wave-uniform).
  const int tok0 = tb0 + 32 * grp;
  const bool full = nch == 4 && tb0 >= q.lo_max && tb0 + 128 <= q.hi_min;
  // the column's own visible keys among the lane's 32
  const int jl = q.vis_lo[0] - tok0;
  const int jh = grp < nch ? q.vis_hi[0] - tok0 : jl;

  // The unit's largest value scale, each lane reading tokens 2 c16 and
  // 2 c16 + 1 of its own chunk (non-negative floats: compared as integers;
  // the scales of keys nobody sees were zeroed in LDS, and a missing chunk
  // reads chunk 0's), reduced while the key product runs.
  float cmax = 0.0f;
  if (PER_TOKEN) {
    const f32x2 vv = *(const LDS_AS f32x2*)(sb + 32 + 2 * c16);
    cmax = wave_max_nonneg(vv[0], vv[1]);
  }

  // The key product (eight tiles, the next tile's operands read ahead of
  // this tile's MFMAs), at raised wave priority: a wave that reaches its
  // matrix block issues it back to back while the other wave of the SIMD
  // works through its softmax on the VALU.
  f32x4 lg4[8];
  {
    i32x8 KA[2];
    KA[0] = key_tile(0);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (t + 1 < 8) KA[(t + 1) & 1] = key_tile(t + 1);
      const f32x4 zz = {0.f, 0.f, 0.f, 0.f};
      lg4[t] = mfma_fp8_k128(KA[t & 1], q.hi[0], zz);
      lg4[t] = mfma_fp8_k128(KA[t & 1], q.lo[0], lg4[t]);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  // y: the key product times the per-token key scale (the base-2 logit is
  // y * post, post > 0), -inf for keys the column does not see.  The unit's
  // maximum is taken on y, so the references settle before any exponent is
  // formed and every x = y * post + C is computed once, with the final C.
  const float post = q.fac[0];  // > 0 (prepare_query)
  float x[32];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    f32x4 ks = {1.f, 1.f, 1.f, 1.f};
    if (PER_TOKEN) ks = *(const LDS_AS f32x4*)(sb + 4 * t);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[4 * t + i] = PER_TOKEN ? lg4[t][i] * ks[i] : lg4[t][i];
  }
  if (!full) {
    // a real branch: speculated, these selects would run on every unit
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < 32; ++k) x[k] = (k >= jl && k < jh) ? x[k] : kNegInf;
  }
  float xmax = kNegInf;
#pragma unroll
  for (int k = 0; k < 32; ++k) xmax = fmaxf(xmax, x[k]);
  // The column's maximum base-2 logit this unit is max y * post.  The
  // maximum reference moves to it when it passes the reference by more than
  // kLazyMax (and on the column's first visible key); the value-scale
  // reference moves to the unit's largest scale when that exceeds twice it.
  // Every probability is then at most 2^(kPBias + kLazyMax) times a
  // value-scale ratio of at most 2.
  const float lmax = max_over_groups(xmax) * post;
  const bool move = lmax > s.m2[0] + kLazyMax;
  const bool vmove = PER_TOKEN && cmax > 2.0f * s.vsmax;  // wave-uniform
  const float mnew = move ? lmax : s.m2[0];
  const float muse = mnew == kNegInf ? 0.0f : mnew;
  const float alpha = move ? __builtin_amdgcn_exp2f(s.m2[0] - muse) : 1.0f;
  s.m2[0] = mnew;
  float vratio = 1.0f;
  if (vmove) {
    vratio = s.vsmax > 0.0f ? s.vsmax * __builtin_amdgcn_rcpf(cmax) : 1.0f;
    s.vsmax = cmax;
  }
  const float vmul = PER_TOKEN && s.vsmax > 0.0f ? s.vsmax : 1.0f;
  // x = y * post + C, C from the settled references (the column's maximum m,
  // 0 while it has none, and the value-scale reference)
  const float C = kPBias - muse - (PER_TOKEN ? __builtin_amdgcn_logf(vmul) : 0.0f);
  // probabilities 2^x (times the value scale) into the fp8 hi + lo
  // operands PH, PL and their sum psum (stale value scales were zeroed in
  // LDS: a masked key gives 0 * 0)
  float psum;
  i32x8 PH, PL;
  auto probabilities = [&]() {
    psum = 0.0f;
#pragma unroll
    for (int k8 = 0; k8 < 4; ++k8) {
      f32x4 v0 = {1.f, 1.f, 1.f, 1.f}, v1 = v0;
      if (PER_TOKEN) {
        v0 = *(const LDS_AS f32x4*)(sb + 32 + 8 * k8);
        v1 = *(const LDS_AS f32x4*)(sb + 36 + 8 * k8);
      }
      float pr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ev = __builtin_amdgcn_exp2f(__builtin_fmaf(x[8 * k8 + i], post, C));
        psum += ev;
        pr[i] = PER_TOKEN ? ev * (i < 4 ? v0[i] : v1[i - 4]) : ev;
      }
      long phi, plo;
      split8_fp8<PER_TOKEN>(pr, phi, plo);  // per-token: pr = ev * scale
      PH[2 * k8] = (int)(uint32_t)phi;
      PH[2 * k8 + 1] = (int)(uint32_t)((uint64_t)phi >> 32);
      PL[2 * k8] = (int)(uint32_t)plo;
      PL[2 * k8 + 1] = (int)(uint32_t)((uint64_t)plo >> 32);
    }
  };
  probabilities();
  const float f = alpha * vratio;
  if (__ballot(f != 1.0f)) scale_inplace(s.acc[0], f);
  // value operands (stale bytes of edge chunks were zeroed in LDS), the
  // next tile's read ahead of this tile's products
  auto value_tile = [&](int j) {
    const i32x4 v0 = *(const LDS_AS i32x4*)(vb + j * 256);
    const i32x4 v1 = *(const LDS_AS i32x4*)(vb + j * 256 + 2048);
    return i32x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  };
  i32x8 VA[2];
  VA[0] = value_tile(0);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j + 1 < 8) VA[(j + 1) & 1] = value_tile(j + 1);
    mfma_k128_pair(s.acc[0][j], VA[j & 1], PH, PL);
  }
  __builtin_amdgcn_s_setprio(0);
  s.lsum[0] = s.lsum[0] * alpha + psum * vmul;
}

// One 32-token chunk of keys and values, staged in LDS at sk (keys: two
// 16-token halves [8 dim chunks][16 tokens][16 B], kKHalf apart; values:
// [2 halves][128 head dims][16 tokens]; per-token K then V scales), folded
// into the wave's online softmax.  tb is the chunk's first token.
template <int NCG, bool PER_TOKEN>
__device__ __forceinline__ void compute_chunk(WaveState<NCG>& s, const QueryTile<NCG>& q,
                                              const LDS_AS unsigned char* sk, int krow, int grp, int c16, int tb) {
  f32x4 la[1][NCG], lb[1][NCG];
  chunk_logits<NCG>(q, sk, krow, grp, la[0], lb[0]);
  const LDS_AS unsigned char* const sks[1] = {sk};
  const LDS_AS float* const sss[1] = {(const LDS_AS float*)(sk + kKBytes + kVBytes)};
  const int tbs[1] = {tb};
  chunk_softmax_pv<NCG, PER_TOKEN, 1>(s, q, la, lb, sks, sss, grp, c16, tbs);
}

// Workgroup geometry.  A workgroup covers `slots_per_workgroup`
// consecutive slots of one (sequence, kv head).  Its waves form `groups`
// groups of `wslot` waves; group g owns local slots g, g + groups, ... and
// the waves of a group deal that slot's 32-token chunks round robin.  Each
// wave streams the chunks of all its slots back to back through its LDS
// ring, so the pipeline runs across slot boundaries.  When a wave owns
// several slots (MULTI) it finalises each slot's partial as soon as the
// slot ends and folds it into a running combination; otherwise the slot
// partials are produced by the workgroup merge at the end.  A workgroup
// that covers every slot of its (sequence, kv head) also merges them into
// the final output.
//
// Block table, context lengths and scales come in as separate restrict
// pointers so that their wave-uniform loads become scalar (SMEM) loads:
// page lookups then count on lgkmcnt and never force a wait on the vmcnt
// of the direct-to-LDS data loads in flight.
template <int NCG, bool PER_TOKEN, bool BS16, int STAGES, bool MULTI, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void pa_fp8_partition_kernel(const pa_fp8_partition_args a,
                                                                    const int32_t* __restrict__ block_tables,
                                                                    const int32_t* __restrict__ kv_indptr,
                                                                    const int32_t* __restrict__ context_lengths,
                                                                    const float* __restrict__ key_scale,
                                                                    const float* __restrict__ value_scale) {
  constexpr int kStageBytes = kKBytes + kVBytes + (PER_TOKEN ? kScaleBytes : 0);
  constexpr int kWaveBytes = STAGES * kStageBytes;
  constexpr int kNT = 64 * WAVES;
  constexpr int kMergeBytes = 2 * WAVES * 16 * 4 + WAVES * kHead * 16 * 4;
  constexpr int kSmemBytes = WAVES * kWaveBytes > kMergeBytes ? WAVES * kWaveBytes : kMergeBytes;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kSmemBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4;
  const int c16 = lane & 15;

  const int P = a.num_partitions;
  const int SPW = a.slots_per_workgroup;
  const int PG = pa_cdiv(P, SPW);
  int bid = blockIdx.x;
  const int pg = bid % PG;
  bid /= PG;
  const int h = bid % a.num_kv_heads;
  const int b = bid / a.num_kv_heads;
  const int zs = pg * SPW;
  const int nslots = pa_min(P - zs, SPW);
  const bool owner = PG == 1;
  const bool direct_out = owner && a.output != nullptr;
  const bool want_partials = a.exp_sums != nullptr;
  const int wslot = nslots >= WAVES ? 1 : WAVES / nslots;
  const int groups = WAVES / wslot;
  const int gid = wave / wslot;
  const int rank = wave - gid * wslot;

  const int ql = a.query_length;
  const int gqa = a.query_group_size;
  const int eq = ql * gqa;
  const int W = a.sliding_window;
  const int ctx = context_lengths[b];

  int lo_all, hi_all, unused;
  pa_plan_visible(ctx, 0, ql, W, &lo_all, &unused);
  pa_plan_visible(ctx, ql - 1, ql, W, &unused, &hi_all);

  const int bs = a.block_size;
  const int bs_shift = BS16 ? 4 : __builtin_ctz((unsigned)bs);
  const int64_t row_off = kv_indptr ? (int64_t)kv_indptr[b] : (int64_t)b * a.stride_bt_seq;
  const int row_len = kv_indptr ? kv_indptr[b + 1] - kv_indptr[b] : a.max_blocks_per_seq;
  const int32_t* bt_row = block_tables + row_off;
  const int last_page = pa_min(pa_cdiv(ctx, bs) - 1, row_len - 1);
  const bool has_pages = row_len > 0;
  const int nblocks = a.num_blocks;

  // Chunks of slot z: first chunk token (32-aligned) and how many of the
  // slot's chunks wave-rank `rank` takes.  Wave-uniform.
  auto slot_range = [&](int z, int& cbeg, int& nmine) {
    int t0, t1;
    pa_plan_slot_tokens(ctx, P, z, W, ql, &t0, &t1);
    const int a0 = pa_max(t0, lo_all);
    const int a1 = pa_min(t1, hi_all);
    cbeg = a0 & ~(kChunk - 1);
    nmine = 0;
    if (a1 > a0 && has_pages) {
      const int n = pa_cdiv(a1 - cbeg, kChunk);
      nmine = n > rank ? (n - rank + wslot - 1) / wslot : 0;
    }
  };

  if (nslots == 1) {
    // One slot per workgroup: an empty slot writes (0, -inf, 0) and stops
    // (reference empty-slot semantics, kernels/pa_decode_swa.py:1493-1504).
    int t0, t1;
    pa_plan_slot_tokens(ctx, P, zs, W, ql, &t0, &t1);
    if (!(pa_min(t1, hi_all) > pa_max(t0, lo_all) && has_pages)) {
      const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int idx = tid; idx < eq * (kHead / 8); idx += kNT) {
        const int e = idx / (kHead / 8);
        const int d0 = (idx % (kHead / 8)) * 8;
        if (want_partials) store_partial8(a, b, h, zs, e, d0, z);
        if (direct_out) store_output8(a, b, h, e, d0, z);
      }
      if (want_partials)
        for (int e = tid; e < eq; e += kNT) store_stats(a, b, h, zs, e, 0.0f, kNegInf);
      return;
    }
  }

  // ---------------- query: raw loads (issued before the first KV chunk) ----------------
  i32x4 qraw[NCG][4];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    const int e = cg * 16 + c16;
    if (e < eq) {
      const int qi = e / gqa;
      const int g = e - qi * gqa;
      const uint16_t* qp = (const uint16_t*)a.query + (int64_t)(b * ql + qi) * a.stride_q_tok +
                           (int64_t)(h * gqa + g) * a.stride_q_head;
      qraw[cg][0] = *(const i32x4*)(qp + 16 * grp);
      qraw[cg][1] = *(const i32x4*)(qp + 16 * grp + 8);
      qraw[cg][2] = *(const i32x4*)(qp + 16 * (grp + 4));
      qraw[cg][3] = *(const i32x4*)(qp + 16 * (grp + 4) + 8);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qraw[cg][i] = i32x4{0, 0, 0, 0};
    }
  }

  const uint8_t* kbase = (const uint8_t*)a.key_cache + (int64_t)h * a.stride_k_head;
  const uint8_t* vbase = (const uint8_t*)a.value_cache + (int64_t)h * a.stride_v_head;
  const float* ksbase = PER_TOKEN ? key_scale + (int64_t)h * a.stride_ks_head : nullptr;
  const float* vsbase = PER_TOKEN ? value_scale + (int64_t)h * a.stride_ks_head : nullptr;

  LDS_AS unsigned char* ring = (LDS_AS unsigned char*)smem + wave * kWaveBytes;

  // Per-lane byte offsets of the direct-to-LDS loads.  Every load
  // instruction reads from a single page, so its address is a wave-uniform
  // page base plus one of these constants.  Lane l of a 1 KiB load fills
  // LDS bytes 16l .. 16l+15 of its destination.
  //   keys   : (16-dim chunk 4q + l/16, token l%16) of a 16-token half
  //   values : trans layout -> bytes 16l of a [head dim][16 tokens] group;
  //            plain layout -> head dim 64q + l, 16 tokens
  const int koff_lane = BS16 ? lane * 16 : (lane >> 4) * (bs * 16) + (lane & 15) * 16;
  const int voff_plain = lane * bs;

  auto clamp_page = [&](int p) -> int {
    pa_note(p < 0 || p >= nblocks, PA_VIOLATION_PAGE);
    p = p < 0 ? 0 : p;
    return p < nblocks ? p : nblocks - 1;
  };
  // Block-table entries of the (one or two) pages of the chunk starting at
  // token tb.  Reads past the context reuse the last page (its tokens are
  // masked).  Clamped into the cache only when used, one step later, so the
  // scalar loads overlap the current chunk's compute.
  auto fetch_pages = [&](int tb, int& q0, int& q1) {
    const int lp0 = tb >> bs_shift;
    q0 = bt_row[pa_min(lp0, last_page)];
    q1 = BS16 ? bt_row[pa_min(lp0 + 1, last_page)] : q0;
  };

  auto issue = [&](int tb, int st, int raw0, int raw1) {
    const int p0 = clamp_page(raw0);
    const int p1 = BS16 ? clamp_page(raw1) : p0;
    LDS_AS unsigned char* sk = ring + st * kStageBytes;
    LDS_AS unsigned char* sv = sk + kKBytes;
    if (BS16) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint8_t* kp = kbase + (int64_t)(hh ? p1 : p0) * a.stride_k_block;
        const uint8_t* vp = vbase + (int64_t)(hh ? p1 : p0) * a.stride_v_block;
#pragma unroll
        for (int q = 0; q < 2; ++q) lds_dma16(kp + koff_lane + q * 1024, sk + hh * kKHalf + q * 1024);
#pragma unroll
        for (int q = 0; q < 2; ++q) lds_dma16(vp + lane * 16 + q * 1024, sv + hh * 2048 + q * 1024);
      }
    } else {
      const int s0 = tb & (bs - 1);
      const uint8_t* kp = kbase + (int64_t)p0 * a.stride_k_block + s0 * 16;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          lds_dma16(kp + hh * 256 + q * (4 * bs * 16) + koff_lane, sk + hh * kKHalf + q * 1024);
      if (a.trans_v) {
        const uint8_t* vp = vbase + (int64_t)p0 * a.stride_v_block + (s0 >> 4) * (kHead * 16);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int q = 0; q < 2; ++q) lds_dma16(vp + hh * 2048 + q * 1024 + lane * 16, sv + hh * 2048 + q * 1024);
      } else {
        const uint8_t* vp = vbase + (int64_t)p0 * a.stride_v_block + s0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            lds_dma16(vp + hh * 16 + q * (64 * bs) + voff_plain, sv + hh * 2048 + q * 1024);
      }
    }
    if (PER_TOKEN) {
      LDS_AS unsigned char* ss = sv + kVBytes;
      if (lane < 16) {
        const int tt = (lane & 7) * 4;
        const int pg2 = BS16 ? (tt >= 16 ? p1 : p0) : p0;
        const int sidx = BS16 ? (tt & 15) : (tb & (bs - 1)) + tt;
        const float* base = lane < 8 ? ksbase : vsbase;
        lds_dma16_cached(base + (int64_t)pg2 * a.stride_ks_block + sidx, ss);
      }
    }
  };

  // ---------------- issue cursor: the next chunk of this wave to load ----------------
  int ic_l = gid;  // local slot index
  int ic_j = 0;    // chunk index within this wave's share of the slot
  int ic_cbeg = 0, ic_n = 0;
  if (ic_l < nslots) slot_range(zs + ic_l, ic_cbeg, ic_n);
  auto ic_skip_empty = [&]() {
    while (ic_l < nslots && ic_j >= ic_n) {
      ic_l += groups;
      ic_j = 0;
      if (ic_l < nslots) slot_range(zs + ic_l, ic_cbeg, ic_n);
    }
  };
  ic_skip_empty();
  auto ic_tb = [&]() { return ic_cbeg + (rank + ic_j * wslot) * kChunk; };

  WaveState<NCG> st;
  st.reset();
  // Combination of the finished slots of this wave (MULTI only; in value
  // units: per-tensor / per-token value scales already applied).
  float mC[MULTI ? NCG : 1], lC[MULTI ? NCG : 1];
  f32x4 accC[MULTI ? NCG : 1][8];
  if (MULTI) {
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      mC[cg] = kNegInf;
      lC[cg] = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) accC[cg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // Pipeline: chunks g+1 .. g+STAGES-1 (in this wave's global order) are in
  // flight while chunk g is computed; the page indices of the next chunk to
  // issue are fetched one step ahead so their scalar-load latency is hidden.
  int np0 = 0, np1 = 0;
  if (ic_l < nslots) fetch_pages(ic_tb(), np0, np1);
#pragma unroll
  for (int k = 0; k < STAGES - 1; ++k) {
    if (ic_l < nslots) {
      issue(ic_tb(), k, np0, np1);
      ++ic_j;
      ic_skip_empty();
      if (ic_l < nslots) fetch_pages(ic_tb(), np0, np1);
    }
  }

  // ---------------- query: scale, split into fp8 hi + lo ----------------
  QueryTile<NCG> qt;
  const float k_tensor_scale = PER_TOKEN ? 1.0f : key_scale[0];
  const float v_tensor_scale = PER_TOKEN ? 1.0f : value_scale[0];
  prepare_query<NCG>(qt, qraw, a.query_dtype, a.softmax_scale * kLog2e * k_tensor_scale, ctx, ql, gqa, W, c16);
  // Key row r of QK tile t (0, 1) is chunk token 8*(r/4) + 4t + r%4: that
  // token's 16-byte pieces for dim chunks grp and grp+4.
  const int krow = (c16 >> 3) * kKHalf + (8 * ((c16 >> 2) & 1) + (c16 & 3)) * 16;

  int gc = 0;  // chunks of this wave computed so far
  for (int l = gid; l < nslots; l += groups) {
    const int z = zs + l;
    int cbeg, nmine;
    slot_range(z, cbeg, nmine);
    for (int k = 0; k < nmine; ++k) {
      const int stg = gc % STAGES;
      if (ic_l < nslots) {
        issue(ic_tb(), (gc + STAGES - 1) % STAGES, np0, np1);
        ++ic_j;
        ic_skip_empty();
        if (ic_l < nslots) fetch_pages(ic_tb(), np0, np1);
        // Loads retire in order: leave the newest chunks' loads in flight.
        constexpr int kLoadsPerChunk = 8 + (PER_TOKEN ? 1 : 0);
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk * (STAGES - 1)));
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      ++gc;
      const int tb = cbeg + (rank + k * wslot) * kChunk;
      const LDS_AS unsigned char* sk = ring + stg * kStageBytes;
      compute_chunk<NCG, PER_TOKEN>(st, qt, sk, krow, grp, c16, tb);
    }
    if (MULTI) {
      // Slot z is complete (this wave owns it alone): write its partial and
      // fold it into the wave's running combination.
      const float vfin = PER_TOKEN ? st.vsmax : v_tensor_scale;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const float L = sum_over_groups(st.lsum[cg]);
        const float m = st.m2[cg];
        const int e = cg * 16 + c16;
        if (want_partials && e < eq) {
          const float sc = L > 0.0f ? vfin / L : 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) store_partial4(a, b, h, z, e, 16 * j + 4 * grp, st.acc[cg][j] * sc);
          if (grp == 0) store_stats(a, b, h, z, e, L * (1.0f / 256.0f), m * kLn2);
        }
        const float Mn = fmaxf(mC[cg], m);
        const float Mu = Mn == kNegInf ? 0.0f : Mn;
        const float fc = __builtin_amdgcn_exp2f(mC[cg] - Mu);
        const float fs = __builtin_amdgcn_exp2f(m - Mu);
        const float fsv = fs * vfin;
#pragma unroll
        for (int j = 0; j < 8; ++j) accC[cg][j] = accC[cg][j] * fc + st.acc[cg][j] * fsv;
        lC[cg] = lC[cg] * fc + L * fs;
        mC[cg] = Mn;
      }
      st.reset();
    }
  }

  // ---------------- workgroup merge ----------------
  // Each wave publishes (max, sum, value-unit accumulator) per column; sets
  // of waves are then combined by log-sum-exp: each group of `wslot` waves
  // into its slot's partial (unless MULTI waves already wrote them), and,
  // for a workgroup that covers every slot, all waves into the output.
  const float vfin_end = PER_TOKEN ? st.vsmax : v_tensor_scale;
  float* mbuf = (float*)smem;             // [wave][16]
  float* lbuf = mbuf + WAVES * 16;        // [wave][16]
  float* abuf = lbuf + WAVES * 16;        // [wave][head dim][16]
  const int ngp = (!MULTI && want_partials) ? pa_min(groups, nslots) : 0;
  const int nsets = ngp + (direct_out ? 1 : 0);
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    float Mst, Lst, sc;
    if (MULTI) {
      Mst = mC[cg];
      Lst = lC[cg];
      sc = 1.0f;
    } else {
      Mst = st.m2[cg];
      Lst = sum_over_groups(st.lsum[cg]);
      sc = vfin_end;
    }
    __syncthreads();
    if (grp == 0) {
      mbuf[wave * 16 + c16] = Mst;
      lbuf[wave * 16 + c16] = Lst;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        abuf[(wave * kHead + 16 * j + 4 * grp + i) * 16 + c16] = (MULTI ? accC[cg][j][i] : st.acc[cg][j][i]) * sc;
    __syncthreads();
    for (int idx = tid; idx < nsets * 256; idx += kNT) {
      const int set = idx >> 8;
      const int col = (idx >> 4) & 15;
      const int d0 = (idx & 15) * 8;
      const int e = cg * 16 + col;
      if (e >= eq) continue;
      const int w0 = set < ngp ? set * wslot : 0;
      const int w1 = set < ngp ? w0 + wslot : WAVES;
      float Mc = kNegInf;
      for (int w = w0; w < w1; ++w) Mc = fmaxf(Mc, mbuf[w * 16 + col]);
      const float Mcu = Mc == kNegInf ? 0.0f : Mc;
      float L = 0.0f;
      float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int w = w0; w < w1; ++w) {
        const float f = __builtin_amdgcn_exp2f(mbuf[w * 16 + col] - Mcu);
        L += lbuf[w * 16 + col] * f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] += abuf[(w * kHead + d0 + i) * 16 + col] * f;
      }
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] *= inv;
      if (set < ngp) {
        const int z = zs + set;
        store_partial8(a, b, h, z, e, d0, o);
        if (d0 == 0) store_stats(a, b, h, z, e, L * (1.0f / 256.0f), Mc * kLn2);
      } else {
        store_output8(a, b, h, e, d0, o);
      }
    }
  }
}

// ============================================================================
// Per-wave streaming decode (work list or balanced split)
// ============================================================================

// Cost of a (sequence, kv head) pair's start, in chunks, in the per-wave
// balanced split: a run that holds more pieces (each with its query setup
// and its output or partial store) gets fewer chunks.
#ifndef PA_FP8_PIECE_COST
#define PA_FP8_PIECE_COST 1
#endif
constexpr int kStreamPieceCost = PA_FP8_PIECE_COST;
// The same for the cooperative kernel's workgroup runs, whose pieces also
// start with a 64-column query setup and end in a partly filled unit.
#ifndef PA_FP8_COOP_PIECE_COST
#define PA_FP8_COOP_PIECE_COST 4
#endif
constexpr int kCoopPieceCost = PA_FP8_COOP_PIECE_COST;

// A balanced launch gives every wave at least this many chunks (it uses
// fewer waves for small problems).
constexpr int kMinChunksPerWave = 8;

// One piece of a wave's walk: chunks [tb0, tb0 + 32 n) of (sequence b, kv
// head h).  target < 0: the piece is the whole (sequence, kv head) and
// goes to the output; otherwise it is a partial (balanced: partial id;
// work list: partial row of query 0).
struct Piece {
  int b, h, ctx, lo_all, hi_all;
  int tb0, n;
  int target;
  int orow;       // output row of query 0 of the sequence
  int desc_cnt;   // balanced: pieces of the pair, when this piece starts it
  int last_page;  // last page index of the sequence's page list
  int64_t bt_off; // offset of the sequence's page list in block_tables
  int cut;        // bin walk: bit 0 the work began before the piece, bit 1 it goes on after it
  int wstart;     // bin walk: position of the work's first chunk in the bin
};

// Wave-uniform read of read-only kernel input through the constant address
// space, so it is a scalar (SMEM) load counted on lgkmcnt: it never waits on
// the vmcnt of the direct-to-LDS loads in flight.
__device__ __forceinline__ int ld_uniform(const int32_t* p, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

// Sequence-level fields of a piece: context, visible range, page list.
__device__ __forceinline__ void piece_sequence(Piece& p, const pa_fp8_stream_args& a, const int32_t* kv_indptr,
                                               const int32_t* context_lengths, int b) {
  p.b = b;
  p.ctx = ld_uniform(context_lengths, b);
  int u;
  pa_plan_visible(p.ctx, 0, a.query_length, a.sliding_window, &p.lo_all, &u);
  pa_plan_visible(p.ctx, a.query_length - 1, a.query_length, a.sliding_window, &u, &p.hi_all);
  int row_len;
  if (kv_indptr) {
    p.bt_off = ld_uniform(kv_indptr, b);
    row_len = ld_uniform(kv_indptr, b + 1) - (int)p.bt_off;
  } else {
    p.bt_off = (int64_t)b * a.stride_bt_seq;
    row_len = a.max_blocks_per_seq;
  }
  p.last_page = pa_min(pa_cdiv(p.ctx, a.block_size) - 1, row_len - 1);
  if (p.last_page < 0) p.hi_all = p.lo_all;  // no pages: nothing visible
  p.orow = b * a.query_length;
}

// Balanced split: chunks of all (sequence, kv head) pairs, sequence-major
// with kv heads inner, each pair preceded by A units of start cost, cut into
// nw equal runs (pa_plan_run_begin).  With a
// head group G > 1 the split runs over (sequence, group of G adjacent kv
// heads, chunk) and each run is walked by G consecutive waves in step, wave
// i taking head i of every group: the waves of a workgroup then read the
// same pages of adjacent heads at the same time, and adjacent heads'
// per-token scales, which share 128-byte lines, are fetched once.
struct BalancedWalk {
  int b, h, nb, c, first, wid, run, G, A, nw;
  // Positions in the split's cost order (a pair's group costs A, then one
  // per chunk): of the next chunk, of the end of this run, of the current
  // group's start; and the total.
  long long pos, end, P, T;
  Piece seq;  // sequence-level fields of b

  __device__ __forceinline__ bool next(Piece& p, const pa_fp8_stream_args& a, const int32_t* kv_indptr,
                                       const int32_t* context_lengths) {
    if (pos >= end) return false;
    p = seq;
    p.h = h;
    p.tb0 = (seq.lo_all & ~(kChunk - 1)) + c * kChunk;
    const long long rem = end - pos;
    p.n = rem < nb - c ? (int)rem : nb - c;
    const bool whole = c == 0 && p.n == nb;
    p.target = whole ? -1 : 2 * wid + (first ? 0 : 1);
    p.desc_cnt = c != 0 ? 0 : (whole ? 1 : pa_plan_run_of_chunk(P + A + nb - 1, T, nw) - run + 1);
    first = 0;
    c += p.n;
    pos += p.n;
    if (pos < end && c == nb) {
      c = 0;
      P += nb + A;
      pos = P + A;
      if ((h += G) >= a.num_kv_heads) {
        h -= a.num_kv_heads;  // head i of the next sequence's first group
        do {
          if (b + 1 >= a.num_seqs) {  // inconsistent context lengths: stop
            pos = end;
            break;
          }
          ++b;
          piece_sequence(seq, a, kv_indptr, context_lengths, b);
          nb = seq.hi_all > seq.lo_all ? pa_cdiv(seq.hi_all - (seq.lo_all & ~(kChunk - 1)), kChunk) : 0;
        } while (nb == 0);
      }
    }
    return true;
  }
};

// Chunks [tb0, tb0 + 32 n) of a work over partitions [kv0, kv1) (cumulative,
// pb = the sequence's first) of a sequence with context ctx, visible keys
// [lo_all, hi_all) and last page last_page (< 0: no pages, nothing visible).
// Works of one sequence meet at partition boundaries, which are chunk
// boundaries, so their chunk ranges tile the sequence's.
__device__ __forceinline__ void work_chunks(int ctx, int lo_all, int hi_all, int last_page, int pb, int kv0, int kv1,
                                            int& tb0, int& n) {
  const int a0 = pa_max((kv0 - pb) * PA_PARTITION_TOKENS, lo_all);
  const int a1 = pa_min(pa_min((kv1 - pb) * PA_PARTITION_TOKENS, ctx), last_page < 0 ? lo_all : hi_all);
  if (a1 > a0) {
    tb0 = a0 & ~(kChunk - 1);
    n = pa_cdiv(a1 - tb0, kChunk);
  } else {
    tb0 = 0;
    n = 0;
  }
}

// Work-list walk: works [idx, end) of a bin.
struct WorklistWalk {
  int idx, end;
  __device__ __forceinline__ bool next(Piece& p, const pa_fp8_stream_args& a, const int32_t* kv_indptr,
                                       const int32_t* context_lengths, const int32_t* work_info,
                                       const int32_t* partition_indptr) {
    if (idx >= end) return false;
    const int64_t w = 8 * (int64_t)idx;
    ++idx;
    const int b = ld_uniform(work_info, w), ploc = ld_uniform(work_info, w + 1), qo0 = ld_uniform(work_info, w + 2);
    const int kv0 = ld_uniform(work_info, w + 4), kv1 = ld_uniform(work_info, w + 5);
    const int qh0 = ld_uniform(work_info, w + 7) & 0xffff;
    piece_sequence(p, a, kv_indptr, context_lengths, b);
    p.h = qh0 / a.query_group_size;
    const int pb = ld_uniform(partition_indptr, b);
    work_chunks(p.ctx, p.lo_all, p.hi_all, p.last_page, pb, kv0, kv1, p.tb0, p.n);
    p.target = ploc < 0 ? -1 : ploc + a.query_length;
    p.cut = 0;
    p.wstart = 0;
    p.orow = qo0;
    p.desc_cnt = 0;
    return true;
  }
};

// Head group of a balanced launch of per-wave runs over H kv heads and
// num_workers waves for eq query columns: the largest power of two up to a
// workgroup's waves that divides both (so a group's waves share a
// workgroup), else 1.
__host__ __device__ constexpr int balanced_group(int H, int num_workers, int eq) {
  int g = stream_waves(stream_nq(eq));
  while (g > 1 && (H % g != 0 || num_workers % g != 0)) g >>= 1;
  return g;
}

// Start of worker `wid`'s walk in a balanced launch over `num_workers`
// workers (waves or workgroups) in head groups of G (run wid / G, head
// wid % G of each group): every context length is loaded once (lane l
// holds sequences l*K .. l*K+K-1, K <= 16), scanned across the wave, and
// the run's first (sequence, head group, chunk) is located with a ballot
// and scalar readlanes.  Returns false when the run is empty.
__device__ __forceinline__ bool balanced_start(BalancedWalk& w, const pa_fp8_stream_args& a,
                                               const int32_t* __restrict__ kv_indptr,
                                               const int32_t* __restrict__ context_lengths, int wid, int lane,
                                               int G, int A) {
  const int H = a.num_kv_heads / G;  // head groups
  const int ql = a.query_length;
  const int W = a.sliding_window;
  // Chunks per sequence: lane l holds sequences l*K .. l*K+K-1.
  const int B = a.num_seqs;
  const int K = pa_cdiv(B, 64);
  // All loads first (indices clamped into the batch), then the counts.
  int cnt[16], rl[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int bb = pa_min(lane * K + k, B - 1);
    cnt[k] = context_lengths[bb];
    const int32_t* rows = kv_indptr ? kv_indptr : context_lengths;
    const int r0 = rows[bb], r1 = rows[kv_indptr ? bb + 1 : bb];
    rl[k] = kv_indptr ? r1 - r0 : 1;
  }
  int mine = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const bool real = k < K && lane * K + k < B;
    cnt[k] = real && rl[k] > 0 ? pa_plan_seq_chunks(cnt[k], ql, W) : 0;
    mine += cnt[k] > 0 ? cnt[k] + A : 0;
  }
  int incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  const int excl = incl - mine;
  // Wave-uniform from here on (readlane), so the walk lives in SGPRs and
  // its page lookups are scalar loads.
  const long long T = (long long)__builtin_amdgcn_readlane(incl, 63) * H;
  long long nwl = T / kMinChunksPerWave;
  nwl = nwl < 1 ? 1 : nwl;
  const int runs = a.num_workers / G;
  const int nw = nwl < runs ? (int)nwl : runs;
  const int run = wid / G;
  if (run >= nw) return false;
  const long long g0 = pa_plan_run_begin(run, T, nw);
  const long long g1 = pa_plan_run_begin(run + 1, T, nw);
  if (g1 <= g0) return false;
  // The lane whose sequences hold chunk g0, then the sequence itself.
  const uint64_t hit = __ballot(mine > 0 && (long long)excl * H <= g0 && g0 < (long long)incl * H);
  if (hit == 0) return false;  // cannot happen: the lanes' ranges tile [0, T)
  const int ls = __builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit));
  long long S = __builtin_amdgcn_readlane(excl, ls);
  int b0 = -1, n0 = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int ck = __builtin_amdgcn_readlane(cnt[k], ls);
    const int qk = ck > 0 ? ck + A : 0;
    if (b0 < 0 && k < K) {
      if ((S + qk) * H > g0) {
        b0 = ls * K + k;
        n0 = ck;
      } else {
        S += qk;
      }
    }
  }
  if (b0 < 0 || n0 <= 0) return false;  // as above
  const long long off = g0 - S * H;
  const int q0 = n0 + A;  // cost of one group of sequence b0
  const int hg = (int)(off / q0);
  const int o = (int)(off - (long long)hg * q0);
  w.b = b0;
  w.nb = n0;
  w.h = hg * G + (wid - run * G);
  w.c = o > A ? o - A : 0;  // a start inside the group's overhead takes chunk 0
  w.P = S * H + (long long)hg * q0;
  w.pos = w.P + A + w.c;
  w.end = g1;
  if (w.pos >= w.end) return false;  // the run holds only overhead
  w.first = 1;
  w.wid = wid;
  w.run = run;
  w.G = G;
  w.A = A;
  w.nw = nw;
  w.T = T;
  piece_sequence(w.seq, a, kv_indptr, context_lengths, b0);
  return true;
}

// 4 consecutive head dims of an output row in the output dtype.
__device__ __forceinline__ void store_out4(void* out, int dtype, int64_t off, f32x4 v) {
  if (dtype == PA_DTYPE_F32) {
    *(f32x4*)((float*)out + off) = v;
  } else {
    const bool bf = dtype == PA_DTYPE_BF16;
    const uint32_t w0 = bf ? (f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16))
                           : (f32_to_f16_bits(v[0]) | (f32_to_f16_bits(v[1]) << 16));
    const uint32_t w1 = bf ? (f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16))
                           : (f32_to_f16_bits(v[2]) | (f32_to_f16_bits(v[3]) << 16));
    *(i32x2*)((uint16_t*)out + off) = i32x2{(int)w0, (int)w1};
  }
}

// Direct-to-LDS loads of one 32-token chunk of kv head ih (first token tb;
// page p0, and for 16-token pages p1 for tokens tb + 16 ..) into the stage
// at sk: keys (two 16-token halves kKHalf apart), values, and with
// per-token scales the chunk's 32 K then 32 V scales.  8 (+1) load
// instructions, each reading one page: a wave-uniform page base plus a
// per-lane offset.
template <bool PER_TOKEN, bool BS16>
__device__ __forceinline__ void dma_chunk(const pa_fp8_stream_args& a, const float* __restrict__ key_scale,
                                          const float* __restrict__ value_scale, LDS_AS unsigned char* sk, int ih,
                                          int tb, int p0, int p1, int lane) {
  const int bs = a.block_size;
  const int koff_lane = BS16 ? lane * 16 : (lane >> 4) * (bs * 16) + (lane & 15) * 16;
  const uint8_t* kbase = (const uint8_t*)a.key_cache + (int64_t)ih * a.stride_k_head;
  const uint8_t* vbase = (const uint8_t*)a.value_cache + (int64_t)ih * a.stride_v_head;
  LDS_AS unsigned char* sv = sk + kKBytes;
  if (BS16) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint8_t* kp = kbase + (int64_t)(hh ? p1 : p0) * a.stride_k_block;
      const uint8_t* vp = vbase + (int64_t)(hh ? p1 : p0) * a.stride_v_block;
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) lds_dma16(kp + koff_lane + q2 * 1024, sk + hh * kKHalf + q2 * 1024);
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) lds_dma16(vp + lane * 16 + q2 * 1024, sv + hh * 2048 + q2 * 1024);
    }
  } else {
    const int s0 = tb & (bs - 1);
    const uint8_t* kp = kbase + (int64_t)p0 * a.stride_k_block + s0 * 16;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2)
        lds_dma16(kp + hh * 256 + q2 * (4 * bs * 16) + koff_lane, sk + hh * kKHalf + q2 * 1024);
    if (a.trans_v) {
      const uint8_t* vp = vbase + (int64_t)p0 * a.stride_v_block + (s0 >> 4) * (kHead * 16);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2)
          lds_dma16(vp + hh * 2048 + q2 * 1024 + lane * 16, sv + hh * 2048 + q2 * 1024);
    } else {
      const uint8_t* vp = vbase + (int64_t)p0 * a.stride_v_block + s0;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2)
          lds_dma16(vp + hh * 16 + q2 * (64 * bs) + lane * bs, sv + hh * 2048 + q2 * 1024);
    }
  }
  if (PER_TOKEN) {
    LDS_AS unsigned char* ss = sv + kVBytes;
    if (lane < 16) {
      const int tt = (lane & 7) * 4;
      const int pg2 = BS16 ? (tt >= 16 ? p1 : p0) : p0;
      const int sidx = BS16 ? (tt & 15) : (tb & (bs - 1)) + tt;
      const float* base = (lane < 8 ? key_scale : value_scale) + (int64_t)ih * a.stride_ks_head;
      lds_dma16_cached(base + (int64_t)pg2 * a.stride_ks_block + sidx, ss);
    }
  }
}

// Zeroes the value bytes of tokens outside [lo, hi) in one 16-token half
// of a chunk's value image in LDS ([head dim][16 tokens], 128 rows of 16
// bytes starting at token th): lane l rewrites rows l and l + 64.
__device__ __forceinline__ void zero_stale_values(LDS_AS unsigned char* v, int th, int lo, int hi, int lane) {
  const int klo = pa_min(pa_max(lo - th, 0), 16);
  const int khi = pa_min(pa_max(hi - th, klo), 16);
  if (klo == 0 && khi == 16) return;
  i32x4 keep;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int l4 = pa_min(pa_max(klo - 4 * w, 0), 4), h4 = pa_min(pa_max(khi - 4 * w, l4), 4);
    const uint32_t below_hi = h4 >= 4 ? ~0u : (1u << (8 * h4)) - 1;
    const uint32_t below_lo = l4 >= 4 ? ~0u : (1u << (8 * l4)) - 1;
    keep[w] = (int)(below_hi & ~below_lo);
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    LDS_AS i32x4* row = (LDS_AS i32x4*)(v + (r * 64 + lane) * 16);
    *row = *row & keep;
  }
}

// A finished piece's result for query column e (lane (grp, e % 16) holds
// head dims 16 j + 4 grp .. + 3 in acc[j]): the output rows when the piece
// is a whole (sequence, kv head), else a partial row and its natural-log
// lse (work list: float32 rows target + qi; balanced split: bf16 row of
// partial id target).  m is the column's base-2 maximum, L its sum of 2^(pbias + l - m),
// and acc * vfin / L the normalised output.
template <bool WORKLIST>
__device__ __forceinline__ void store_piece(const pa_fp8_stream_args& a, void* __restrict__ output,
                                            float* __restrict__ part_out, float* __restrict__ part_lse,
                                            const Piece& p, const f32x4 (&acc)[8], float L, float m, float vfin,
                                            int e, int grp, float pbias = 8.0f) {
  const int gqa = a.query_group_size;
  const int eq = a.query_length * gqa;
  if (e >= eq) return;
  const int qi = e / gqa;
  const int g = e - qi * gqa;
  const int qh = p.h * gqa + g;
  const float sc = L > 0.0f ? vfin / L : 0.0f;
  if (p.target < 0) {
    const int64_t off = (int64_t)(p.orow + qi) * a.stride_out_tok + (int64_t)qh * a.stride_out_head + 4 * grp;
#pragma unroll
    for (int j = 0; j < 8; ++j) store_out4(output, a.output_dtype, off + 16 * j, acc[j] * sc);
  } else {
    int64_t po, pl;
    if (WORKLIST) {
      po = (int64_t)(p.target + qi) * a.stride_po_row + (int64_t)qh * kHead;
      pl = (int64_t)(p.target + qi) * a.stride_pl_row + qh;
    } else {
      pl = (int64_t)p.target * eq + e;
      po = pl * kHead;
    }
    if constexpr (WORKLIST) {
#pragma unroll
      for (int j = 0; j < 8; ++j) *(f32x4*)(part_out + po + 16 * j + 4 * grp) = acc[j] * sc;
    } else {
      // The balanced split's partial rows are internal to the call: bf16
      // halves their write and merge traffic (about 2^-9 relative, twice).
      uint16_t* pb = (uint16_t*)part_out;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f32x4 v = acc[j] * sc;
        *(uint2*)(pb + po + 16 * j + 4 * grp) = uint2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16),
                                                      f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
      }
    }
    if (grp == 0) part_lse[pl] = L > 0.0f ? kLn2 * (m + __builtin_amdgcn_logf(L) - pbias) : kNegInf;
  }
}

// Each wave walks its pieces through a private LDS ring (2 stages of one
// 32-token chunk each) plus two query images (the current piece's and the
// next one's: a piece's query rows are loaded by direct-to-LDS DMA just
// before its first chunk, so they ride the same in-order vmcnt pipeline).
// One 16-column query block (query_length * gqa <= 16).
template <bool PER_TOKEN, bool BS16, bool WORKLIST, int NQ>
__global__ __launch_bounds__(64 * stream_waves(NQ)) void pa_fp8_stream_kernel(
    const pa_fp8_stream_args a, const int32_t* __restrict__ block_tables, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ context_lengths, const float* __restrict__ key_scale,
    const float* __restrict__ value_scale, const int32_t* __restrict__ work_indptr,
    const int32_t* __restrict__ work_info, const int32_t* __restrict__ partition_indptr,
    int32_t* __restrict__ segdesc, float* __restrict__ part_out, float* __restrict__ part_lse,
    void* __restrict__ output) {
  // Every store goes through a restrict pointer, so the loads of the page
  // lists, lengths and work list stay scalar (SMEM) loads inside the walk.
  constexpr int NCG = 1;
  constexpr int kStageBytes = kKBytes + kVBytes + (PER_TOKEN ? kScaleBytes : 0);
  constexpr int kQBytes = NQ * 1024;  // NQ * 4 query columns x 128 dims x 2 B
  constexpr int kWaveBytes = kStages * kStageBytes + 2 * kQBytes;
  constexpr int kLoadsPerChunk = 8 + (PER_TOKEN ? 1 : 0);
  static_assert(kStages == 2, "the streaming pipeline keeps one chunk in flight");
  __shared__ __attribute__((aligned(16))) unsigned char smem[stream_waves(NQ) * kWaveBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4;
  const int c16 = lane & 15;
  const int wid = blockIdx.x * stream_waves(NQ) + wave;
  const int ql = a.query_length;
  const int gqa = a.query_group_size;
  const int eq = ql * gqa;
  const int bs = a.block_size;
  const int bs_shift = BS16 ? 4 : __builtin_ctz((unsigned)bs);
  const int nblocks = a.num_blocks;

  // ---------------- this wave's walk ----------------
  using Walk = typename std::conditional<WORKLIST, WorklistWalk, BalancedWalk>::type;
  Walk walk;
  if constexpr (WORKLIST) {
    if (wid >= a.num_workers) return;
    walk.idx = ld_uniform(work_indptr, wid);
    walk.end = ld_uniform(work_indptr, wid + 1);
  } else {
    const int G = balanced_group(a.num_kv_heads, a.num_workers, eq);
    if (!balanced_start(walk, a, kv_indptr, context_lengths, wid, lane, G, kStreamPieceCost)) return;
  }
  auto next_piece = [&](Piece& p) -> bool {
    if constexpr (WORKLIST)
      return walk.next(p, a, kv_indptr, context_lengths, work_info, partition_indptr);
    else
      return walk.next(p, a, kv_indptr, context_lengths);
  };

  LDS_AS unsigned char* ring = (LDS_AS unsigned char*)smem + wave * kWaveBytes;
  LDS_AS unsigned char* qimg = ring + kStages * kStageBytes;
  auto clamp_page = [&](int p) -> int {
    pa_note(p < 0 || p >= nblocks, PA_VIOLATION_PAGE);
    p = p < 0 ? 0 : p;
    return p < nblocks ? p : nblocks - 1;
  };

  // ---------------- piece window ----------------
  // `cur` is being computed, `nxt` follows.  The issue side, one chunk
  // ahead, never goes past `nxt` (it pauses instead), so one walker serves
  // both sides and the scalar state stays in SGPRs.
  Piece cur, nxt;
  bool has_cur = next_piece(cur);
  if (!has_cur) return;
  bool has_nxt = next_piece(nxt);

  // Issue cursor: next chunk at token itb, irem chunks left in its piece
  // (nxt when iw, else cur); ifirst: that chunk opens the piece.
  int itb = 0, ih = 0, ilast = 0, irem = 0, iw = 0, iorow = 0;
  int64_t ibt = 0;
  bool iok = false, ifirst = false;
  int np0 = 0, np1 = 0;  // page ids of the next chunk (prefetched)
  auto fetch_pages = [&]() {
    const int lp0 = itb >> bs_shift;
    np0 = ld_uniform(block_tables, ibt + pa_min(lp0, ilast));
    np1 = BS16 ? ld_uniform(block_tables, ibt + pa_min(lp0 + 1, ilast)) : np0;
  };
  auto issue_enter = [&](const Piece& p, int which) {
    itb = p.tb0;
    ih = p.h;
    ibt = p.bt_off;
    ilast = p.last_page;
    irem = p.n;
    iorow = p.orow;
    iw = which;
    iok = true;
    ifirst = true;
    fetch_pages();
  };
  if (cur.n > 0)
    issue_enter(cur, 0);
  else if (has_nxt && nxt.n > 0)
    issue_enter(nxt, 1);

  int iq = 0;  // query image the next piece's rows go to
  // Issues the next chunk (and, first in a piece, the piece's query rows)
  // into stage st; returns whether query rows were issued.
  auto issue_chunk = [&](int st) -> bool {
    const bool q = ifirst;
    if (ifirst) {
      // Query rows of columns 4i + lane/16 (clamped to a real column).
      LDS_AS unsigned char* qd = qimg + iq * kQBytes;
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int e = pa_min(4 * i + (lane >> 4), eq - 1);
        const int qi = e / gqa;
        const int g = e - qi * gqa;
        const unsigned char* src = (const unsigned char*)a.query +
                                   2 * ((int64_t)(iorow + qi) * a.stride_q_tok +
                                        (int64_t)(ih * gqa + g) * a.stride_q_head) +
                                   (lane & 15) * 16;
        lds_dma16_cached(src, qd + i * 1024);
      }
      iq ^= 1;
      ifirst = false;
    }
    const int p0 = clamp_page(np0);
    const int p1 = BS16 ? clamp_page(np1) : p0;
    dma_chunk<PER_TOKEN, BS16>(a, key_scale, value_scale, ring + st * kStageBytes, ih, itb, p0, p1, lane);
    itb += kChunk;
    if (--irem > 0)
      fetch_pages();
    else if (iw == 0 && has_nxt && nxt.n > 0)
      issue_enter(nxt, 1);
    else
      iok = false;
    return q;
  };

  // ---------------- compute side ----------------
  const float k_tensor_scale = PER_TOKEN ? 1.0f : key_scale[0];
  const float v_tensor_scale = PER_TOKEN ? 1.0f : value_scale[0];
  const float logit_scale = a.softmax_scale * kLog2e * k_tensor_scale;
  const int krow = (c16 >> 3) * kKHalf + (8 * ((c16 >> 2) & 1) + (c16 & 3)) * 16;
  WaveState<NCG> st;
  st.reset();
  QueryTile<NCG> qt;
  int cq = 0;      // query image of the next piece to compute
  int gc = 0;      // chunks computed (stage = gc % 2)
  int issued = 0;  // chunks issued
  if (iok) {
    issue_chunk(0);
    issued = 1;
  }
  while (has_cur) {
    for (int k = 0; k < cur.n; ++k) {
      const int stg = gc & 1;
      if (issued == gc) {
        // The issue side paused past an empty piece: chunk gc goes now.
        issue_chunk(stg);
        ++issued;
      }
      if (iok) {
        // In order: [chunk gc] ... [query rows?] [chunk gc + 1]; wait for
        // everything up to chunk gc.
        ++issued;
        if (issue_chunk(stg ^ 1))
          __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk + NQ));
        else
          __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk));
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      ++gc;
      if (k == 0) {
        // The piece's query rows arrived before its first chunk.
        const LDS_AS unsigned char* qs = qimg + cq * kQBytes + c16 * 256;
        cq ^= 1;
        i32x4 qraw[1][4];
        if (c16 < eq) {
          qraw[0][0] = *(const LDS_AS i32x4*)(qs + 32 * grp);
          qraw[0][1] = *(const LDS_AS i32x4*)(qs + 32 * grp + 16);
          qraw[0][2] = *(const LDS_AS i32x4*)(qs + 32 * (grp + 4));
          qraw[0][3] = *(const LDS_AS i32x4*)(qs + 32 * (grp + 4) + 16);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) qraw[0][i] = i32x4{0, 0, 0, 0};
        }
        prepare_query<NCG>(qt, qraw, a.query_dtype, logit_scale, cur.ctx, ql, gqa, a.sliding_window, c16);
      }
      compute_chunk<NCG, PER_TOKEN>(st, qt, ring + stg * kStageBytes, krow, grp, c16, cur.tb0 + k * kChunk);
    }
    // ---- the piece is complete: output row or partial ----
    const float vfin = PER_TOKEN ? st.vsmax : v_tensor_scale;
    store_piece<WORKLIST>(a, output, part_out, part_lse, cur, st.acc[0], sum_over_groups(st.lsum[0]), st.m2[0],
                          vfin, c16, grp);
    if (!WORKLIST && cur.desc_cnt > 0 && lane == 0)
      *(i32x2*)(segdesc + 2 * ((int64_t)cur.b * a.num_kv_heads + cur.h)) = i32x2{cur.target, cur.desc_cnt};
    st.reset();
    // ---- move the window ----
    cur = nxt;
    has_cur = has_nxt;
    has_nxt = has_cur && next_piece(nxt);
    if (iw == 1) iw = 0;
    if (!iok && has_nxt && nxt.n > 0) issue_enter(nxt, 1);
  }
}

// ============================================================================
// Work-list decode: workgroups over consecutive bins
// ============================================================================
//
// The reference plans its persistent route over CU * 3 bins and launches one
// workgroup per bin (kernels/pa_decode_fp8.py:1766-1771, 3144-3184).  Here a
// workgroup of W waves takes a run of consecutive bins -- one per CU: every
// CU's three bins, whose works are contiguous in the work list -- and
// treats their works, laid end to end, as one sequence of N chunks: wave r
// takes chunks [rN/W, (r+1)N/W).  A work cut between waves is merged inside
// the workgroup once every wave is done: each wave leaves the state of its
// first piece (when cut) and of its last piece (when cut) in its LDS ring,
// and the wave that holds a cut work's last chunk folds the others' states
// into it and writes the work's result.  Eight waves of two 8.3 KiB stages
// each (17 KiB with per-token scales) fill one CU: two waves per SIMD, the
// same occupancy as the balanced split.
#ifndef PA_FP8_BIN_WAVES
#define PA_FP8_BIN_WAVES 8
#endif
constexpr int kBinWaves = PA_FP8_BIN_WAVES;

// Walk of this wave's run [r0, r1) of its workgroup's chunk sequence: the
// works of the workgroup's bins in order, each clipped to the run.  A work
// with no chunk belongs to the wave whose (non-empty) run contains its
// position, or the last wave when it sits at the end.
struct BinWalk {
  WorklistWalk w;
  int pos, r0, r1;
  bool last;
  __device__ __forceinline__ bool next(Piece& p, const pa_fp8_stream_args& a, const int32_t* kv_indptr,
                                       const int32_t* context_lengths, const int32_t* work_info,
                                       const int32_t* partition_indptr) {
    while (w.next(p, a, kv_indptr, context_lengths, work_info, partition_indptr)) {
      const int s = pos, e = pos + p.n;
      pos = e;
      if (s > r1) {
        w.idx = w.end;
        return false;
      }
      if (p.n == 0) {
        if ((s >= r0 && s < r1) || (last && s == r1)) return true;
        continue;
      }
      const int c0 = pa_max(s, r0), c1 = pa_min(e, r1);
      if (c1 <= c0) continue;
      p.tb0 += (c0 - s) * kChunk;
      p.n = c1 - c0;
      p.cut = (c0 > s ? 1 : 0) | (c1 < e ? 2 : 0);
      p.wstart = s;
      return true;
    }
    return false;
  }
};

// Merge slot of a cut piece in LDS: value-unit accumulators [128 head dims]
// [16 columns], then the columns' base-2 maxima and sums.
constexpr int kSlotAcc = kHead * 16 * 4;
constexpr int kSlotBytes = kSlotAcc + 2 * 16 * 4;

__device__ __forceinline__ void slot_write(LDS_AS unsigned char* slot, const f32x4 (&acc)[8], float m, float L,
                                           int grp, int c16) {
  LDS_AS float* f = (LDS_AS float*)slot;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) f[(16 * j + 4 * grp + i) * 16 + c16] = acc[j][i];
  if (grp == 0) {
    f[kSlotAcc / 4 + c16] = m;
    f[kSlotAcc / 4 + 16 + c16] = L;
  }
}

template <bool PER_TOKEN, bool BS16>
__global__ __launch_bounds__(64 * kBinWaves) void pa_fp8_bin_kernel(
    const pa_fp8_stream_args a, const int32_t* __restrict__ block_tables, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ context_lengths, const float* __restrict__ key_scale,
    const float* __restrict__ value_scale, const int32_t* __restrict__ work_indptr,
    const int32_t* __restrict__ work_info, const int32_t* __restrict__ partition_indptr,
    float* __restrict__ part_out, float* __restrict__ part_lse, void* __restrict__ output) {
  constexpr int W = kBinWaves;
  constexpr int kStageBytes = kKBytes + kVBytes + (PER_TOKEN ? kScaleBytes : 0);
  constexpr int kWaveBytes = 2 * kStageBytes;
  constexpr int kLoadsPerChunk = 8 + (PER_TOKEN ? 1 : 0);
  constexpr int kQLoads = 4;  // query row loads per lane
  static_assert(2 * kSlotBytes <= kWaveBytes, "a wave's two merge slots fit in its ring");
  __shared__ __attribute__((aligned(16))) unsigned char smem[W * kWaveBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4;
  const int c16 = lane & 15;
  // This workgroup's bins [bin0, bin1): an equal share of the plan's.
  const int bin0 = (int)((int64_t)blockIdx.x * a.num_workers / gridDim.x);
  const int bin1 = (int)((int64_t)(blockIdx.x + 1) * a.num_workers / gridDim.x);
  const int ql = a.query_length;
  const int gqa = a.query_group_size;
  const int eq = ql * gqa;
  const int bs = a.block_size;
  const int bs_shift = BS16 ? 4 : __builtin_ctz((unsigned)bs);
  const int nblocks = a.num_blocks;
  const int w0 = ld_uniform(work_indptr, bin0), w1 = ld_uniform(work_indptr, bin1);

  // ---------------- the bins' chunk count and this wave's run ----------------
  // One work per lane: its chunk count (vector loads of the work, the
  // sequence's length and first partition), 64 works per pass.
  auto chunks_of = [&](int wk) -> int {
    if (wk >= w1) return 0;
    const int b = work_info[8 * (int64_t)wk];
    const int kv0 = work_info[8 * (int64_t)wk + 4], kv1 = work_info[8 * (int64_t)wk + 5];
    const int ctx = context_lengths[b];
    const int pb = partition_indptr[b];
    int lo_all, hi_all, u;
    pa_plan_visible(ctx, 0, ql, a.sliding_window, &lo_all, &u);
    pa_plan_visible(ctx, ql - 1, ql, a.sliding_window, &u, &hi_all);
    const int row_len = kv_indptr ? kv_indptr[b + 1] - kv_indptr[b] : a.max_blocks_per_seq;
    const int last_page = pa_min(pa_cdiv(ctx, bs) - 1, row_len - 1);
    int tb0, n;
    work_chunks(ctx, lo_all, hi_all, last_page, pb, kv0, kv1, tb0, n);
    return n;
  };
  auto wave_incl_scan = [&](int v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, 64);
      if (lane >= o) v += t;
    }
    return v;
  };
  const int n_first = chunks_of(w0 + lane);
  int N = __builtin_amdgcn_readlane(wave_incl_scan(n_first), 63);
  for (int base = w0 + 64; base < w1; base += 64) N += __builtin_amdgcn_readlane(wave_incl_scan(chunks_of(base + lane)), 63);
  const int R0 = (int)((int64_t)wave * N / W), R1 = (int)((int64_t)(wave + 1) * N / W);
  // First work of the run: the first that ends past R0, or an empty one at
  // R0 or later.
  int wstart_idx = w1, spos = N;
  {
    int pos = 0;
    for (int base = w0; base < w1; base += 64) {
      const int n = base == w0 ? n_first : chunks_of(base + lane);
      const int incl = wave_incl_scan(n);
      const int s = pos + incl - n, e = pos + incl;
      const uint64_t hit = __ballot(base + lane < w1 && (e > R0 || (n == 0 && s >= R0)));
      if (hit) {
        const int l = __builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit));
        wstart_idx = base + l;
        spos = __builtin_amdgcn_readlane(s, l);
        break;
      }
      pos += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  BinWalk walk;
  walk.w.idx = wstart_idx;
  walk.w.end = w1;
  walk.pos = spos;
  walk.r0 = R0;
  walk.r1 = R1;
  walk.last = wave == W - 1;
  auto next_piece = [&](Piece& p) -> bool {
    return walk.next(p, a, kv_indptr, context_lengths, work_info, partition_indptr);
  };

  LDS_AS unsigned char* ring = (LDS_AS unsigned char*)smem + wave * kWaveBytes;
  auto clamp_page = [&](int p) -> int {
    pa_note(p < 0 || p >= nblocks, PA_VIOLATION_PAGE);
    p = p < 0 ? 0 : p;
    return p < nblocks ? p : nblocks - 1;
  };

  // ---------------- piece window and issue cursor (as the stream kernel) ----------------
  Piece cur, nxt;
  bool has_cur = next_piece(cur);
  bool has_nxt = has_cur && next_piece(nxt);
  int itb = 0, ih = 0, ilast = 0, irem = 0, iw = 0, iorow = 0;
  int64_t ibt = 0;
  bool iok = false, ifirst = false;
  int np0 = 0, np1 = 0;
  auto fetch_pages = [&]() {
    const int lp0 = itb >> bs_shift;
    np0 = ld_uniform(block_tables, ibt + pa_min(lp0, ilast));
    np1 = BS16 ? ld_uniform(block_tables, ibt + pa_min(lp0 + 1, ilast)) : np0;
  };
  auto issue_enter = [&](const Piece& p, int which) {
    itb = p.tb0;
    ih = p.h;
    ibt = p.bt_off;
    ilast = p.last_page;
    irem = p.n;
    iorow = p.orow;
    iw = which;
    iok = true;
    ifirst = true;
    fetch_pages();
  };
  if (has_cur && cur.n > 0)
    issue_enter(cur, 0);
  else if (has_nxt && nxt.n > 0)
    issue_enter(nxt, 1);

  // Query rows of the next piece (lane (grp, c16): column c16's head dims
  // 16 grp .. +15 and 16 (grp + 4) .. +15), loaded into registers just
  // before the piece's first chunk, so they retire before it.
  i32x4 qn[4];
  auto issue_chunk = [&](int st) -> bool {
    const bool q = ifirst;
    if (ifirst) {
      const int e = pa_min(c16, eq - 1);
      const int qi = e / gqa;
      const int g = e - qi * gqa;
      const uint16_t* qp = (const uint16_t*)a.query + (int64_t)(iorow + qi) * a.stride_q_tok +
                           (int64_t)(ih * gqa + g) * a.stride_q_head;
      qn[0] = *(const i32x4*)(qp + 16 * grp);
      qn[1] = *(const i32x4*)(qp + 16 * grp + 8);
      qn[2] = *(const i32x4*)(qp + 16 * (grp + 4));
      qn[3] = *(const i32x4*)(qp + 16 * (grp + 4) + 8);
      ifirst = false;
    }
    dma_chunk<PER_TOKEN, BS16>(a, key_scale, value_scale, ring + st * kStageBytes, ih, itb, clamp_page(np0),
                               BS16 ? clamp_page(np1) : 0, lane);
    itb += kChunk;
    if (--irem > 0)
      fetch_pages();
    else if (iw == 0 && has_nxt && nxt.n > 0)
      issue_enter(nxt, 1);
    else
      iok = false;
    return q;
  };

  // ---------------- compute side ----------------
  const float k_tensor_scale = PER_TOKEN ? 1.0f : key_scale[0];
  const float v_tensor_scale = PER_TOKEN ? 1.0f : value_scale[0];
  const float logit_scale = a.softmax_scale * kLog2e * k_tensor_scale;
  const int krow = (c16 >> 3) * kKHalf + (8 * ((c16 >> 2) & 1) + (c16 & 3)) * 16;
  WaveState<1> st;
  st.reset();
  QueryTile<1> qt;
  // The wave's first piece with chunks, when cut: its state waits in
  // registers until the ring is free (value units).
  f32x4 accA[8];
  float mA = kNegInf, LA = 0.0f;
  bool hasA = false, hasB = false;
  Piece pA;
  pA.cut = 0;
  pA.wstart = 0;
  bool first_piece = true;
  int gc = 0, issued = 0;
  if (iok) {
    issue_chunk(0);
    issued = 1;
  }
  while (has_cur) {
    for (int k = 0; k < cur.n; ++k) {
      const int stg = gc & 1;
      if (issued == gc) {
        issue_chunk(stg);
        ++issued;
      }
      if (k == 0) {
        // [query rows][chunk gc] are the newest loads: wait for the rows
        // and turn them into operands before the next issue reuses qn.
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk));
        i32x4 qraw[1][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qraw[0][i] = c16 < eq ? qn[i] : i32x4{0, 0, 0, 0};
        prepare_query<1>(qt, qraw, a.query_dtype, logit_scale, cur.ctx, ql, gqa, a.sliding_window, c16);
      }
      if (iok) {
        ++issued;
        if (issue_chunk(stg ^ 1))
          __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk + kQLoads));
        else
          __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk));
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      ++gc;
      compute_chunk<1, PER_TOKEN>(st, qt, ring + stg * kStageBytes, krow, grp, c16, cur.tb0 + k * kChunk);
    }
    // ---- the piece is complete ----
    const float vfin = PER_TOKEN ? st.vsmax : v_tensor_scale;
    const float L = sum_over_groups(st.lsum[0]);
    if (cur.cut == 0) {
      store_piece<true>(a, output, part_out, part_lse, cur, st.acc[0], L, st.m2[0], vfin, c16, grp);
    } else if (first_piece) {
#pragma unroll
      for (int j = 0; j < 8; ++j) accA[j] = st.acc[0][j] * vfin;
      mA = st.m2[0];
      LA = L;
      pA = cur;
      hasA = true;
    } else {
      // A cut piece that is not the wave's first ends its run: nothing is
      // in flight any more, so its state goes to the ring's second slot.
      f32x4 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = st.acc[0][j] * vfin;
      slot_write(ring + kSlotBytes, acc, st.m2[0], L, grp, c16);
      hasB = true;
    }
    // An empty work (no chunk) is never cut and does not count as the
    // wave's first piece: a cut piece right after it starts the run.
    if (cur.n > 0) first_piece = false;
    st.reset();
    cur = nxt;
    has_cur = has_nxt;
    has_nxt = has_cur && next_piece(nxt);
    if (iw == 1) iw = 0;
    if (!iok && has_nxt && nxt.n > 0) issue_enter(nxt, 1);
  }
  (void)hasB;

  // ---------------- cut works: merge across the waves ----------------
  // Every load of this wave has retired (its last chunk waited for all).
  if (hasA) slot_write(ring, accA, mA, LA, grp, c16);
  __syncthreads();
  // The wave holding a cut work's last chunk (its first piece, cut at the
  // start, not at the end) merges the work: wave r's piece of it sits in
  // r's first slot when r's run starts inside the work, else (the work's
  // first wave) in r's second slot.
  if (hasA && pA.cut == 1) {
    const int s = pA.wstart;
    float M = kNegInf;
#pragma unroll
    for (int r = 0; r < W; ++r) {
      const int Rr = (int)((int64_t)r * N / W), Rn = (int)((int64_t)(r + 1) * N / W);
      if (r > wave || Rn <= s || Rn <= Rr) continue;
      const LDS_AS float* f = (const LDS_AS float*)((LDS_AS unsigned char*)smem + r * kWaveBytes +
                                                     (Rr >= s ? 0 : kSlotBytes));
      M = fmaxf(M, f[kSlotAcc / 4 + c16]);
    }
    const float Mu = M == kNegInf ? 0.0f : M;
    float L = 0.0f;
    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < W; ++r) {
      const int Rr = (int)((int64_t)r * N / W), Rn = (int)((int64_t)(r + 1) * N / W);
      if (r > wave || Rn <= s || Rn <= Rr) continue;
      const LDS_AS float* f = (const LDS_AS float*)((LDS_AS unsigned char*)smem + r * kWaveBytes +
                                                     (Rr >= s ? 0 : kSlotBytes));
      const float fr = __builtin_amdgcn_exp2f(f[kSlotAcc / 4 + c16] - Mu);
      L += f[kSlotAcc / 4 + 16 + c16] * fr;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] += f[(16 * j + 4 * grp + i) * 16 + c16] * fr;
    }
    store_piece<true>(a, output, part_out, part_lse, pA, acc, L, M, 1.0f, c16, grp);
  }
}

// Cooperative column-split decode for 17..64 query columns per kv head
// (two to four 16-column blocks).  A workgroup has one wave per column
// block; all of its waves read the same 32-token chunks from one shared
// LDS ring of chunk slots, each wave DMAing an equal share of every chunk
// (its last wave also the chunk's per-token scales).  A wave holds only its
// own block's accumulators and query operands, and a chunk is fetched from
// HBM once for all blocks.  Work comes from the same walks as
// pa_fp8_stream_kernel, at workgroup granularity (a run of the balanced
// split, or one bin of the work list); every wave writes its own columns of
// each piece.  A piece's query rows are loaded into registers during the
// previous piece's last unit.
//
// The workgroup computes its chunks in units: one wait, one barrier and
// one online-softmax step per unit, and a value product on the K = 128 MFMA
// (unit_softmax_pv).  The ring has S chunk slots; while a unit is computed
// the next S - U chunks are in flight, and after its barrier the ring is
// refilled up to S chunks past its start, which covers the next unit when
// S >= 2 U: four waves of the balanced split run units of four chunks over
// nine slots (77 KiB), two workgroups per CU; otherwise units of two over
// six slots, three workgroups per CU (the work list then keeps the
// reference's CU * 3 bins resident).
constexpr int kFarToken = 1 << 30;  // first token of a unit's missing chunk

constexpr int coop_slots(int nw, bool worklist) { return nw == 4 && !worklist ? 9 : 6; }
constexpr int coop_unit(int nw, bool worklist) { return nw == 4 && !worklist ? 4 : 2; }
constexpr int coop_wgs_per_cu(int nw, bool worklist) { return nw == 4 && !worklist ? 2 : 3; }
// Waves per SIMD those workgroups need (a workgroup's waves sit on distinct
// SIMDs): the occupancy the kernel is compiled for.
constexpr int coop_waves_per_simd(int nw, bool worklist) { return (coop_wgs_per_cu(nw, worklist) * nw + 3) / 4; }

template <int NW, bool PER_TOKEN, bool BS16, bool WORKLIST>
__global__ __launch_bounds__(64 * NW, coop_waves_per_simd(NW, WORKLIST)) void pa_fp8_coop_kernel(
    const pa_fp8_stream_args a, const int32_t* __restrict__ block_tables, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ context_lengths, const float* __restrict__ key_scale,
    const float* __restrict__ value_scale, const int32_t* __restrict__ work_indptr,
    const int32_t* __restrict__ work_info, const int32_t* __restrict__ partition_indptr,
    int32_t* __restrict__ segdesc, float* __restrict__ part_out, float* __restrict__ part_lse,
    void* __restrict__ output) {
  static_assert(NW == 2 || NW == 4, "two or four waves share a chunk");
  constexpr int S = coop_slots(NW, WORKLIST);
  constexpr int U = coop_unit(NW, WORKLIST);  // chunks per unit
  static_assert(S >= 2 * U, "the refill after a unit's barrier covers the next unit");
  // Chunk slot: keys, values, per-token K then V scales.
  constexpr int kSlotBytes = kKBytes + kVBytes + (PER_TOKEN ? kScaleBytes : 0);
  // Chunk j of the launch is loaded whole by wave j % NW: 8 one-KiB key and
  // value loads and, with per-token scales, one scale load.
  constexpr int kChunkLoads = 8 + (PER_TOKEN ? 1 : 0);
  __shared__ __attribute__((aligned(16))) unsigned char smem[S * kSlotBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4;
  const int c16 = lane & 15;
  const int wid = blockIdx.x;
  const int ql = a.query_length;
  const int gqa = a.query_group_size;
  const int eq = ql * gqa;
  const int bs = a.block_size;
  const int bs_shift = BS16 ? 4 : __builtin_ctz((unsigned)bs);
  const int nblocks = a.num_blocks;
  const int e = wave * 16 + c16;  // this lane's query column

  using Walk = typename std::conditional<WORKLIST, WorklistWalk, BalancedWalk>::type;
  Walk walk;
  if constexpr (WORKLIST) {
    if (wid >= a.num_workers) return;
    walk.idx = ld_uniform(work_indptr, wid);
    walk.end = ld_uniform(work_indptr, wid + 1);
  } else {
    if (!balanced_start(walk, a, kv_indptr, context_lengths, wid, lane, 1, kCoopPieceCost)) return;
  }
  auto next_piece = [&](Piece& p) -> bool {
    if constexpr (WORKLIST)
      return walk.next(p, a, kv_indptr, context_lengths, work_info, partition_indptr);
    else
      return walk.next(p, a, kv_indptr, context_lengths);
  };
  const int koff_lane = BS16 ? lane * 16 : (lane >> 4) * (bs * 16) + (lane & 15) * 16;
  const int voff_plain = lane * bs;
  auto clamp_page = [&](int p) -> int {
    pa_note(p < 0 || p >= nblocks, PA_VIOLATION_PAGE);
    p = p < 0 ? 0 : p;
    return p < nblocks ? p : nblocks - 1;
  };

  // ---------------- piece window ----------------
  // The walk is seen through two pieces: `cur` is being computed, `nxt`
  // follows.  The issue side runs ahead of the compute side but never past
  // `nxt`: once it has issued all of `nxt` it pauses until the compute side
  // moves on.  One walker serves both sides, which keeps the scalar state
  // small enough to stay in SGPRs.
  Piece cur, nxt;
  bool has_cur = next_piece(cur);
  if (!has_cur) return;
  bool has_nxt = next_piece(nxt);

  // Issue cursor: next chunk at token itb of kv head ih, irem chunks left
  // in its piece, which is nxt when iw (else cur).
  int itb = 0, ih = 0, ilast = 0, irem = 0, iw = 0;
  int ipos = 0;  // position of the next chunk in its piece
  int64_t ibt = 0;
  // A chunk's eight 1 KiB loads, fixed for the launch: load i is keys for
  // i < 4 (else values), 16-token half hh = (i >> 1) & 1, 1 KiB piece
  // q2 = i & 1.  The wave that loads a chunk computes its key and value page
  // addresses once (page base + in-page offset) and adds per-lane constants.
  // In-page offset of a chunk at page slot s0: keys s0 << 4, values
  // (s0 >> vsh1) << vsh2.
  const int vsh1 = a.trans_v ? 4 : 0;
  const int vsh2 = a.trans_v ? 11 : 0;
  int loff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool ki = i < 4;
    const int hh = (i >> 1) & 1, q2 = i & 1;
    if (BS16)
      loff[i] = (ki ? koff_lane : lane * 16) + q2 * 1024;
    else if (ki)
      loff[i] = hh * 256 + q2 * (4 * bs * 16) + koff_lane;
    else if (a.trans_v)
      loff[i] = hh * 2048 + q2 * 1024 + lane * 16;
    else
      loff[i] = hh * 16 + q2 * (64 * bs) + voff_plain;
  }
  const uint8_t* ikb = (const uint8_t*)a.key_cache;    // + ih * stride_k_head
  const uint8_t* ivb = (const uint8_t*)a.value_cache;  // + ih * stride_v_head
  // Page strides fit 31 bits (checked on the host), so a page's offset is
  // one unsigned 32 x 32 -> 64-bit product.
  const uint32_t ksb = (uint32_t)a.stride_k_block;
  const uint32_t vsb = (uint32_t)a.stride_v_block;
  const uint32_t ssb = (uint32_t)a.stride_ks_block;
  // a scale load's lane: its scale row base for the piece's kv head
  const int tt = (lane & 7) * 4;
  const float* const sbase0 = ((lane & 8) ? value_scale : key_scale) + (BS16 ? (tt & 15) : tt);
  const float* sbase = sbase0;
  bool iok = false;
  int np0 = 0, np1 = 0;  // page ids of the next chunk (prefetched)
  int nlp = -1;          // logical page of np0 (pages of 64 tokens and more hold several chunks)
  auto fetch_pages = [&]() {
    const int lp0 = pa_min(itb >> bs_shift, ilast);
    if (BS16) {
      np0 = ld_uniform(block_tables, ibt + lp0);
      np1 = ld_uniform(block_tables, ibt + pa_min(lp0 + 1, ilast));
    } else if (lp0 != nlp) {
      np0 = ld_uniform(block_tables, ibt + lp0);
      np1 = np0;
      nlp = lp0;
    }
  };
  auto issue_enter = [&](const Piece& p, int which) {
    itb = p.tb0;
    ih = p.h;
    ibt = p.bt_off;
    ilast = p.last_page;
    irem = p.n;
    ipos = 0;
    iw = which;
    iok = true;
    ikb = (const uint8_t*)a.key_cache + (int64_t)ih * a.stride_k_head;
    ivb = (const uint8_t*)a.value_cache + (int64_t)ih * a.stride_v_head;
    if (PER_TOKEN) sbase = sbase0 + (int64_t)ih * a.stride_ks_head;
    nlp = -1;
    fetch_pages();
  };
  if (cur.n > 0)
    issue_enter(cur, 0);
  else if (has_nxt && nxt.n > 0)
    issue_enter(nxt, 1);

  // This wave's share of the next chunk (and, for the scale wave, the
  // chunk's 32 K and 32 V scales: lane l < 16 carries 4 tokens' scales, keys
  // or values by bit 3) into chunk slot `issued % S` (islot).
  int issued = 0;    // chunks this workgroup has issued
  int islot = 0;     // their next slot: issued % S
  auto issue_next = [&]() {
    if (issued % NW == wave) {  // workgroup-uniform: every wave walks the same chunks
      const int p0 = clamp_page(np0);
      const int p1 = BS16 ? clamp_page(np1) : p0;
      const int s0 = itb & (bs - 1);
      const int64_t kin = BS16 ? 0 : (int64_t)(s0 << 4);
      const int64_t vin = BS16 ? 0 : (int64_t)((s0 >> vsh1) << vsh2);
      LDS_AS unsigned char* sk = (LDS_AS unsigned char*)smem + islot * kSlotBytes;
      const uint8_t* k0 = ikb + (uint64_t)(uint32_t)p0 * ksb + kin;
      const uint8_t* k1 = BS16 ? ikb + (uint64_t)(uint32_t)p1 * ksb : k0;
      const uint8_t* v0 = ivb + (uint64_t)(uint32_t)p0 * vsb + vin;
      const uint8_t* v1 = BS16 ? ivb + (uint64_t)(uint32_t)p1 * vsb : v0;
      // Four-chunk units: key token r of the chunk at unit position c goes to
      // row r ^ 4c of its 16-token half (lane l of a key load fetches token
      // (l & 15) ^ 4c), so the QK reads -- four tokens of each of the unit's
      // four chunks per 16 lanes -- hit 16 different rows instead of the same
      // banks of four slots.
      const int kswz = U == 4 ? (ipos & 3) << 6 : 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int hh = (i >> 1) & 1, q2 = i & 1;
        const uint8_t* src =
            i < 4 ? ((BS16 && hh) ? k1 : k0) + (loff[i] ^ kswz) : ((BS16 && hh) ? v1 : v0) + loff[i];
        const int dst = (i < 4 ? hh * kKHalf : kKBytes + hh * 2048) + q2 * 1024;
        lds_dma16(src, sk + dst);
      }
      if (PER_TOKEN && lane < 16) {
        const int pg = BS16 ? (tt >= 16 ? p1 : p0) : p0;
        const int sidx = BS16 ? 0 : (itb & (bs - 1));
        lds_dma16_cached(sbase + (uint64_t)(uint32_t)pg * ssb + sidx, sk + kKBytes + kVBytes);
      }
    }
    islot = islot + 1 == S ? 0 : islot + 1;
    ++issued;
    ++ipos;
    itb += kChunk;
    if (--irem > 0)
      fetch_pages();
    else if (iw == 0 && has_nxt && nxt.n > 0)
      issue_enter(nxt, 1);
    else
      iok = false;
  };

  // ---------------- query rows of a piece (registers) ----------------
  i32x4 qraw[1][4];
  auto load_query = [&](const Piece& p) {
    if (e < eq) {
      const int qi = e / gqa;
      const int g = e - qi * gqa;
      const uint16_t* qp = (const uint16_t*)a.query + (int64_t)(p.orow + qi) * a.stride_q_tok +
                           (int64_t)(p.h * gqa + g) * a.stride_q_head;
      qraw[0][0] = *(const i32x4*)(qp + 16 * grp);
      qraw[0][1] = *(const i32x4*)(qp + 16 * grp + 8);
      qraw[0][2] = *(const i32x4*)(qp + 16 * (grp + 4));
      qraw[0][3] = *(const i32x4*)(qp + 16 * (grp + 4) + 8);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) qraw[0][i] = i32x4{0, 0, 0, 0};
    }
  };

  const float k_tensor_scale = PER_TOKEN ? 1.0f : key_scale[0];
  const float v_tensor_scale = PER_TOKEN ? 1.0f : value_scale[0];
  const float logit_scale = a.softmax_scale * kLog2e * k_tensor_scale;
  const int krow = (c16 >> 3) * kKHalf + (8 * ((c16 >> 2) & 1) + (c16 & 3)) * 16;
  WaveState<1> st;
  st.reset();
  QueryTile<1> qt;

  // Query rows are loaded during the previous piece's last unit when the
  // next piece is known by then (qready), else at the piece's first unit.
  bool qready = false;
  int gc = 0;     // chunks computed
  int cslot = 0;  // gc % S
  while (iok && issued < S) issue_next();

  while (has_cur) {
    const int units = (cur.n + U - 1) / U;
    for (int u = 0; u < units; ++u) {
      const int nch = pa_min(U, cur.n - U * u);
      if (issued < gc + nch) {
        // The issue side paused past an empty piece: this unit's chunks go
        // now, once every wave is done with the previous unit (their slots
        // held chunks S back).  Workgroup-uniform: every wave walks the same
        // pieces.
        asm volatile("s_barrier" ::: "memory");
        while (issued < gc + nch) issue_next();
      }
      // This wave's chunks of the unit: its chunks issued after them (chunk
      // j is this wave's when j % NW == wave) may stay in flight (loads
      // retire in order; query rows issued in between are only waited for
      // early).
      const int own_newer = (issued + NW - 1 - wave) / NW - (gc + nch + NW - 1 - wave) / NW;
      if (own_newer >= 3)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(3 * kChunkLoads));
      else if (own_newer == 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * kChunkLoads));
      else if (own_newer == 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(kChunkLoads));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
      // Value bytes of page slots outside the sequence's visible keys
      // [lo_all, hi_all) -- a page's tail past the context, slots before a
      // window -- may hold any byte, e4m3fn NaN included, which a zero
      // probability does not cancel.  The wave that loaded a chunk zeroes
      // them (edge units only; workgroup-uniform test), so the value
      // products need no masks.
      {
        const int ub = cur.tb0 + u * (U * kChunk);
        if (ub < cur.lo_all || ub + nch * kChunk > cur.hi_all) {
          for (int ch = 0; ch < nch; ++ch) {
            if ((gc + ch) % NW != wave) continue;
            int sl = cslot + ch;
            sl = sl >= S ? sl - S : sl;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
              zero_stale_values((LDS_AS unsigned char*)smem + sl * kSlotBytes + kKBytes + hh * 2048,
                                ub + ch * kChunk + 16 * hh, cur.lo_all, cur.hi_all, lane);
            if (PER_TOKEN) {
              // and the chunk's per-token K and V scales of those keys
              // (lane l: K scale l < 32, else V scale l - 32), so that the
              // softmax reads zeros there rather than stale bits
              const int t = ub + ch * kChunk + (lane & 31);
              if (t < cur.lo_all || t >= cur.hi_all)
                ((LDS_AS float*)((LDS_AS unsigned char*)smem + sl * kSlotBytes + kKBytes + kVBytes))[lane] = 0.0f;
            }
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
      }
      // Every wave's share of the unit is in LDS and every wave is done
      // with the previous unit.  A bare s_barrier: the DMA completion was
      // awaited explicitly above (a fenced barrier would also wait for the
      // chunks still in flight).
      asm volatile("s_barrier" ::: "memory");
      if (u == 0) {
        if (!qready) load_query(cur);
        prepare_query<1>(qt, qraw, a.query_dtype, logit_scale, cur.ctx, ql, gqa, a.sliding_window, c16, wave * 16);
      }
      if (u == units - 1) {
        qready = has_nxt && nxt.n > 0;
        if (qready) load_query(nxt);
      }

      // Slots of chunks before gc are free: every wave has passed this
      // unit's barrier, so it is done with them.
      while (iok && issued < gc + S) issue_next();
      const LDS_AS unsigned char* sks[U];
      const LDS_AS float* sss[U];
      int tbs[U];
      const int tb0 = cur.tb0 + u * (U * kChunk);
#pragma unroll
      for (int ch = 0; ch < U; ++ch) {
        // a missing chunk reads the unit's first slot and is masked
        int sl = cslot + (ch < nch ? ch : 0);
        sl = sl >= S ? sl - S : sl;
        sks[ch] = (const LDS_AS unsigned char*)smem + sl * kSlotBytes;
        sss[ch] = (const LDS_AS float*)(sks[ch] + kKBytes + kVBytes);
        tbs[ch] = ch < nch ? tb0 + ch * kChunk : kFarToken;
      }
      if constexpr (U == 4) {
        unit4_softmax_pv<PER_TOKEN, S, kSlotBytes>(st, qt, (const LDS_AS unsigned char*)smem, cslot, nch, tb0, grp,
                                                   c16);
      } else {
        f32x4 la[U][1], lb[U][1];
#pragma unroll
        for (int ch = 0; ch < U; ++ch) chunk_logits<1>(qt, sks[ch], krow, grp, la[ch], lb[ch]);
        unit_softmax_pv<PER_TOKEN, U>(st, qt, la, lb, sks, sss, grp, c16, tbs);
      }
      gc += nch;
      cslot += nch;
      cslot = cslot >= S ? cslot - S : cslot;
    }
    mfma_drain(st.acc[0]);
    // ---- the piece is complete: this wave's columns ----
    const float vfin = PER_TOKEN ? st.vsmax : v_tensor_scale;
    store_piece<WORKLIST>(a, output, part_out, part_lse, cur, st.acc[0], sum_over_groups(st.lsum[0]), st.m2[0],
                          vfin, e, grp, kPBias);
    if (!WORKLIST && cur.desc_cnt > 0 && wave == 0 && lane == 0)
      *(i32x2*)(segdesc + 2 * ((int64_t)cur.b * a.num_kv_heads + cur.h)) = i32x2{cur.target, cur.desc_cnt};
    st.reset();
    // ---- move the window ----
    cur = nxt;
    has_cur = has_nxt;
    has_nxt = has_cur && next_piece(nxt);
    if (iw == 1) iw = 0;  // the issue cursor's piece is now cur
    if (!iok && has_nxt && nxt.n > 0) issue_enter(nxt, 1);
  }
}

// Log-sum-exp merge of n partial rows into 2 head dims per lane:
// lse_at(i) and row_at(i) (element offset of the row) address item i.  All
// loads of a batch of up to kBatch rows are issued before any is used.
template <int kBatch, typename LseAt, typename RowAt>
__device__ __forceinline__ void merge_rows(int n, const float* lse, const float* rows, LseAt lse_at, RowAt row_at,
                                           int lane, float& o0, float& o1) {
  float M = kNegInf, tot = 0.0f;
  o0 = 0.0f;
  o1 = 0.0f;
  for (int p0 = 0; p0 < n; p0 += kBatch) {
    const int nb = n - p0 < kBatch ? n - p0 : kBatch;
    const float l = lane < nb ? lse[lse_at(p0 + lane)] : kNegInf;
    f32x2 x[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int q = i < nb ? i : nb - 1;
      x[i] = *(const f32x2*)(rows + row_at(p0 + q) + 2 * lane);
    }
    float mb = l;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mb = fmaxf(mb, shfl_xor(mb, o));
    const float Mn = fmaxf(M, mb);
    if (Mn == kNegInf) continue;
    const float w = l == kNegInf ? 0.0f : __expf(l - Mn);
    float ws = w;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ws += shfl_xor(ws, o);
    const float fold = M == kNegInf ? 0.0f : __expf(M - Mn);
    tot = tot * fold + ws;
    o0 *= fold;
    o1 *= fold;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const float wi = __shfl(w, i, 64);
      if (i < nb) {
        o0 += wi * x[i][0];
        o1 += wi * x[i][1];
      }
    }
    M = Mn;
  }
  const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
  o0 *= inv;
  o1 *= inv;
}

__device__ __forceinline__ void store_out2(void* out, int dtype, int64_t off, float o0, float o1) {
  if (dtype == PA_DTYPE_F32) {
    *(f32x2*)((float*)out + off) = f32x2{o0, o1};
  } else if (dtype == PA_DTYPE_F16) {
    *(uint32_t*)((uint16_t*)out + off) = f32_to_f16_bits(o0) | (f32_to_f16_bits(o1) << 16);
  } else {
    *(uint32_t*)((uint16_t*)out + off) = f32_to_bf16_bits(o0) | (f32_to_bf16_bits(o1) << 16);
  }
}

// Merge of a balanced launch: one wave per (sequence, kv head, block of
// 4J query columns).  Load j of a piece reads columns 4j .. 4j+3 of the
// block, 1 KiB of consecutive bf16 rows: lane l takes column 4j + l / 16 and
// head dims 8(l % 16) .. +7.  Each lane folds the pieces of its J columns
// (running log-sum-exp), with every load of a batch of pieces issued before
// use.  Pairs a single run held whole were written by the decode; pairs with
// no visible key get zeros; a cut pair's pieces are partial id segdesc[0]
// (the first run's) and the first piece (id 2w) of the pair's wave w in each
// following run (w G further on with head groups of G).
template <int J>
__global__ __launch_bounds__(256) void pa_fp8_segment_merge_kernel(const pa_fp8_stream_args a,
                                                                   const int32_t* segdesc, const uint16_t* part_out,
                                                                   const float* part_lse) {
  constexpr int kCols = 4 * J;      // columns per wave
  // pieces whose loads are in flight together: two for 16-column blocks,
  // which keeps the kernel at four waves per SIMD (126 VGPRs; four pieces
  // take 170), so 1024 pairs of 64 columns merge in one round of
  // workgroups
  constexpr int kBatch = J == 4 ? 2 : 16 / J;
  static_assert(kHead == 128, "16 lanes cover one 256-byte bf16 row");
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int ql = a.query_length, gqa = a.query_group_size, eq = ql * gqa;
  const int nblk = (eq + kCols - 1) / kCols;
  const int64_t rows = (int64_t)a.num_seqs * a.num_kv_heads * nblk;
  if (row >= rows) return;
  const int blk = (int)(row % nblk);
  const int h = (int)((row / nblk) % a.num_kv_heads);
  const int b = (int)(row / ((int64_t)nblk * a.num_kv_heads));
  // The pair's descriptor is read together with its length (it is only
  // meaningful, and only used, when the pair has visible keys).
  const int ctx = a.context_lengths[b];
  const i32x2 d = *(const i32x2*)(segdesc + 2 * ((int64_t)b * a.num_kv_heads + h));
  int rl = 1;
  if (a.kv_indptr) rl = a.kv_indptr[b + 1] - a.kv_indptr[b];
  const int nb = rl > 0 ? pa_plan_seq_chunks(ctx, ql, a.sliding_window) : 0;
  const int d0 = 8 * (lane & 15);
  // Runs of the per-wave split (<= 16 columns) walk head groups: the pieces
  // of one pair are G wave ids apart.
  const int G = eq <= 16 ? balanced_group(a.num_kv_heads, a.num_workers, eq) : 1;
  int e[J], ec[J];  // column, and the column whose row a lane past eq reads instead
#pragma unroll
  for (int j = 0; j < J; ++j) {
    e[j] = blk * kCols + 4 * j + (lane >> 4);
    ec[j] = e[j] < eq ? e[j] : eq - 1;
  }
  f32x4 o[J][2];
#pragma unroll
  for (int j = 0; j < J; ++j) o[j][0] = o[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (nb > 0) {
    const int pid0 = d[0], cnt = d[1];
    if (cnt <= 1) return;  // written by the decode
    const int w0 = pid0 >> 1;
    float M[J], tot[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      M[j] = kNegInf;
      tot[j] = 0.0f;
    }
    for (int i0 = 0; i0 < cnt; i0 += kBatch) {
      float l[kBatch][J];
      uint4 x[kBatch][J];  // bf16 rows (store_piece)
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = i0 + k < cnt ? i0 + k : cnt - 1;
        const int64_t pid = i == 0 ? pid0 : 2 * ((int64_t)w0 + (int64_t)i * G);
#pragma unroll
        for (int j = 0; j < J; ++j) {
          l[k][j] = part_lse[pid * eq + ec[j]];
          x[k][j] = *(const uint4*)(part_out + (pid * eq + ec[j]) * kHead + d0);
        }
      }
      // Branch-free fold: a piece past cnt or with no visible key gets
      // weight 0 (and fold 1 once the column has a maximum), which leaves the
      // state unchanged.
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const bool in = i0 + k < cnt;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const float lk = in ? l[k][j] : kNegInf;
          const float Mn = fmaxf(M[j], lk);
          const float fold = M[j] == kNegInf ? 0.0f : __expf(M[j] - Mn);
          const float w = lk == kNegInf ? 0.0f : __expf(lk - Mn);
          tot[j] = tot[j] * fold + w;
          const uint4 u = lk == kNegInf ? uint4{0u, 0u, 0u, 0u} : x[k][j];
          const f32x4 lo = {__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                            __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u)};
          const f32x4 hi = {__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                            __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u)};
          o[j][0] = o[j][0] * fold + lo * w;
          o[j][1] = o[j][1] * fold + hi * w;
          M[j] = Mn;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float inv = tot[j] > 0.0f ? 1.0f / tot[j] : 0.0f;
      o[j][0] *= inv;
      o[j][1] *= inv;
    }
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (e[j] >= eq) continue;
    const int qi = e[j] / gqa, g = e[j] - qi * gqa;
    const int64_t off =
        (int64_t)(b * ql + qi) * a.stride_out_tok + (int64_t)(h * gqa + g) * a.stride_out_head + d0;
    store_out4(a.output, a.output_dtype, off, o[j][0]);
    store_out4(a.output, a.output_dtype, off + 4, o[j][1]);
  }
}

// Merge of work-list partials: one wave per (group, query, query head).
__global__ __launch_bounds__(256) void pa_fp8_worklist_reduce_kernel(const pa_fp8_worklist_reduce_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int Hq = a.num_query_heads, mq = a.max_query_length;
  if (row >= (int64_t)a.num_groups * mq * Hq) return;
  const int qh = (int)(row % Hq);
  const int qi = (int)((row / Hq) % mq);
  const int g = (int)(row / ((int64_t)Hq * mq));
  const int p0 = a.reduce_indptr[g], p1 = a.reduce_indptr[g + 1];
  if (p1 <= p0) return;
  const int qo0 = a.reduce_final_map[2 * g], qo1 = a.reduce_final_map[2 * g + 1];
  if (qi >= qo1 - qo0) return;
  const int32_t* pmap = a.reduce_partial_map + p0;
  float o0, o1;
  merge_rows<8>(
      p1 - p0, a.partial_lse, a.partial_output,
      [&](int i) { return (int64_t)(pmap[i] + qi) * a.stride_pl_row + qh; },
      [&](int i) { return (int64_t)(pmap[i] + qi) * a.stride_po_row + (int64_t)qh * kHead; }, lane, o0, o1);
  store_out2(a.output, a.output_dtype, (int64_t)(qo0 + qi) * a.stride_out_tok + (int64_t)qh * a.stride_out_head + 2 * lane,
             o0, o1);
}

// Work-list merge for head size 128 with query heads in blocks of eight:
// one wave per (reduce group, query row, block).  Load j of a piece reads
// two float32 rows (query heads 2 j, 2 j + 1 of the block, 1 KiB of
// consecutive bytes): lane l takes head 2 j + l / 32 and head dims
// 4 (l % 32) .. + 3.  Two pieces are in flight at a time, folded as the
// balanced merge folds them (a piece without visible keys gets weight 0).
// Against one wave per output row, a group is looked up by 8x fewer waves,
// and each load instruction moves 1 KiB instead of 512 bytes.
__global__ __launch_bounds__(256) void pa_fp8_worklist_reduce8_kernel(const pa_fp8_worklist_reduce_args a) {
  constexpr int J = 4;       // loads per piece
  constexpr int kBatch = 2;  // pieces in flight
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int Hq = a.num_query_heads, mq = a.max_query_length;
  const int nhb = Hq / 8;
  if (w >= (int64_t)a.num_groups * mq * nhb) return;
  const int hb = (int)(w % nhb);
  const int qi = (int)((w / nhb) % mq);
  const int g = (int)(w / ((int64_t)nhb * mq));
  const int p0 = a.reduce_indptr[g], p1 = a.reduce_indptr[g + 1];
  if (p1 <= p0) return;
  const int qo0 = a.reduce_final_map[2 * g], qo1 = a.reduce_final_map[2 * g + 1];
  if (qi >= qo1 - qo0) return;
  const int32_t* pmap = a.reduce_partial_map + p0;
  const int n = p1 - p0;
  const int d0 = 4 * (lane & 31);
  int qh[J];
#pragma unroll
  for (int j = 0; j < J; ++j) qh[j] = 8 * hb + 2 * j + (lane >> 5);
  float M[J], tot[J];
  f32x4 o[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    M[j] = kNegInf;
    tot[j] = 0.0f;
    o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int i0 = 0; i0 < n; i0 += kBatch) {
    float l[kBatch][J];
    f32x4 x[kBatch][J];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int i = i0 + k < n ? i0 + k : n - 1;
      const int64_t prow = (int64_t)pmap[i] + qi;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        l[k][j] = a.partial_lse[prow * a.stride_pl_row + qh[j]];
        x[k][j] = *(const f32x4*)(a.partial_output + prow * a.stride_po_row + (int64_t)qh[j] * kHead + d0);
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const bool in = i0 + k < n;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const float lk = in ? l[k][j] : kNegInf;
        const float Mn = fmaxf(M[j], lk);
        const float fold = M[j] == kNegInf ? 0.0f : __expf(M[j] - Mn);
        const float wk = lk == kNegInf ? 0.0f : __expf(lk - Mn);
        tot[j] = tot[j] * fold + wk;
        const f32x4 xv = lk == kNegInf ? f32x4{0.f, 0.f, 0.f, 0.f} : x[k][j];
        o[j] = o[j] * fold + xv * wk;
        M[j] = Mn;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float inv = tot[j] > 0.0f ? 1.0f / tot[j] : 0.0f;
    store_out4(a.output, a.output_dtype,
               (int64_t)(qo0 + qi) * a.stride_out_tok + (int64_t)qh[j] * a.stride_out_head + d0, o[j] * inv);
  }
}

// One wave per (sequence, kv head, column); lane l covers head dims 2l,
// 2l+1.  For each batch of up to 32 slots every load -- the slot's max and
// sum (one slot per lane) and the lane's two values of every slot's partial
// row -- is issued before any is used, so a row costs one memory round trip
// per 32 slots; max and sum are then reduced across the wave.
__global__ __launch_bounds__(256) void pa_fp8_lse_reduce_kernel(const pa_fp8_reduce_args a) {
  constexpr int kBatch = 32;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int eq = a.query_length * a.query_group_size;
  const int64_t rows = (int64_t)a.num_seqs * a.num_kv_heads * eq;
  if (row >= rows) return;
  const int e = (int)(row % eq);
  const int h = (int)((row / eq) % a.num_kv_heads);
  const int b = (int)(row / ((int64_t)eq * a.num_kv_heads));
  const int P = a.num_partitions;
  const int64_t sbase = (int64_t)b * a.stride_es_seq + (int64_t)h * a.stride_es_head + e;
  const int64_t tbase =
      (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head + (int64_t)e * a.stride_to_group + 2 * lane;
  // Running log-sum-exp state over the batches.
  float M = kNegInf, tot = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int p0 = 0; p0 < P; p0 += kBatch) {
    const int n = P - p0 < kBatch ? P - p0 : kBatch;
    const int p = p0 + lane;
    const bool mine = lane < n;
    const float m = mine ? a.max_logits[sbase + p * a.stride_es_part] : kNegInf;
    const float es = mine ? a.exp_sums[sbase + p * a.stride_es_part] : 0.0f;
    float x0[kBatch], x1[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int q = i < n ? i : n - 1;
      const int64_t off = tbase + (int64_t)(p0 + q) * a.stride_to_part;
      if (a.tmp_dtype == PA_DTYPE_F32) {
        const f32x2 t = *(const f32x2*)((const float*)a.tmp_out + off);
        x0[i] = t[0];
        x1[i] = t[1];
      } else {
        const uint32_t t = *(const uint32_t*)((const uint16_t*)a.tmp_out + off);
        x0[i] = bf16_bits_to_f32(t & 0xffffu);
        x1[i] = bf16_bits_to_f32(t >> 16);
      }
    }
    float mb = m;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mb = fmaxf(mb, shfl_xor(mb, o));
    const float Mn = fmaxf(M, mb);
    if (Mn == kNegInf) continue;  // every slot so far empty
    const float w = m == kNegInf ? 0.0f : es * __expf(m - Mn);
    float ws = w;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ws += shfl_xor(ws, o);
    const float fold = M == kNegInf ? 0.0f : __expf(M - Mn);
    tot = tot * fold + ws;
    o0 *= fold;
    o1 *= fold;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const float wi = __shfl(w, i, 64);
      if (i < n) {
        o0 += wi * x0[i];
        o1 += wi * x1[i];
      }
    }
    M = Mn;
  }
  const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
  o0 *= inv;
  o1 *= inv;
  const int gqa = a.query_group_size;
  const int qi = e / gqa, g = e - qi * gqa;
  const int64_t off = (int64_t)b * a.stride_out_seq + (int64_t)qi * a.stride_out_ql +
                      (int64_t)h * a.stride_out_kv_head + (int64_t)g * a.stride_out_group + 2 * lane;
  if (a.output_dtype == PA_DTYPE_F32) {
    *(f32x2*)((float*)a.output + off) = f32x2{o0, o1};
  } else if (a.output_dtype == PA_DTYPE_F16) {
    *(uint32_t*)((uint16_t*)a.output + off) = f32_to_f16_bits(o0) | (f32_to_f16_bits(o1) << 16);
  } else {
    *(uint32_t*)((uint16_t*)a.output + off) = f32_to_bf16_bits(o0) | (f32_to_bf16_bits(o1) << 16);
  }
}

// ===========================================================================
// Generic decode: head size D = 64, 128, 192 or 256, any number of query
// columns per kv head
// ===========================================================================
// The reference's small-block, window and persistent routes take any head
// size that is a multiple of 64 and tile any query_length * gqa into
// 16-column MFMA groups (kernels/pa_decode_fp8.py:2084-2085, 2101, 3058).
// The tuned kernels above are built for D = 128 and up to 64 columns; every
// other shape runs here, behind the same entry points and with the same
// outputs.  A wave owns one 16-column block of one (sequence, kv head) and
// streams a token range with K and V read straight from HBM into MFMA
// operand registers (no LDS, no barriers: the waves of a workgroup are
// independent, one per column block, and the grid's second dimension tiles
// the blocks):
//   * QK on v_mfma_f32_16x16x32_fp8_fp8, head dims along K: per 16-token
//     tile, D / 32 MFMAs for each of the query's fp8 hi and lo terms; lane
//     (grp, c16) supplies key row c16 (a token) and dims 8 grp .. 8 grp + 7
//     of every 32-dim block, and gets the logits of tokens 4 grp .. 4 grp + 3
//     of the tile for column c16;
//   * PV on the same instruction with the chunk's 32 tokens along K: k-byte
//     8 grp + i is token 4 grp + i (i < 4) or 16 + 4 grp + i - 4 of the
//     chunk -- exactly the tokens whose logits the lane holds -- so the
//     probabilities need no exchange; D / 16 output tiles, hi and lo
//     probability terms.
// The softmax is the online one of the tuned kernels (base-2 logits, a
// power-of-two query scale, probabilities 2^(8 + l - m) <= 256 split into
// two fp8 terms, per-token value scales folded into the probabilities
// against a running reference).  Value bytes of tokens outside the
// sequence's visible keys (stale page tails, slots before a window) are
// zeroed before the value product, and their scales are zero.

constexpr float kGenPBias = 8.0f;
constexpr float kGenPUnscale = 1.0f / 256.0f;  // 2^-kGenPBias

template <int D>
struct GenState {
  f32x4 acc[D / 16];
  float m2;     // base-2 running maximum of the column's scaled logits
  float lsum;   // this lane's share of sum 2^(pbias + l - m2)
  float vsref;  // value-scale reference (1 for per-tensor scales)
  __device__ __forceinline__ void reset(bool per_token) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    m2 = kNegInf;
    lsum = 0.0f;
    vsref = per_token ? 0.0f : 1.0f;
  }
};

// One (sequence, kv head) as a wave sees it: page list, bases and the
// column block's query.
template <int D>
struct GenCtx {
  const uint8_t* kbase;  // key_cache + h * stride_k_head
  const uint8_t* vbase;
  const float* ksbase;   // per-token scales + h * stride_ks_head
  const float* vsbase;
  const int32_t* pages;  // the sequence's page list
  int ctx, last_page;
  int lo_all, hi_all, lo_max, hi_min;  // union / intersection of the columns' keys
  long qhi[D / 32], qlo[D / 32];
  float fac;             // base-2 logit factor of the lane's column (> 0)
  int vis_lo, vis_hi;    // keys the lane's column sees
};

struct GenArgs {
  const void* query;
  const uint8_t* key_cache;
  const uint8_t* value_cache;
  const int32_t* block_tables;
  const int32_t* kv_indptr;
  const int32_t* context_lengths;
  const float* key_scale;
  const float* value_scale;
  int64_t stride_q_tok, stride_q_head;
  int64_t stride_k_block, stride_k_head;
  int64_t stride_v_block, stride_v_head;
  int64_t stride_bt_seq;
  int64_t stride_ks_block, stride_ks_head;
  int num_seqs, num_kv_heads, query_length, query_group_size;
  int block_size, num_blocks, max_blocks_per_seq, sliding_window, trans_v, query_dtype;
  float softmax_scale;
  // final output
  void* output;
  int output_dtype;
  int64_t stride_out_tok, stride_out_head;
  // slot partials (partition launches)
  float* exp_sums;
  float* max_logits;
  void* tmp_out;
  int tmp_dtype;
  int64_t stride_es_seq, stride_es_head, stride_es_part;
  int64_t stride_to_seq, stride_to_head, stride_to_part, stride_to_group;
  int num_partitions;
  int owner;  // kGenSlot, kGenOwnerSlots or kGenOwnerRange
  // work list
  const int32_t* work_indptr;
  const int32_t* work_info;
  const int32_t* partition_indptr;
  float* partial_output;
  float* partial_lse;
  int64_t stride_po_row, stride_pl_row;
};

// Sequence b, kv head h, the wave's column block (first column e0): page
// list, bounds, and the query columns as fp8 hi + lo B operands scaled by a
// power of two (prepare_query's scheme, for D dims).  Query row of column e:
// orow + e / gqa.
// First head dim of the 8 that lane group grp supplies to K-block blk of the
// key product (v_mfma_f32_16x16x32_fp8_fp8, head dims along K).  The dot
// product does not depend on how dims are dealt to the K slots, as long as
// queries and keys agree: K-blocks 2 j and 2 j + 1 take the two halves of
// 16-dim chunk 4 j + grp, so a lane reads each key row's chunk with one
// 16-byte load.  D / 32 is even for every head size served here.
__device__ __forceinline__ int gen_qk_dim(int blk, int grp) { return 64 * (blk >> 1) + 16 * grp + 8 * (blk & 1); }

template <int D, bool PER_TOKEN>
__device__ __forceinline__ bool gen_setup(GenCtx<D>& c, const GenArgs& a, int b, int h, int orow, int e0,
                                          int grp, int c16) {
  const int ql = a.query_length, gqa = a.query_group_size, eq = ql * gqa;
  c.ctx = ld_uniform(a.context_lengths, b);
  int row_len;
  if (a.kv_indptr) {
    const int p0 = ld_uniform(a.kv_indptr, b);
    c.pages = a.block_tables + p0;
    row_len = ld_uniform(a.kv_indptr, b + 1) - p0;
  } else {
    c.pages = a.block_tables + (int64_t)b * a.stride_bt_seq;
    row_len = a.max_blocks_per_seq;
  }
  c.last_page = pa_min(pa_cdiv(c.ctx, a.block_size) - 1, row_len - 1);
  pa_plan_visible(c.ctx, 0, ql, a.sliding_window, &c.lo_all, &c.hi_min);
  pa_plan_visible(c.ctx, ql - 1, ql, a.sliding_window, &c.lo_max, &c.hi_all);
  if (c.last_page < 0) c.hi_all = c.lo_all;
  c.kbase = a.key_cache + (int64_t)h * a.stride_k_head;
  c.vbase = a.value_cache + (int64_t)h * a.stride_v_head;
  c.ksbase = PER_TOKEN ? a.key_scale + (int64_t)h * a.stride_ks_head : a.key_scale;
  c.vsbase = PER_TOKEN ? a.value_scale + (int64_t)h * a.stride_ks_head : a.value_scale;

  const int e = e0 + c16;
  const bool valid = e < eq;
  const int qi = valid ? e / gqa : 0;
  const int g = valid ? e - qi * gqa : 0;
  float v[D / 32][8];
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk) {
    i32x4 w = i32x4{0, 0, 0, 0};
    if (valid)
      w = *(const i32x4*)((const uint16_t*)a.query + (int64_t)(orow + qi) * a.stride_q_tok +
                          (int64_t)(h * gqa + g) * a.stride_q_head + gen_qk_dim(blk, grp));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = (uint32_t)w[i];
      v[blk][2 * i] = a.query_dtype == PA_DTYPE_F16 ? f16_bits_to_f32(u & 0xffffu) : bf16_bits_to_f32(u & 0xffffu);
      v[blk][2 * i + 1] = a.query_dtype == PA_DTYPE_F16 ? f16_bits_to_f32(u >> 16) : bf16_bits_to_f32(u >> 16);
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[blk][i]));
  amax = max_over_groups(amax);
  int sexp = 261 - (int)((__float_as_uint(amax) >> 23) & 0xffu);
  sexp = sexp < 1 ? 1 : (sexp > 254 ? 254 : sexp);
  const float logit_scale = a.softmax_scale * kLog2e * (PER_TOKEN ? 1.0f : a.key_scale[0]);
  const float sq0 = amax > 0.0f ? __uint_as_float((uint32_t)sexp << 23) : 1.0f;
  const float sq = logit_scale < 0.0f ? -sq0 : sq0;
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk) {
    float xs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[i] = v[blk][i] * sq;
    split8_fp8(xs, c.qhi[blk], c.qlo[blk]);
  }
  c.fac = fmaxf(logit_scale / sq, 1e-30f);
  int lo = 0, hi = 0;
  if (valid) pa_plan_visible(c.ctx, qi, ql, a.sliding_window, &lo, &hi);
  c.vis_lo = lo;
  c.vis_hi = hi;
  c.lo_all = __builtin_amdgcn_readfirstlane(c.lo_all);
  c.hi_all = __builtin_amdgcn_readfirstlane(c.hi_all);
  c.lo_max = __builtin_amdgcn_readfirstlane(c.lo_max);
  c.hi_min = __builtin_amdgcn_readfirstlane(c.hi_min);
  return true;
}

__device__ __forceinline__ int gen_page(const GenArgs& a, const int32_t* pages, int last_page, int tok) {
  int lp = pa_min(tok / a.block_size, last_page);
  int p = ld_uniform(pages, lp);
  pa_note(p < 0 || p >= a.num_blocks, PA_VIOLATION_PAGE);
  p = p < 0 ? 0 : p;
  return p < a.num_blocks ? p : a.num_blocks - 1;
}

// Byte mask keeping the bytes of tokens [lo, hi) among the 4 tokens t .. t + 3.
// Probability bytes of the key product's layout -- lane group g holds
// tokens 4 g .. 4 g + 3 of each 16-token half, half 0 in the low word --
// reordered to the value product's: lane group g supplies tokens
// 8 (g >> 1) .. +7 of half g & 1.  Groups 0 and 1 (and 2 and 3) trade one
// word: v_permlane16_swap leaves group 2k + h with (half h of group 2k,
// half h of group 2k + 1).
__device__ __forceinline__ long gen_pv_order(long p) {
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)(uint64_t)p, (uint32_t)((uint64_t)p >> 32), false, false);
  return (long)((uint64_t)r[0] | ((uint64_t)r[1] << 32));
}

__device__ __forceinline__ uint32_t gen_keep4(int t, int lo, int hi) {
  const int l = pa_min(pa_max(lo - t, 0), 4), u = pa_min(pa_max(hi - t, l), 4);
  const uint32_t below_u = u >= 4 ? ~0u : (1u << (8 * u)) - 1;
  const uint32_t below_l = l >= 4 ? ~0u : (1u << (8 * l)) - 1;
  return below_u & ~below_l;
}

// One 32-token chunk's operands in registers: the lane's key pieces for the
// two 16-token tiles, its value words for every 16-dim output tile and its
// tokens' scales.  Loaded a chunk ahead of their use (gen_range), so a
// chunk's memory latency overlaps the previous chunk's arithmetic.  With
// VPF false (D >= 192, for registers) the values are loaded at the start of
// their own chunk instead, still ahead of its key product.
template <int D, bool PER_TOKEN>
struct GenChunk {
  static constexpr bool VPF = D <= 128;
  // Two chunk buffers (the next chunk's keys in flight during this one's
  // arithmetic) up to D = 256; above, one buffer, so that the accumulators,
  // query operands and one chunk's operands fit the register file.
  static constexpr bool KPF = D <= 256;
  long kr[2][D / 32];
  uint64_t vw[D / 16];
  float ks[8], vs[8];
  int pg[2], sb[2];
};

template <int D, bool PER_TOKEN>
__device__ __forceinline__ void gen_load_values(GenChunk<D, PER_TOKEN>& ch, const GenCtx<D>& c, const GenArgs& a,
                                                int grp, int c16) {
  // head dim 16 j + c16, tokens 8 (grp >> 1) .. +7 of the chunk's half
  // grp & 1: one 8-byte load per output tile (gen_pv_order)
  const int bs = a.block_size;
  const bool half = grp & 1;  // selects, not indices (a runtime index would put ch in scratch)
  const int sv = (half ? ch.sb[1] : ch.sb[0]) + 8 * (grp >> 1);
  const uint8_t* vp = c.vbase + (int64_t)(half ? ch.pg[1] : ch.pg[0]) * a.stride_v_block;
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    const int d = 16 * j + c16;
    const int64_t off = a.trans_v ? ((int64_t)(sv >> 4) * D + d) * 16 + (sv & 15) : (int64_t)d * bs + sv;
    ch.vw[j] = __builtin_nontemporal_load((const uint64_t*)(vp + off));
  }
}

template <int D, bool PER_TOKEN>
__device__ __forceinline__ void gen_load(GenChunk<D, PER_TOKEN>& ch, const GenCtx<D>& c, const GenArgs& a, int tc,
                                         int grp, int c16) {
  const int bs = a.block_size;
#pragma unroll
  for (int tau = 0; tau < 2; ++tau) {
    ch.pg[tau] = gen_page(a, c.pages, c.last_page, tc + 16 * tau);
    ch.sb[tau] = (tc + 16 * tau) % bs;
  }
  // key row c16 of each 16-token tile: the lane's 16-dim chunk 4 j + grp,
  // one 16-byte load for K-blocks 2 j and 2 j + 1 (gen_qk_dim)
#pragma unroll
  for (int tau = 0; tau < 2; ++tau) {
    const uint8_t* kp = c.kbase + (int64_t)ch.pg[tau] * a.stride_k_block + (ch.sb[tau] + c16) * 16 +
                        (int64_t)grp * bs * 16;
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      const i32x4 w = __builtin_nontemporal_load((const i32x4*)(kp + (int64_t)(4 * j) * bs * 16));
      ch.kr[tau][2 * j] = (long)((uint64_t)(uint32_t)w[0] | ((uint64_t)(uint32_t)w[1] << 32));
      ch.kr[tau][2 * j + 1] = (long)((uint64_t)(uint32_t)w[2] | ((uint64_t)(uint32_t)w[3] << 32));
    }
  }
  if (PER_TOKEN) {
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
      const int64_t so = (int64_t)ch.pg[tau] * a.stride_ks_block + ch.sb[tau] + 4 * grp;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ch.ks[4 * tau + i] = c.ksbase[so + i];
        ch.vs[4 * tau + i] = c.vsbase[so + i];
      }
    }
  }
  if constexpr (GenChunk<D, PER_TOKEN>::VPF) gen_load_values(ch, c, a, grp, c16);
}

// Online softmax of the lane's column over the chunk at tc (keys [A, B) used;
// t0, t1 bound the visible ones).
template <int D, bool PER_TOKEN>
__device__ __forceinline__ void gen_chunk(GenState<D>& st, GenChunk<D, PER_TOKEN>& ch, const GenCtx<D>& c,
                                          const GenArgs& a, int tc, int t0, int t1, int A, int B, int vis_lo,
                                          int vis_hi, int grp, int c16) {
  if constexpr (!GenChunk<D, PER_TOKEN>::VPF) gen_load_values(ch, c, a, grp, c16);
  // ---- logits of tokens tc + 16 tau + 4 grp + i ----
  f32x4 lt[2];
#pragma unroll
  for (int tau = 0; tau < 2; ++tau) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int blk = 0; blk < D / 32; ++blk) {
      acc = mfma_fp8(ch.kr[tau][blk], c.qhi[blk], acc);
      acc = mfma_fp8(ch.kr[tau][blk], c.qlo[blk], acc);
    }
    lt[tau] = acc;
  }
  float x[8], vs[8];
#pragma unroll
  for (int tau = 0; tau < 2; ++tau)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[4 * tau + i] = lt[tau][i];
      vs[4 * tau + i] = 1.0f;
    }
  if (PER_TOKEN) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[k] *= ch.ks[k];
      vs[k] = ch.vs[k];
    }
  }
  // ---- masks (edge chunks only) ----
  const bool all_vis = tc >= pa_max(t0, c.lo_max) && tc + 32 <= pa_min(t1, c.hi_min);
  if (!all_vis) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = tc + 16 * (k >> 2) + 4 * grp + (k & 3);
      x[k] = (t >= vis_lo && t < vis_hi) ? x[k] : kNegInf;
      if (PER_TOKEN) vs[k] = (t >= A && t < B) ? vs[k] : 0.0f;
    }
  }
  // ---- online softmax ----
  float cmax = kNegInf;
#pragma unroll
  for (int k = 0; k < 8; ++k) cmax = fmaxf(cmax, x[k]);
  cmax = max_over_groups(cmax) * c.fac;
  const float mnew = fmaxf(st.m2, cmax);
  const float muse = mnew == kNegInf ? 0.0f : mnew;
  const float alpha = __builtin_amdgcn_exp2f(st.m2 - muse);
  float vratio = 1.0f, vinv = 1.0f;
  if (PER_TOKEN) {
    float vmax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) vmax = fmaxf(vmax, vs[k]);
    vmax = max_over_groups(vmax);
    const float vnew = fmaxf(st.vsref, vmax);
    vratio = st.vsref > 0.0f ? st.vsref / vnew : 1.0f;
    vinv = vnew > 0.0f ? 1.0f / vnew : 0.0f;
    st.vsref = vnew;
  }
  st.m2 = mnew;
  const float f = alpha * vratio;
  if (__ballot(f != 1.0f)) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) st.acc[j] *= f;
  }
  const float bias = kGenPBias - muse;
  float psum = 0.0f, pr[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[k], c.fac, bias));
    psum += p;
    pr[k] = PER_TOKEN ? p * (vs[k] * vinv) : p;
  }
  st.lsum = st.lsum * alpha + psum;
  long phi, plo;
  split8_fp8(pr, phi, plo);
  // ---- value product: the lane supplies tokens 8 (grp >> 1) .. +7 of half
  // grp & 1 (its value words), so the probabilities move to that order ----
  uint64_t keep = ~0ull;
  const bool stale = tc < A || tc + 32 > B;
  if (stale) {
    const int t = tc + 16 * (grp & 1) + 8 * (grp >> 1);
    keep = (uint64_t)gen_keep4(t, A, B) | ((uint64_t)gen_keep4(t + 4, A, B) << 32);
  }
  const long ph = gen_pv_order(phi), pl = gen_pv_order(plo);
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    const long vv = (long)(ch.vw[j] & keep);
    st.acc[j] = mfma_fp8(vv, ph, st.acc[j]);
    st.acc[j] = mfma_fp8(vv, pl, st.acc[j]);
  }
}

// Online softmax of the lane's column over keys [t0, t1) into st: chunks in
// pairs through two operand buffers (no register copies, whose waits would
// also wait for the next chunk's loads), each chunk's loads issued before
// the previous chunk's arithmetic.
template <int D, bool PER_TOKEN>
__device__ void gen_range(GenState<D>& st, const GenCtx<D>& c, const GenArgs& a, int t0, int t1, int grp,
                          int c16) {
  // keys any column may use, and the stale-byte bound
  const int A = pa_max(t0, c.lo_all), B = pa_min(t1, c.hi_all);
  if (B <= A) return;
  const int vis_lo = pa_max(c.vis_lo, t0), vis_hi = pa_min(c.vis_hi, t1);
  int tc = A & ~31;
  if constexpr (!GenChunk<D, PER_TOKEN>::KPF) {
    GenChunk<D, PER_TOKEN> ch;
    for (; tc < B; tc += 32) {
      gen_load(ch, c, a, tc, grp, c16);
      gen_chunk(st, ch, c, a, tc, t0, t1, A, B, vis_lo, vis_hi, grp, c16);
    }
    return;
  }
  GenChunk<D, PER_TOKEN> ch0, ch1;
  gen_load(ch0, c, a, tc, grp, c16);
  while (true) {
    const bool more1 = tc + 32 < B;
    if (more1) gen_load(ch1, c, a, tc + 32, grp, c16);
    gen_chunk(st, ch0, c, a, tc, t0, t1, A, B, vis_lo, vis_hi, grp, c16);
    if (!more1) break;
    const bool more2 = tc + 64 < B;
    if (more2) gen_load(ch0, c, a, tc + 64, grp, c16);
    gen_chunk(st, ch1, c, a, tc + 32, t0, t1, A, B, vis_lo, vis_hi, grp, c16);
    if (!more2) break;
    tc += 64;
  }
}

// s := s merged with t (two disjoint key ranges of one column).
template <int D, bool PER_TOKEN>
__device__ __forceinline__ void gen_merge(GenState<D>& s, const GenState<D>& t) {
  const float m = fmaxf(s.m2, t.m2);
  if (__ballot(m != kNegInf) == 0) return;
  const float mu = m == kNegInf ? 0.0f : m;
  const float as = __builtin_amdgcn_exp2f(s.m2 - mu), at = __builtin_amdgcn_exp2f(t.m2 - mu);
  float fs = as, ft = at, vref = 1.0f;
  if (PER_TOKEN) {
    vref = fmaxf(s.vsref, t.vsref);
    fs *= vref > 0.0f ? s.vsref / vref : 0.0f;
    ft *= vref > 0.0f ? t.vsref / vref : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < D / 16; ++j) s.acc[j] = s.acc[j] * fs + t.acc[j] * ft;
  s.lsum = s.lsum * as + t.lsum * at;
  s.m2 = m;
  s.vsref = vref;
}

// Normalised result of the lane's column: out = acc * scale; returns the
// column's natural-log log-sum-exp (-inf when it saw no key) and, in *es /
// *ml, the exp-sum and maximum of the slot-partial convention.
template <int D, bool PER_TOKEN>
__device__ __forceinline__ float gen_finish(const GenState<D>& st, const GenArgs& a, float& scale, float& es,
                                            float& ml) {
  const float L = sum_over_groups(st.lsum);
  const float vfin = PER_TOKEN ? st.vsref : a.value_scale[0];
  scale = L > 0.0f ? vfin / L : 0.0f;
  es = L > 0.0f ? L * kGenPUnscale : 0.0f;  // sum 2^(l - m) = L / 2^pbias
  ml = L > 0.0f ? kLn2 * st.m2 : kNegInf;
  return L > 0.0f ? kLn2 * (st.m2 + __builtin_amdgcn_logf(L) - kGenPBias) : kNegInf;
}

__device__ __forceinline__ void gen_store4(void* base, int dtype, int64_t off, f32x4 v) {
  if (dtype == PA_DTYPE_F32) {
    *(f32x4*)((float*)base + off) = v;
  } else if (dtype == PA_DTYPE_F16) {
    *(uint2*)((uint16_t*)base + off) = uint2{f32_to_f16_bits(v[0]) | (f32_to_f16_bits(v[1]) << 16),
                                             f32_to_f16_bits(v[2]) | (f32_to_f16_bits(v[3]) << 16)};
  } else {
    *(uint2*)((uint16_t*)base + off) = uint2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16),
                                             f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
  }
}

// Partition launch modes (GenArgs::owner).
enum : int {
  kGenSlot = 0,        // workgroup (b, h, slot): the slot's partials
  kGenOwnerSlots = 1,  // workgroup (b, h): every slot's partials, folded into `output`
  kGenOwnerRange = 2,  // workgroup (b, h): one pass over every visible key into `output`
};

// Partition launches: workgroup (b, h, slot) -- or (b, h) in the owner
// modes -- and column block 4 * blockIdx.y + wave.  A slot stores exp_sums /
// max_logits / tmp_out for its columns.  kGenOwnerSlots walks every slot,
// stores its partials, folds them and writes `output`; kGenOwnerRange (no
// partials asked for) streams the whole visible range with one state.
template <int D, bool PER_TOKEN, int MODE>
__global__ __launch_bounds__(256) void pa_fp8_generic_partition_kernel(const GenArgs a) {
  constexpr bool OWNER = MODE != kGenSlot;
  const int lane = threadIdx.x & 63, grp = lane >> 4, c16 = lane & 15;
  const int wave = threadIdx.x >> 6;
  const int eq = a.query_length * a.query_group_size;
  const int e0 = (4 * (int)blockIdx.y + wave) * 16;
  if (e0 >= eq) return;
  const int P = a.num_partitions;
  const int per = OWNER ? 1 : P;
  const int z0 = OWNER ? 0 : (int)(blockIdx.x % per);
  const int bh = (int)(blockIdx.x / per);
  const int h = bh % a.num_kv_heads, b = bh / a.num_kv_heads;
  GenCtx<D> c;
  gen_setup<D, PER_TOKEN>(c, a, b, h, b * a.query_length, e0, grp, c16);
  const int e = e0 + c16;
  const bool valid = e < eq;
  auto write_output = [&](const GenState<D>& s) {
    float sc, es, ml;
    gen_finish<D, PER_TOKEN>(s, a, sc, es, ml);
    const int qi = e / a.query_group_size, g = e - qi * a.query_group_size;
    const int64_t off = (int64_t)(b * a.query_length + qi) * a.stride_out_tok +
                        (int64_t)(h * a.query_group_size + g) * a.stride_out_head + 4 * grp;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) gen_store4(a.output, a.output_dtype, off + 16 * j, s.acc[j] * sc);
  };
  if constexpr (MODE == kGenOwnerRange) {
    // gen_range clips [0, ctx) to the keys some column sees (window included)
    GenState<D> st;
    st.reset(PER_TOKEN);
    gen_range<D, PER_TOKEN>(st, c, a, 0, c.ctx, grp, c16);
    if (valid) write_output(st);
    return;
  }
  GenState<D> fin;  // kGenOwnerSlots: the slots folded so far (unused otherwise)
  if (OWNER) fin.reset(PER_TOKEN);
  const int z1 = OWNER ? P : z0 + 1;
  for (int z = z0; z < z1; ++z) {
    int t0, t1;
    pa_plan_slot_tokens(c.ctx, P, z, a.sliding_window, a.query_length, &t0, &t1);
    GenState<D> st;
    st.reset(PER_TOKEN);
    gen_range<D, PER_TOKEN>(st, c, a, t0, t1, grp, c16);
    if (a.exp_sums) {
      float sc, es, ml;
      gen_finish<D, PER_TOKEN>(st, a, sc, es, ml);
      if (valid) {
        const int64_t so = (int64_t)b * a.stride_es_seq + (int64_t)h * a.stride_es_head + (int64_t)z * a.stride_es_part + e;
        if (grp == 0) {
          a.exp_sums[so] = es;
          a.max_logits[so] = ml;
        }
        const int64_t to = (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head + (int64_t)z * a.stride_to_part +
                           (int64_t)e * a.stride_to_group + 4 * grp;
#pragma unroll
        for (int j = 0; j < D / 16; ++j) gen_store4(a.tmp_out, a.tmp_dtype, to + 16 * j, st.acc[j] * sc);
      }
    }
    if constexpr (OWNER) gen_merge<D, PER_TOKEN>(fin, st);
  }
  if constexpr (OWNER) {
    if (valid) write_output(fin);
  }
}

// Work-list launches: workgroup = bin blockIdx.x (its works in order), column
// block 4 * blockIdx.y + wave.  A work writes output rows qo_start + qi
// (partial row < 0) or float32 partial rows ploc + query_length + qi and
// their log-sum-exp.
template <int D, bool PER_TOKEN>
__global__ __launch_bounds__(256) void pa_fp8_generic_worklist_kernel(const GenArgs a) {
  const int lane = threadIdx.x & 63, grp = lane >> 4, c16 = lane & 15;
  const int wave = threadIdx.x >> 6;
  const int gqa = a.query_group_size, eq = a.query_length * gqa;
  const int e0 = (4 * (int)blockIdx.y + wave) * 16;
  if (e0 >= eq) return;
  const int e = e0 + c16;
  const bool valid = e < eq;
  const int qi = valid ? e / gqa : 0, g = valid ? e - qi * gqa : 0;
  const int w0 = ld_uniform(a.work_indptr, blockIdx.x), w1 = ld_uniform(a.work_indptr, blockIdx.x + 1);
  for (int w = w0; w < w1; ++w) {
    const int64_t wi = 8 * (int64_t)w;
    const int b = ld_uniform(a.work_info, wi), ploc = ld_uniform(a.work_info, wi + 1);
    const int qo0 = ld_uniform(a.work_info, wi + 2);
    const int kv0 = ld_uniform(a.work_info, wi + 4), kv1 = ld_uniform(a.work_info, wi + 5);
    const int h = (ld_uniform(a.work_info, wi + 7) & 0xffff) / gqa;
    GenCtx<D> c;
    gen_setup<D, PER_TOKEN>(c, a, b, h, qo0, e0, grp, c16);
    const int pb = ld_uniform(a.partition_indptr, b);
    const int t0 = (kv0 - pb) * PA_PARTITION_TOKENS, t1 = pa_min((kv1 - pb) * PA_PARTITION_TOKENS, c.ctx);
    GenState<D> st;
    st.reset(PER_TOKEN);
    gen_range<D, PER_TOKEN>(st, c, a, t0, t1, grp, c16);
    float sc, es, ml;
    const float lse = gen_finish<D, PER_TOKEN>(st, a, sc, es, ml);
    if (!valid) continue;
    const int qh = h * gqa + g;
    if (ploc < 0) {
      const int64_t off = (int64_t)(qo0 + qi) * a.stride_out_tok + (int64_t)qh * a.stride_out_head + 4 * grp;
#pragma unroll
      for (int j = 0; j < D / 16; ++j) gen_store4(a.output, a.output_dtype, off + 16 * j, st.acc[j] * sc);
    } else {
      const int64_t row = ploc + a.query_length + qi;
#pragma unroll
      for (int j = 0; j < D / 16; ++j)
        *(f32x4*)(a.partial_output + row * a.stride_po_row + (int64_t)qh * D + 16 * j + 4 * grp) = st.acc[j] * sc;
      if (grp == 0) a.partial_lse[row * a.stride_pl_row + qh] = lse;
    }
  }
}

// Log-sum-exp merges for any head size: lane l of a wave takes head dims
// l + 64 k, k < NK = D / 64 (the 128-dim kernels above keep their
// two-adjacent-dims layout).
template <int NK>
__global__ __launch_bounds__(256) void pa_fp8_generic_lse_reduce_kernel(const pa_fp8_reduce_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int eq = a.query_length * a.query_group_size;
  const int64_t rows = (int64_t)a.num_seqs * a.num_kv_heads * eq;
  if (row >= rows) return;
  const int e = (int)(row % eq);
  const int h = (int)((row / eq) % a.num_kv_heads);
  const int b = (int)(row / ((int64_t)eq * a.num_kv_heads));
  const int64_t sbase = (int64_t)b * a.stride_es_seq + (int64_t)h * a.stride_es_head + e;
  const int64_t tbase = (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head + (int64_t)e * a.stride_to_group + lane;
  // Slots in batches of kBatch whose loads are all in flight together,
  // folded with a running maximum (empty slots, max -inf, are skipped).
  constexpr int kBatch = 8;
  float M = kNegInf, tot = 0.0f, o[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) o[k] = 0.0f;
  for (int p0 = 0; p0 < a.num_partitions; p0 += kBatch) {
    float m[kBatch], es[kBatch], x[kBatch][NK];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int p = p0 + i;
      m[i] = kNegInf;
      es[i] = 0.0f;
#pragma unroll
      for (int k = 0; k < NK; ++k) x[i][k] = 0.0f;
      if (p < a.num_partitions) {  // wave-uniform
        m[i] = a.max_logits[sbase + p * a.stride_es_part];
        es[i] = a.exp_sums[sbase + p * a.stride_es_part];
        const int64_t off = tbase + (int64_t)p * a.stride_to_part;
#pragma unroll
        for (int k = 0; k < NK; ++k)
          x[i][k] = a.tmp_dtype == PA_DTYPE_F32 ? ((const float*)a.tmp_out)[off + 64 * k]
                                                : bf16_bits_to_f32(((const uint16_t*)a.tmp_out)[off + 64 * k]);
      }
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (m[i] == kNegInf) continue;
      const float Mn = fmaxf(M, m[i]);
      const float fold = M == kNegInf ? 0.0f : __expf(M - Mn);
      const float w = es[i] * __expf(m[i] - Mn);
      tot = tot * fold + w;
#pragma unroll
      for (int k = 0; k < NK; ++k) o[k] = o[k] * fold + w * x[i][k];
      M = Mn;
    }
  }
  const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
  const int gqa = a.query_group_size;
  const int qi = e / gqa, g = e - qi * gqa;
  const int64_t off = (int64_t)b * a.stride_out_seq + (int64_t)qi * a.stride_out_ql + (int64_t)h * a.stride_out_kv_head +
                      (int64_t)g * a.stride_out_group + lane;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const float v = o[k] * inv;
    if (a.output_dtype == PA_DTYPE_F32)
      ((float*)a.output)[off + 64 * k] = v;
    else if (a.output_dtype == PA_DTYPE_F16)
      ((uint16_t*)a.output)[off + 64 * k] = (uint16_t)f32_to_f16_bits(v);
    else
      ((uint16_t*)a.output)[off + 64 * k] = (uint16_t)f32_to_bf16_bits(v);
  }
}

template <int NK>
__global__ __launch_bounds__(256) void pa_fp8_generic_worklist_reduce_kernel(const pa_fp8_worklist_reduce_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int Hq = a.num_query_heads, mq = a.max_query_length;
  if (row >= (int64_t)a.num_groups * mq * Hq) return;
  const int qh = (int)(row % Hq);
  const int qi = (int)((row / Hq) % mq);
  const int g = (int)(row / ((int64_t)Hq * mq));
  const int p0 = a.reduce_indptr[g], p1 = a.reduce_indptr[g + 1];
  if (p1 <= p0) return;
  const int qo0 = a.reduce_final_map[2 * g], qo1 = a.reduce_final_map[2 * g + 1];
  if (qi >= qo1 - qo0) return;
  const int32_t* pmap = a.reduce_partial_map + p0;
  const int D = 64 * NK;
  // Pieces in batches of kBatch whose loads are all in flight together,
  // folded with a running maximum (pieces with lse -inf are skipped).
  constexpr int kBatch = 8;
  const int n = p1 - p0;
  float M = kNegInf, tot = 0.0f, o[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) o[k] = 0.0f;
  for (int i0 = 0; i0 < n; i0 += kBatch) {
    float l[kBatch], x[kBatch][NK];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      l[j] = kNegInf;
#pragma unroll
      for (int k = 0; k < NK; ++k) x[j][k] = 0.0f;
      if (i0 + j < n) {  // wave-uniform
        const int64_t prow = (int64_t)pmap[i0 + j] + qi;
        l[j] = a.partial_lse[prow * a.stride_pl_row + qh];
        const float* r = a.partial_output + prow * a.stride_po_row + (int64_t)qh * D + lane;
#pragma unroll
        for (int k = 0; k < NK; ++k) x[j][k] = r[64 * k];
      }
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (l[j] == kNegInf) continue;
      const float Mn = fmaxf(M, l[j]);
      const float fold = M == kNegInf ? 0.0f : __expf(M - Mn);
      const float w = __expf(l[j] - Mn);
      tot = tot * fold + w;
#pragma unroll
      for (int k = 0; k < NK; ++k) o[k] = o[k] * fold + w * x[j][k];
      M = Mn;
    }
  }
  const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
  const int64_t off = (int64_t)(qo0 + qi) * a.stride_out_tok + (int64_t)qh * a.stride_out_head + lane;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const float v = o[k] * inv;
    if (a.output_dtype == PA_DTYPE_F32)
      ((float*)a.output)[off + 64 * k] = v;
    else if (a.output_dtype == PA_DTYPE_F16)
      ((uint16_t*)a.output)[off + 64 * k] = (uint16_t)f32_to_f16_bits(v);
    else
      ((uint16_t*)a.output)[off + 64 * k] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// Host side: the generic path takes every multiple of 64 from 64 to 512 and
// any column count.
static bool generic_head_ok(int d) { return d >= 64 && d <= 512 && d % 64 == 0; }

template <int D, bool PT>
static hipError_t launch_generic_partition(const GenArgs& g, dim3 grid, dim3 block, hipStream_t s) {
  if (g.owner == kGenOwnerRange)
    hipLaunchKernelGGL((pa_fp8_generic_partition_kernel<D, PT, kGenOwnerRange>), grid, block, 0, s, g);
  else if (g.owner == kGenOwnerSlots)
    hipLaunchKernelGGL((pa_fp8_generic_partition_kernel<D, PT, kGenOwnerSlots>), grid, block, 0, s, g);
  else
    hipLaunchKernelGGL((pa_fp8_generic_partition_kernel<D, PT, kGenSlot>), grid, block, 0, s, g);
  return hipGetLastError();
}
template <int D, bool PT>
static hipError_t launch_generic_worklist(const GenArgs& g, dim3 grid, dim3 block, hipStream_t s) {
  hipLaunchKernelGGL((pa_fp8_generic_worklist_kernel<D, PT>), grid, block, 0, s, g);
  return hipGetLastError();
}

template <int D, typename F>
static hipError_t generic_call(bool pt, F&& f) {
  return pt ? f(std::integral_constant<int, D>{}, std::true_type{}) : f(std::integral_constant<int, D>{}, std::false_type{});
}

template <typename F>
static hipError_t generic_dispatch(int d, bool pt, F&& f) {
  switch (d) {
    case 64: return generic_call<64>(pt, f);
    case 128: return generic_call<128>(pt, f);
    case 192: return generic_call<192>(pt, f);
    case 256: return generic_call<256>(pt, f);
    case 320: return generic_call<320>(pt, f);
    case 384: return generic_call<384>(pt, f);
    case 448: return generic_call<448>(pt, f);
    default: return generic_call<512>(pt, f);
  }
}

GenArgs gen_common(const void* query, const void* key_cache, const void* value_cache, const int32_t* block_tables,
                   const int32_t* kv_indptr, const int32_t* context_lengths, const float* key_scale,
                   const float* value_scale) {
  GenArgs g = {};
  g.query = query;
  g.key_cache = (const uint8_t*)key_cache;
  g.value_cache = (const uint8_t*)value_cache;
  g.block_tables = block_tables;
  g.kv_indptr = kv_indptr;
  g.context_lengths = context_lengths;
  g.key_scale = key_scale;
  g.value_scale = value_scale;
  return g;
}

template <typename Args>
void gen_shape(GenArgs& g, const Args& a) {
  g.stride_q_tok = a.stride_q_tok;
  g.stride_q_head = a.stride_q_head;
  g.stride_k_block = a.stride_k_block;
  g.stride_k_head = a.stride_k_head;
  g.stride_v_block = a.stride_v_block;
  g.stride_v_head = a.stride_v_head;
  g.stride_bt_seq = a.stride_bt_seq;
  g.stride_ks_block = a.stride_ks_block;
  g.stride_ks_head = a.stride_ks_head;
  g.num_seqs = a.num_seqs;
  g.num_kv_heads = a.num_kv_heads;
  g.query_length = a.query_length;
  g.query_group_size = a.query_group_size;
  g.block_size = a.block_size;
  g.num_blocks = a.num_blocks;
  g.max_blocks_per_seq = a.max_blocks_per_seq;
  g.sliding_window = a.sliding_window;
  g.trans_v = a.trans_v;
  g.query_dtype = a.query_dtype;
  g.softmax_scale = a.softmax_scale;
  g.output = a.output;
  g.output_dtype = a.output_dtype;
  g.stride_out_tok = a.stride_out_tok;
  g.stride_out_head = a.stride_out_head;
}

// Columns per kv head beyond the tuned kernels' 64, or a head size other
// than 128: the generic kernels (workgroup of one wave per 16-column block,
// up to four; the grid's second dimension tiles the blocks).
int generic_partition(const pa_fp8_partition_args& a, bool owner, hipStream_t s) {
  GenArgs g = gen_common(a.query, a.key_cache, a.value_cache, a.block_tables, a.kv_indptr, a.context_lengths,
                         a.key_scale, a.value_scale);
  gen_shape(g, a);
  g.exp_sums = a.exp_sums;
  g.max_logits = a.max_logits;
  g.tmp_out = a.tmp_out;
  g.tmp_dtype = a.tmp_dtype;
  g.stride_es_seq = a.stride_es_seq;
  g.stride_es_head = a.stride_es_head;
  g.stride_es_part = a.stride_es_part;
  g.stride_to_seq = a.stride_to_seq;
  g.stride_to_head = a.stride_to_head;
  g.stride_to_part = a.stride_to_part;
  g.stride_to_group = a.stride_to_group;
  g.num_partitions = a.num_partitions;
  g.owner = !owner ? kGenSlot : a.exp_sums ? kGenOwnerSlots : kGenOwnerRange;
  const int ncg = pa_cdiv(a.query_length * a.query_group_size, 16);
  const int64_t gx = (int64_t)a.num_seqs * a.num_kv_heads * (owner ? 1 : a.num_partitions);
  const int gy = pa_cdiv(ncg, 4);
  if (gx == 0) return PA_OK;
  if (gx > 0x7fffffffLL || gy > 65535) return PA_ERR_SHAPE;
  const dim3 grid((unsigned)gx, (unsigned)gy), block(64 * pa_min(ncg, 4));
  hipError_t err = generic_dispatch(a.head_size, a.per_token_kv != 0, [&](auto d, auto pt) {
    return launch_generic_partition<decltype(d)::value, decltype(pt)::value>(g, grid, block, s);
  });
  return err == hipSuccess ? PA_OK : (int)err;
}

int generic_worklist(const pa_fp8_stream_args& a, hipStream_t s) {
  GenArgs g = gen_common(a.query, a.key_cache, a.value_cache, a.block_tables, a.kv_indptr, a.context_lengths,
                         a.key_scale, a.value_scale);
  gen_shape(g, a);
  g.work_indptr = a.work_indptr;
  g.work_info = a.work_info;
  g.partition_indptr = a.partition_indptr;
  g.partial_output = a.partial_output;
  g.partial_lse = a.partial_lse;
  g.stride_po_row = a.stride_po_row;
  g.stride_pl_row = a.stride_pl_row;
  const int ncg = pa_cdiv(a.query_length * a.query_group_size, 16);
  const int gy = pa_cdiv(ncg, 4);
  if (gy > 65535) return PA_ERR_SHAPE;
  const dim3 grid((unsigned)a.num_workers, (unsigned)gy), block(64 * pa_min(ncg, 4));
  hipError_t err = generic_dispatch(a.head_size, a.per_token_kv != 0, [&](auto d, auto pt) {
    return launch_generic_worklist<decltype(d)::value, decltype(pt)::value>(g, grid, block, s);
  });
  return err == hipSuccess ? PA_OK : (int)err;
}

template <int NCG, bool PT, bool BS16, bool MULTI, int WAVES>
hipError_t launch_partition(const pa_fp8_partition_args& a, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((pa_fp8_partition_kernel<NCG, PT, BS16, kStages, MULTI, WAVES>), dim3(grid), dim3(64 * WAVES), 0,
                     s, a, a.block_tables, a.kv_indptr, a.context_lengths, a.key_scale, a.value_scale);
  return hipGetLastError();
}

template <int NCG, bool MULTI, int WAVES = kWaves>
hipError_t dispatch_ncg(const pa_fp8_partition_args& a, unsigned grid, hipStream_t s) {
  const bool pt = a.per_token_kv != 0;
  const bool bs16 = a.block_size == 16;
  if (pt)
    return bs16 ? launch_partition<NCG, true, true, MULTI, WAVES>(a, grid, s)
                : launch_partition<NCG, true, false, MULTI, WAVES>(a, grid, s);
  return bs16 ? launch_partition<NCG, false, true, MULTI, WAVES>(a, grid, s)
              : launch_partition<NCG, false, false, MULTI, WAVES>(a, grid, s);
}

// Device a launch on stream s runs on: the stream's own device, or the
// current device for the null stream.
hipError_t stream_device(hipStream_t s, int* dev) {
  if (s == nullptr) return hipGetDevice(dev);
  return hipStreamGetDevice(s, dev);
}

constexpr int kMaxDevices = 64;
// Compute-unit counts by device, filled on first use.  Every writer stores
// the same value for a device, so relaxed atomics suffice.
std::atomic<int> g_cu_count[kMaxDevices];

// Compute units of the device stream s runs on (-1 if unknown).
int device_cu_count(hipStream_t s) {
  int dev = 0;
  if (stream_device(s, &dev) != hipSuccess) return -1;
  const bool cached = dev >= 0 && dev < kMaxDevices;
  if (cached) {
    const int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return -1;
  if (cached) g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Query DMA instructions per piece of a streaming launch (4 columns each).
int stream_lds_bytes(int nq, bool per_token) {
  const int stage = kKBytes + kVBytes + (per_token ? kScaleBytes : 0);
  return stream_waves(nq) * (kStages * stage + 2 * nq * 1024);
}

template <bool PT, bool BS16, bool WL, int NQ>
hipError_t launch_stream(const pa_fp8_stream_args& a, unsigned grid, hipStream_t s, int32_t* desc, float* po,
                         float* pl) {
  hipLaunchKernelGGL((pa_fp8_stream_kernel<PT, BS16, WL, NQ>), dim3(grid), dim3(64 * stream_waves(NQ)), 0, s, a,
                     a.block_tables, a.kv_indptr, a.context_lengths, a.key_scale, a.value_scale, a.work_indptr,
                     a.work_info, a.partition_indptr, desc, po, pl, a.output);
  return hipGetLastError();
}

template <bool WL, int NQ>
hipError_t dispatch_stream_nq(const pa_fp8_stream_args& a, unsigned grid, hipStream_t s, int32_t* desc, float* po,
                              float* pl) {
  const bool pt = a.per_token_kv != 0;
  const bool bs16 = a.block_size == 16;
  if (pt)
    return bs16 ? launch_stream<true, true, WL, NQ>(a, grid, s, desc, po, pl)
                : launch_stream<true, false, WL, NQ>(a, grid, s, desc, po, pl);
  return bs16 ? launch_stream<false, true, WL, NQ>(a, grid, s, desc, po, pl)
              : launch_stream<false, false, WL, NQ>(a, grid, s, desc, po, pl);
}

template <bool WL>
hipError_t dispatch_stream(const pa_fp8_stream_args& a, unsigned grid, hipStream_t s, int32_t* desc, float* po,
                           float* pl) {
  switch (stream_nq(a.query_length * a.query_group_size)) {
    case 1: return dispatch_stream_nq<WL, 1>(a, grid, s, desc, po, pl);
    case 2: return dispatch_stream_nq<WL, 2>(a, grid, s, desc, po, pl);
    default: return dispatch_stream_nq<WL, 4>(a, grid, s, desc, po, pl);
  }
}

template <int NW, bool PT, bool BS16, bool WL>
hipError_t launch_coop(const pa_fp8_stream_args& a, unsigned grid, hipStream_t s, int32_t* desc, float* po,
                       float* pl) {
  hipLaunchKernelGGL((pa_fp8_coop_kernel<NW, PT, BS16, WL>), dim3(grid), dim3(64 * NW), 0, s, a, a.block_tables,
                     a.kv_indptr, a.context_lengths, a.key_scale, a.value_scale, a.work_indptr, a.work_info,
                     a.partition_indptr, desc, po, pl, a.output);
  return hipGetLastError();
}

template <int NW, bool WL>
hipError_t dispatch_coop_nw(const pa_fp8_stream_args& a, unsigned grid, hipStream_t s, int32_t* desc, float* po,
                            float* pl) {
  const bool pt = a.per_token_kv != 0;
  const bool bs16 = a.block_size == 16;
  if (pt)
    return bs16 ? launch_coop<NW, true, true, WL>(a, grid, s, desc, po, pl)
                : launch_coop<NW, true, false, WL>(a, grid, s, desc, po, pl);
  return bs16 ? launch_coop<NW, false, true, WL>(a, grid, s, desc, po, pl)
              : launch_coop<NW, false, false, WL>(a, grid, s, desc, po, pl);
}

// Waves per cooperative workgroup: one per 16-column query block (three
// blocks run on four waves, the fourth computing only masked columns).
int coop_waves(int eq) { return eq <= 32 ? 2 : 4; }

// Resident cooperative workgroups per CU of a balanced launch (LDS: nine
// chunk slots of up to 8.4 KiB for four waves, six for two).
int coop_per_cu(int nw) { return coop_wgs_per_cu(nw, false); }

// Workgroups of a work-list launch: as many as fit on the GPU at once (one
// per CU for eight waves, three for three), at most one per bin.
unsigned bin_workgroups(int bins, hipStream_t s) {
  const int cus = device_cu_count(s);
  const int per_cu = kBinWaves >= 8 ? 1 : (kBinWaves >= 4 ? 2 : 3);
  const int fit = cus > 0 ? cus * per_cu : bins;
  return (unsigned)(bins < fit ? bins : fit);
}

template <bool PT, bool BS16>
hipError_t launch_bin(const pa_fp8_stream_args& a, hipStream_t s) {
  hipLaunchKernelGGL((pa_fp8_bin_kernel<PT, BS16>), dim3(bin_workgroups(a.num_workers, s)), dim3(64 * kBinWaves), 0, s, a,
                     a.block_tables, a.kv_indptr, a.context_lengths, a.key_scale, a.value_scale, a.work_indptr,
                     a.work_info, a.partition_indptr, a.partial_output, a.partial_lse, a.output);
  return hipGetLastError();
}

// One launch of the balanced split: per-wave runs (<= 16 columns) or
// cooperative workgroup runs.
hipError_t dispatch_balanced(const pa_fp8_stream_args& a, hipStream_t s, int32_t* desc, float* po, float* pl) {
  const int eq = a.query_length * a.query_group_size;
  if (eq <= 16)
    return dispatch_stream<false>(a, (unsigned)pa_cdiv(a.num_workers, stream_waves(stream_nq(eq))), s, desc, po, pl);
  return coop_waves(eq) == 2 ? dispatch_coop_nw<2, false>(a, (unsigned)a.num_workers, s, desc, po, pl)
                             : dispatch_coop_nw<4, false>(a, (unsigned)a.num_workers, s, desc, po, pl);
}

// One launch of the work-list decode, one workgroup per bin: the bin
// kernel (<= 16 columns) or the cooperative kernel.
hipError_t dispatch_worklist(const pa_fp8_stream_args& a, hipStream_t s) {
  const int eq = a.query_length * a.query_group_size;
  if (eq <= 16) {
    const bool pt = a.per_token_kv != 0, bs16 = a.block_size == 16;
    if (pt) return bs16 ? launch_bin<true, true>(a, s) : launch_bin<true, false>(a, s);
    return bs16 ? launch_bin<false, true>(a, s) : launch_bin<false, false>(a, s);
  }
  return coop_waves(eq) == 2
             ? dispatch_coop_nw<2, true>(a, (unsigned)a.num_workers, s, nullptr, a.partial_output, a.partial_lse)
             : dispatch_coop_nw<4, true>(a, (unsigned)a.num_workers, s, nullptr, a.partial_output, a.partial_lse);
}

// Checks shared by both streaming entry points.
// generic_ok: the launch may run on the generic kernels (head sizes 64 ..
// 256, any column count); the balanced decode may not.
int check_stream_args(const pa_fp8_stream_args* a, bool generic_ok = false) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (!a->output || !a->query || !a->key_cache || !a->value_cache || !a->block_tables || !a->context_lengths ||
      !a->key_scale || !a->value_scale)
    return PA_ERR_NULL_ARG;
  if (!(generic_ok ? generic_head_ok(a->head_size) : a->head_size == kHead)) return PA_ERR_HEAD_SIZE;
  const int bs = a->block_size;
  if (!(bs == 16 || (bs >= 32 && bs <= 1024 && (bs & (bs - 1)) == 0))) return PA_ERR_BLOCK_SIZE;
  if (a->num_seqs < 0 || a->num_kv_heads <= 0 || a->query_length <= 0 || a->query_group_size <= 0 ||
      a->num_blocks <= 0 || a->max_blocks_per_seq <= 0 || a->sliding_window < 0 || a->num_workers <= 0)
    return PA_ERR_SHAPE;
  if (!generic_ok && a->query_length * a->query_group_size > 64) return PA_ERR_GROUP;
  if (a->query_dtype != PA_DTYPE_BF16 && a->query_dtype != PA_DTYPE_F16) return PA_ERR_DTYPE;
  if (a->output_dtype != PA_DTYPE_BF16 && a->output_dtype != PA_DTYPE_F16 && a->output_dtype != PA_DTYPE_F32)
    return PA_ERR_DTYPE;
  if (!aligned16(a->query) || (a->stride_q_tok % 8) || (a->stride_q_head % 8)) return PA_ERR_ALIGN;
  if (!aligned16(a->key_cache) || !aligned16(a->value_cache) || (a->stride_k_block % 16) ||
      (a->stride_k_head % 16) || (a->stride_v_block % 16) || (a->stride_v_head % 16))
    return PA_ERR_ALIGN;
  if (a->per_token_kv &&
      (!aligned16(a->key_scale) || !aligned16(a->value_scale) || (a->stride_ks_block % 4) || (a->stride_ks_head % 4)))
    return PA_ERR_ALIGN;
  if (!aligned16(a->output) || (a->stride_out_tok % 4) || (a->stride_out_head % 4)) return PA_ERR_ALIGN;
  // a page's offset is computed as a 32 x 32-bit product
  const int64_t smax = 0x7fffffffLL;
  if (a->stride_k_block < 0 || a->stride_k_block > smax || a->stride_v_block < 0 || a->stride_v_block > smax ||
      (a->per_token_kv && (a->stride_ks_block < 0 || a->stride_ks_block > smax)))
    return PA_ERR_SHAPE;
  return PA_OK;
}

// Balanced workspace: pair descriptors, then partial lse (float32), then
// partial rows (bf16), two of each per run.
struct BalancedLayout {
  int64_t desc, lse, out, total;
};
BalancedLayout balanced_layout(int B, int H, int eq, int nw) {
  auto up = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  BalancedLayout l;
  l.desc = 0;
  l.lse = up((int64_t)B * H * 2 * 4);
  l.out = l.lse + up((int64_t)2 * nw * eq * 4);
  l.total = l.out + (int64_t)2 * nw * eq * kHead * 2;  // bf16 rows
  return l;
}

// Device scratch of pa_fp8_decode_balanced_static: the balanced split's
// workspace (pair descriptors, partial lse, partial rows) for callers that
// cannot allocate.  Each device holds its own copy for the life of the
// process; the kernels take its device address (kept per device below),
// never this name, which in host code is only a stand-in.
constexpr int64_t kStaticScratchBytes = (int64_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the scratch on the device stream s runs on, looked up
// once per device with that device current (the caller's current device is
// restored afterwards).
int static_scratch(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = stream_device(s, &dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return PA_ERR_SHAPE;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int cur = 0;
      e = hipGetDevice(&cur);
      if (e != hipSuccess) return (int)e;
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      const hipError_t back = cur != dev ? hipSetDevice(cur) : hipSuccess;
      if (e != hipSuccess) return (int)e;
      if (back != hipSuccess) return (int)back;
      if (p == nullptr) return PA_ERR_NULL_ARG;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return PA_OK;
}

}  // namespace

PA_CHECK_DEFINE_TAKE(pa_violations_paged)

extern "C" {

int pa_fp8_debug_violations(unsigned int* bits) {
  if (!bits) return PA_ERR_NULL_ARG;
  *bits = 0;
  int rc = pa_violations_paged(bits);
  if (rc == 0) rc = pa_violations_mla(bits);
  if (rc == 0) rc = pa_violations_rope_cache(bits);
  if (rc == 0) rc = pa_violations_qk_norm_rope(bits);
  return rc;
}

int pa_fp8_checked_build(void) {
#ifdef PA_FP8_CHECKED
  return 1;
#else
  return 0;
#endif
}

int pa_fp8_decode_partition(const pa_fp8_partition_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (!a->query || !a->key_cache || !a->value_cache || !a->block_tables || !a->context_lengths || !a->key_scale ||
      !a->value_scale)
    return PA_ERR_NULL_ARG;
  const int spw = a->slots_per_workgroup;
  if (spw <= 0 || a->num_partitions <= 0) return PA_ERR_SHAPE;
  const bool owner = spw >= a->num_partitions;  // one workgroup covers every slot
  const bool partials = a->exp_sums || a->max_logits || a->tmp_out;
  if (partials && (!a->exp_sums || !a->max_logits || !a->tmp_out)) return PA_ERR_NULL_ARG;
  if (!owner && !partials) return PA_ERR_NULL_ARG;   // slot partials are the only result
  if (a->output != nullptr && !owner) return PA_ERR_SHAPE;  // output needs every slot
  if (!partials && a->output == nullptr) return PA_ERR_NULL_ARG;
  const bool fused = !partials;
  if (!generic_head_ok(a->head_size)) return PA_ERR_HEAD_SIZE;
  const int bs = a->block_size;
  if (!(bs == 16 || (bs >= 32 && bs <= 1024 && (bs & (bs - 1)) == 0))) return PA_ERR_BLOCK_SIZE;
  if (a->num_seqs < 0 || a->num_kv_heads <= 0 || a->num_partitions <= 0 || a->query_length <= 0 ||
      a->query_group_size <= 0 || a->num_blocks <= 0 || a->max_blocks_per_seq <= 0 || a->sliding_window < 0)
    return PA_ERR_SHAPE;
  const int eq = a->query_length * a->query_group_size;
  const bool generic = a->head_size != kHead || eq > 64;
  if (a->query_dtype != PA_DTYPE_BF16 && a->query_dtype != PA_DTYPE_F16) return PA_ERR_DTYPE;
  if (!fused && a->tmp_dtype != PA_DTYPE_BF16 && a->tmp_dtype != PA_DTYPE_F32) return PA_ERR_DTYPE;
  if (a->output && a->output_dtype != PA_DTYPE_BF16 && a->output_dtype != PA_DTYPE_F16 && a->output_dtype != PA_DTYPE_F32)
    return PA_ERR_DTYPE;
  // 16-byte vector accesses: query rows, cache pages, scale rows, partials.
  if (!aligned16(a->query) || (a->stride_q_tok % 8) || (a->stride_q_head % 8)) return PA_ERR_ALIGN;
  if (!aligned16(a->key_cache) || !aligned16(a->value_cache) || (a->stride_k_block % 16) ||
      (a->stride_k_head % 16) || (a->stride_v_block % 16) || (a->stride_v_head % 16))
    return PA_ERR_ALIGN;
  if (a->per_token_kv &&
      (!aligned16(a->key_scale) || !aligned16(a->value_scale) || (a->stride_ks_block % 4) || (a->stride_ks_head % 4)))
    return PA_ERR_ALIGN;
  if (a->output != nullptr) {
    if (!aligned16(a->output) || (a->stride_out_tok % 8) || (a->stride_out_head % 8)) return PA_ERR_ALIGN;
  }
  if (!fused) {
    if (!aligned16(a->tmp_out) || (a->stride_to_group % 8) || (a->stride_to_part % 8) || (a->stride_to_head % 8) ||
        (a->stride_to_seq % 8))
      return PA_ERR_ALIGN;
  }
  if (generic) return generic_partition(*a, owner, (hipStream_t)stream);
  const int64_t grid = (int64_t)a->num_seqs * a->num_kv_heads * pa_cdiv(a->num_partitions, spw);
  if (grid == 0) return PA_OK;
  if (grid > 0x7fffffffLL) return PA_ERR_SHAPE;
  const int ncg = (eq + 15) / 16;
  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  // A launch of at most one workgroup per CU runs 8-wave workgroups (one
  // per CU by LDS): twice the loads in flight per CU of a 4-wave one.
  const int cus = ncg == 1 ? device_cu_count(s) : -1;
  if (cus > 0 && grid <= cus) {
    const bool multi8 = pa_min(spw, a->num_partitions) > 8;
    err = multi8 ? dispatch_ncg<1, true, 8>(*a, (unsigned)grid, s) : dispatch_ncg<1, false, 8>(*a, (unsigned)grid, s);
    return err == hipSuccess ? PA_OK : (int)err;
  }
  // A wave owns several slots only when a workgroup covers more slots than
  // it has waves; that form keeps a second accumulator set, built for one
  // 16-column group only.
  const bool multi = pa_min(spw, a->num_partitions) > kWaves;
  if (multi && ncg > 1) return PA_ERR_GROUP;
  if (multi) {
    err = dispatch_ncg<1, true>(*a, (unsigned)grid, s);
  } else {
    switch (ncg) {
      case 1: err = dispatch_ncg<1, false>(*a, (unsigned)grid, s); break;
      case 2: err = dispatch_ncg<2, false>(*a, (unsigned)grid, s); break;
      case 3: err = dispatch_ncg<3, false>(*a, (unsigned)grid, s); break;
      default: err = dispatch_ncg<4, false>(*a, (unsigned)grid, s); break;
    }
  }
  return err == hipSuccess ? PA_OK : (int)err;
}

int pa_fp8_decode_reduce(const pa_fp8_reduce_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (!a->output || !a->exp_sums || !a->max_logits || !a->tmp_out) return PA_ERR_NULL_ARG;
  if (!generic_head_ok(a->head_size)) return PA_ERR_HEAD_SIZE;
  if (a->num_seqs < 0 || a->num_kv_heads <= 0 || a->num_partitions <= 0 || a->query_length <= 0 ||
      a->query_group_size <= 0)
    return PA_ERR_SHAPE;
  if (a->output_dtype != PA_DTYPE_BF16 && a->output_dtype != PA_DTYPE_F16 && a->output_dtype != PA_DTYPE_F32)
    return PA_ERR_DTYPE;
  if (a->tmp_dtype != PA_DTYPE_BF16 && a->tmp_dtype != PA_DTYPE_F32) return PA_ERR_DTYPE;
  const int64_t rows = (int64_t)a->num_seqs * a->num_kv_heads * a->query_length * a->query_group_size;
  if (rows == 0) return PA_OK;
  const int64_t grid = (rows + 3) / 4;
  if (grid > 0x7fffffffLL) return PA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const dim3 g1((unsigned)grid), b1(256);
  switch (a->head_size) {
    case 64: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<1>, g1, b1, 0, s, *a); break;
    case 192: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<3>, g1, b1, 0, s, *a); break;
    case 256: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<4>, g1, b1, 0, s, *a); break;
    case 320: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<5>, g1, b1, 0, s, *a); break;
    case 384: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<6>, g1, b1, 0, s, *a); break;
    case 448: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<7>, g1, b1, 0, s, *a); break;
    case 512: hipLaunchKernelGGL(pa_fp8_generic_lse_reduce_kernel<8>, g1, b1, 0, s, *a); break;
    default: hipLaunchKernelGGL(pa_fp8_lse_reduce_kernel, g1, b1, 0, s, *a); break;
  }
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? PA_OK : (int)err;
}

int pa_fp8_stream_workers(int num_cu, int query_length, int query_group_size, int per_token_kv) {
  if (num_cu <= 0 || query_length <= 0 || query_group_size <= 0) return PA_ERR_SHAPE;
  const int eq = query_length * query_group_size;
  if (eq > 64) return PA_ERR_GROUP;
  if (eq > 16) return num_cu * coop_per_cu(coop_waves(eq));
  const int lds = stream_lds_bytes(stream_nq(eq), per_token_kv != 0);
  const int per_cu = 160 * 1024 / lds >= 2 ? 2 : 1;
  return num_cu * per_cu * stream_waves(stream_nq(eq));
}

int64_t pa_fp8_balanced_workspace_bytes(int num_seqs, int num_kv_heads, int query_length, int query_group_size,
                                        int num_workers) {
  if (num_seqs < 0 || num_kv_heads <= 0 || query_length <= 0 || query_group_size <= 0 || num_workers <= 0)
    return PA_ERR_SHAPE;
  return balanced_layout(num_seqs, num_kv_heads, query_length * query_group_size, num_workers).total;
}

int pa_fp8_decode_balanced(const pa_fp8_stream_args* a, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_stream_args(a);
  if (rc != PA_OK) return rc;
  if (a->num_seqs > 1024) return PA_ERR_SHAPE;
  if (!workspace) return PA_ERR_NULL_ARG;
  if (((uintptr_t)workspace & 255u) != 0) return PA_ERR_ALIGN;
  const int eq = a->query_length * a->query_group_size;
  const BalancedLayout l = balanced_layout(a->num_seqs, a->num_kv_heads, eq, a->num_workers);
  if (workspace_bytes < l.total) return PA_ERR_SHAPE;
  if (a->num_seqs == 0) return PA_OK;
  unsigned char* ws = (unsigned char*)workspace;
  int32_t* desc = (int32_t*)(ws + l.desc);
  float* pl = (float*)(ws + l.lse);
  float* po = (float*)(ws + l.out);  // bf16 rows: store_piece<false> writes them as such
  hipError_t err = dispatch_balanced(*a, (hipStream_t)stream, desc, po, pl);
  return err == hipSuccess ? PA_OK : (int)err;
}

int pa_fp8_merge_balanced(const pa_fp8_stream_args* a, const void* workspace, int64_t workspace_bytes,
                          void* stream) {
  int rc = check_stream_args(a);
  if (rc != PA_OK) return rc;
  if (a->num_seqs > 1024) return PA_ERR_SHAPE;
  if (!workspace) return PA_ERR_NULL_ARG;
  if (((uintptr_t)workspace & 255u) != 0) return PA_ERR_ALIGN;
  const int eq = a->query_length * a->query_group_size;
  const BalancedLayout l = balanced_layout(a->num_seqs, a->num_kv_heads, eq, a->num_workers);
  if (workspace_bytes < l.total) return PA_ERR_SHAPE;
  // Up to 4 columns: one load per piece covers them (all lanes busy); else
  // 16 columns per wave, four loads per piece.
  const bool narrow = eq <= 4;
  const int cols = narrow ? 4 : 16;
  const int64_t rows = (int64_t)a->num_seqs * a->num_kv_heads * ((eq + cols - 1) / cols);
  if (rows == 0) return PA_OK;
  const unsigned char* ws = (const unsigned char*)workspace;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (narrow)
    hipLaunchKernelGGL(pa_fp8_segment_merge_kernel<1>, grid, dim3(256), 0, (hipStream_t)stream, *a,
                       (const int32_t*)(ws + l.desc), (const uint16_t*)(ws + l.out), (const float*)(ws + l.lse));
  else
    hipLaunchKernelGGL(pa_fp8_segment_merge_kernel<4>, grid, dim3(256), 0, (hipStream_t)stream, *a,
                       (const int32_t*)(ws + l.desc), (const uint16_t*)(ws + l.out), (const float*)(ws + l.lse));
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? PA_OK : (int)err;
}

int pa_fp8_decode_balanced_static(const pa_fp8_stream_args* a, void* stream) {
  int rc = check_stream_args(a);
  if (rc != PA_OK) return rc;
  if (a->num_seqs > 1024) return PA_ERR_SHAPE;
  const int eq = a->query_length * a->query_group_size;
  const BalancedLayout l = balanced_layout(a->num_seqs, a->num_kv_heads, eq, a->num_workers);
  if (l.total > kStaticScratchBytes) return PA_ERR_SCRATCH;
  if (a->num_seqs == 0) return PA_OK;
  void* ws = nullptr;
  rc = static_scratch((hipStream_t)stream, &ws);
  if (rc != PA_OK) return rc;
  rc = pa_fp8_decode_balanced(a, ws, l.total, stream);
  if (rc != PA_OK) return rc;
  return pa_fp8_merge_balanced(a, ws, l.total, stream);
}

int64_t pa_fp8_static_scratch_bytes(void) { return kStaticScratchBytes; }

int pa_fp8_decode_worklist(const pa_fp8_stream_args* a, void* stream) {
  int rc = check_stream_args(a, true);
  if (rc != PA_OK) return rc;
  if (!a->work_indptr || !a->work_info || !a->partition_indptr || !a->partial_output || !a->partial_lse)
    return PA_ERR_NULL_ARG;
  if (!aligned16(a->partial_output) || (a->stride_po_row % 4)) return PA_ERR_ALIGN;
  if (a->num_seqs == 0) return PA_OK;
  if (a->head_size != kHead || a->query_length * a->query_group_size > 64)
    return generic_worklist(*a, (hipStream_t)stream);
  hipError_t err = dispatch_worklist(*a, (hipStream_t)stream);
  return err == hipSuccess ? PA_OK : (int)err;
}

int pa_fp8_reduce_worklist(const pa_fp8_worklist_reduce_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (!a->output || !a->partial_output || !a->partial_lse || !a->reduce_indptr || !a->reduce_final_map ||
      !a->reduce_partial_map)
    return PA_ERR_NULL_ARG;
  if (!generic_head_ok(a->head_size)) return PA_ERR_HEAD_SIZE;
  if (a->num_groups < 0 || a->num_query_heads <= 0 || a->max_query_length <= 0) return PA_ERR_SHAPE;
  if (a->output_dtype != PA_DTYPE_BF16 && a->output_dtype != PA_DTYPE_F16 && a->output_dtype != PA_DTYPE_F32)
    return PA_ERR_DTYPE;
  if (((uintptr_t)a->partial_output & 7u) || (a->stride_po_row % 2) || ((uintptr_t)a->output & 7u) ||
      (a->stride_out_tok % 2) || (a->stride_out_head % 2))
    return PA_ERR_ALIGN;
  const int64_t rows = (int64_t)a->num_groups * a->max_query_length * a->num_query_heads;
  if (rows == 0) return PA_OK;
  if ((rows + 3) / 4 > 0x7fffffffLL) return PA_ERR_SHAPE;
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  // Head size 128 and at least 128 output rows per group (query length x
  // query heads; multi-token prediction): eight heads per wave, two pieces
  // in flight.  With fewer rows per group the one-row waves are few and
  // their eight pieces in flight suit groups cut into many pieces.  Measured
  // (kernel us): bench workload c5_mtp_p1024, 256 rows per group, 32 -> 12.8;
  // c3_ragged_p1024, 32 rows per group and up to about 30 pieces, 4.7 with
  // one row per wave against 7.2 with eight heads.
  if (a->head_size == kHead && a->num_query_heads % 8 == 0 &&
      (int64_t)a->max_query_length * a->num_query_heads >= 128 && ((uintptr_t)a->partial_output & 15u) == 0 &&
      ((uintptr_t)a->output & 15u) == 0 && a->stride_po_row % 4 == 0 && a->stride_out_tok % 4 == 0 &&
      a->stride_out_head % 4 == 0) {
    const int64_t waves = rows / 8;
    hipLaunchKernelGGL(pa_fp8_worklist_reduce8_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, *a);
    hipError_t err = hipGetLastError();
    return err == hipSuccess ? PA_OK : (int)err;
  }
  switch (a->head_size) {
    case 64: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<1>, grid, dim3(256), 0, s, *a); break;
    case 192: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<3>, grid, dim3(256), 0, s, *a); break;
    case 256: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<4>, grid, dim3(256), 0, s, *a); break;
    case 320: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<5>, grid, dim3(256), 0, s, *a); break;
    case 384: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<6>, grid, dim3(256), 0, s, *a); break;
    case 448: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<7>, grid, dim3(256), 0, s, *a); break;
    case 512: hipLaunchKernelGGL(pa_fp8_generic_worklist_reduce_kernel<8>, grid, dim3(256), 0, s, *a); break;
    default: hipLaunchKernelGGL(pa_fp8_worklist_reduce_kernel, grid, dim3(256), 0, s, *a); break;
  }
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? PA_OK : (int)err;
}

int pa_fp8_worklist_sizes(int num_seqs, int num_kv_heads, int num_cu, int* max_works, int* max_split_tiles) {
  if (!max_works || !max_split_tiles) return PA_ERR_NULL_ARG;
  if (num_seqs < 0 || num_kv_heads <= 0 || num_cu <= 0) return PA_ERR_SHAPE;
  pa_worklist_sizes(num_seqs, num_kv_heads, num_cu, max_works, max_split_tiles);
  return PA_OK;
}

int pa_fp8_plan_worklist(const int32_t* context_lengths, int num_seqs, int num_kv_heads, int query_group_size,
                         int query_length, int num_cu, int kv_granularity, int32_t* work_indptr, int32_t* work_info,
                         int32_t* reduce_indptr, int32_t* reduce_final_map, int32_t* reduce_partial_map) {
  if (!work_indptr || !work_info || !reduce_indptr || !reduce_final_map || !reduce_partial_map) return PA_ERR_NULL_ARG;
  if (num_seqs > 0 && !context_lengths) return PA_ERR_NULL_ARG;
  if (num_seqs < 0 || num_kv_heads <= 0 || query_group_size <= 0 || query_length <= 0 || num_cu <= 0 ||
      (num_cu % num_kv_heads) != 0 || kv_granularity <= 0 || (kv_granularity & (kv_granularity - 1)) != 0)
    return PA_ERR_SHAPE;
  const int n = pa_worklist_plan(context_lengths, num_seqs, num_kv_heads, query_group_size, query_length, num_cu,
                                 kv_granularity, work_indptr, work_info, reduce_indptr, reduce_final_map,
                                 reduce_partial_map);
  return n < 0 ? PA_ERR_SHAPE : n;
}

int pa_fp8_recommended_splits(int num_seqs, int num_kv_heads, int split_kv_blocks, int sliding_window,
                              int partition_tokens, int query_length, int num_cu) {
  return pa_plan_splits(num_seqs, num_kv_heads, split_kv_blocks, sliding_window, partition_tokens, query_length,
                        num_cu);
}

int pa_fp8_plan_slot(int context_length, int num_partitions, int slot, int sliding_window, int query_length, int* t0,
                     int* t1) {
  if (!t0 || !t1) return PA_ERR_NULL_ARG;
  if (num_partitions <= 0 || slot < 0 || context_length < 0 || query_length <= 0) return PA_ERR_SHAPE;
  pa_plan_slot_tokens(context_length, num_partitions, slot, sliding_window, query_length, t0, t1);
  return PA_OK;
}

int pa_fp8_plan_visible(int context_length, int qi, int query_length, int sliding_window, int* lo, int* hi) {
  if (!lo || !hi) return PA_ERR_NULL_ARG;
  pa_plan_visible(context_length, qi, query_length, sliding_window, lo, hi);
  return PA_OK;
}

const char* pa_fp8_version(void) { return "pa_fp8 1.0 gfx950 abi" "1"; }

const char* pa_fp8_error_string(int code) {
  switch (code) {
    case PA_OK: return "ok";
    case PA_ERR_NULL_ARG: return "a required pointer is NULL";
    case PA_ERR_HEAD_SIZE: return "unsupported head_size (a multiple of 64 in [64, 512]; the balanced decode: 128)";
    case PA_ERR_BLOCK_SIZE: return "unsupported block_size (16 or a power of two in [32, 1024])";
    case PA_ERR_GROUP:
      return "query_length * query_group_size above the entry point's limit (64 for the balanced decode and "
             "pa_fp8_stream_workers; 16 for partition workgroups whose waves walk several slots)";
    case PA_ERR_DTYPE: return "unsupported dtype";
    case PA_ERR_SHAPE: return "invalid dimension";
    case PA_ERR_ALIGN: return "pointer or stride not 16-byte aligned";
    case PA_ERR_ABI: return "abi_version mismatch";
    case PA_ERR_SCRATCH: return "the call needs more workspace than the library's static scratch (64 MiB)";
    default: return hipGetErrorString((hipError_t)code);
  }
}

}  // extern "C"
