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

#include "pa_fp8.h"
#include "pa_plan.h"

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
constexpr int kThreads = 64 * kWaves;
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

// x[0..7] -> (hi, lo) with x ~= hi + lo, both packed e4m3fn, byte i = x[i].
__device__ __forceinline__ void split8_fp8(const float* x, long& hi, long& lo) {
  uint32_t h0 = pack4_fp8(x[0], x[1], x[2], x[3]);
  uint32_t h1 = pack4_fp8(x[4], x[5], x[6], x[7]);
  f32x2 b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, false);
  f32x2 b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h0, true);
  f32x2 b2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, false);
  f32x2 b3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h1, true);
  uint32_t l0 = pack4_fp8(x[0] - b0[0], x[1] - b0[1], x[2] - b1[0], x[3] - b1[1]);
  uint32_t l1 = pack4_fp8(x[4] - b2[0], x[5] - b2[1], x[6] - b3[0], x[7] - b3[1]);
  hi = (long)((uint64_t)h0 | ((uint64_t)h1 << 32));
  lo = (long)((uint64_t)l0 | ((uint64_t)l1 << 32));
}

__device__ __forceinline__ f32x4 mfma_fp8(long a, long b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

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

__device__ __forceinline__ void lds_dma16(const void* gsrc, LDS_AS void* ldst) {
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
template <int NCG, bool PER_TOKEN, bool BS16, int STAGES, bool MULTI>
__global__ __launch_bounds__(kThreads) void pa_fp8_partition_kernel(const pa_fp8_partition_args a,
                                                                    const int32_t* __restrict__ block_tables,
                                                                    const int32_t* __restrict__ kv_indptr,
                                                                    const int32_t* __restrict__ context_lengths,
                                                                    const float* __restrict__ key_scale,
                                                                    const float* __restrict__ value_scale) {
  constexpr int kStageBytes = kKBytes + kVBytes + (PER_TOKEN ? kScaleBytes : 0);
  constexpr int kWaveBytes = STAGES * kStageBytes;
  constexpr int kMergeBytes = 2 * kWaves * 16 * 4 + kWaves * kHead * 16 * 4;
  constexpr int kSmemBytes = kWaves * kWaveBytes > kMergeBytes ? kWaves * kWaveBytes : kMergeBytes;
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
  const int wslot = nslots >= kWaves ? 1 : kWaves / nslots;
  const int groups = kWaves / wslot;
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
      for (int idx = tid; idx < eq * (kHead / 8); idx += kThreads) {
        const int e = idx / (kHead / 8);
        const int d0 = (idx % (kHead / 8)) * 8;
        if (want_partials) store_partial8(a, b, h, zs, e, d0, z);
        if (direct_out) store_output8(a, b, h, e, d0, z);
      }
      if (want_partials)
        for (int e = tid; e < eq; e += kThreads) store_stats(a, b, h, zs, e, 0.0f, kNegInf);
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
        lds_dma16(base + (int64_t)pg2 * a.stride_ks_block + sidx, ss);
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

  float m2[NCG], lsum[NCG];
  f32x4 acc[NCG][8];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    m2[cg] = kNegInf;
    lsum[cg] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[cg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float vsmax = 0.0f;  // running max of per-token value scales (per wave, per slot)
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
  // B operand of the 16x16x128 QK product: lane (grp, c) holds the 32 head
  // dims of 16-dim chunks grp and grp+4 of column c, in the byte order of
  // the key rows read below.
  i32x8 qhi8[NCG], qlo8[NCG];
  float qfac[NCG];   // base-2 logit factor per column
  int vis_lo[NCG], vis_hi[NCG];
  const float k_tensor_scale = PER_TOKEN ? 1.0f : key_scale[0];
  const float v_tensor_scale = PER_TOKEN ? 1.0f : value_scale[0];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    const int e = cg * 16 + c16;
    const bool valid = e < eq;
    const int qi = valid ? e / gqa : 0;
    float v[32];
    if (a.query_dtype == PA_DTYPE_F16) {
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
    // Power-of-two scale putting amax into [128, 256): exact in fp32.
    int sexp = 261 - (int)((__float_as_uint(amax) >> 23) & 0xffu);
    sexp = sexp < 1 ? 1 : (sexp > 254 ? 254 : sexp);
    const float sq = amax > 0.0f ? __uint_as_float((uint32_t)sexp << 23) : 1.0f;
#pragma unroll
    for (int sI = 0; sI < 4; ++sI) {
      float xs[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xs[i] = v[8 * sI + i] * sq;
      long hi, lo;
      split8_fp8(xs, hi, lo);
      qhi8[cg][2 * sI] = (int)(uint32_t)hi;
      qhi8[cg][2 * sI + 1] = (int)(uint32_t)((uint64_t)hi >> 32);
      qlo8[cg][2 * sI] = (int)(uint32_t)lo;
      qlo8[cg][2 * sI + 1] = (int)(uint32_t)((uint64_t)lo >> 32);
    }
    qfac[cg] = a.softmax_scale * kLog2e * k_tensor_scale / sq;
    int lo = 0, hi = 0;
    if (valid) pa_plan_visible(ctx, qi, ql, W, &lo, &hi);
    vis_lo[cg] = lo;
    vis_hi[cg] = hi;
  }
  // Chunks inside [lo_max, hi_min) are visible to every query column: no
  // masking there.  lo and hi grow with qi, so the extremes come from the
  // last and the first query.
  int lo_max, hi_min;
  {
    int t0q, t1q;
    pa_plan_visible(ctx, ql - 1, ql, W, &lo_max, &t1q);
    pa_plan_visible(ctx, 0, ql, W, &t0q, &hi_min);
  }

  // Key row r of QK tile t (0, 1) is chunk token 8*(r/4) + 4t + r%4: that
  // token's 16-byte pieces for dim chunks grp and grp+4.
  const int krow = (c16 >> 3) * kKHalf + (8 * ((c16 >> 2) & 1) + (c16 & 3)) * 16;

  int gc = 0;  // chunks of this wave computed so far
  for (int l = gid; l < nslots; l += groups) {
    const int z = zs + l;
    int cbeg, nmine;
    slot_range(z, cbeg, nmine);
    for (int k = 0; k < nmine; ++k) {
      const int st = gc % STAGES;
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
      const LDS_AS unsigned char* sk = ring + st * kStageBytes;
      const LDS_AS unsigned char* sv = sk + kKBytes;

      const i32x4 ka0 = *(const LDS_AS i32x4*)(sk + krow + grp * 256);
      const i32x4 ka1 = *(const LDS_AS i32x4*)(sk + krow + (grp + 4) * 256);
      const i32x4 kb0 = *(const LDS_AS i32x4*)(sk + krow + 64 + grp * 256);
      const i32x4 kb1 = *(const LDS_AS i32x4*)(sk + krow + 64 + (grp + 4) * 256);
      const i32x8 KA = {ka0[0], ka0[1], ka0[2], ka0[3], ka1[0], ka1[1], ka1[2], ka1[3]};
      const i32x8 KB = {kb0[0], kb0[1], kb0[2], kb0[3], kb1[0], kb1[1], kb1[2], kb1[3]};

      // value operands: head dim 16j + c16, tokens 8*grp .. 8*grp+7
      long V[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        V[j] = *(const LDS_AS long*)(sv + (grp >> 1) * 2048 + (16 * j + c16) * 16 + 8 * (grp & 1));

      // This lane's 8 tokens: tb + 8*grp + j.
      const int tok0 = tb + 8 * grp;
      const bool interior = tb >= lo_max && tb + kChunk <= hi_min;
      const bool edge = tb < lo_all || tb + kChunk > hi_all;
      if (edge) {
        // Zero value bytes of tokens no query sees (stale page tails).
        uint64_t keep = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int t = tok0 + j;
          if (t >= lo_all && t < hi_all) keep |= (uint64_t)0xff << (8 * j);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) V[j] = (long)((uint64_t)V[j] & keep);
      }

      float ksc[8], vsc[8];
      float vratio = 1.0f, vinv = 1.0f;
      if (PER_TOKEN) {
        const LDS_AS float* ss = (const LDS_AS float*)(sv + kVBytes);
        f32x4 k0 = *(const LDS_AS f32x4*)(ss + 8 * grp);
        f32x4 k1 = *(const LDS_AS f32x4*)(ss + 8 * grp + 4);
        f32x4 w0 = *(const LDS_AS f32x4*)(ss + 32 + 8 * grp);
        f32x4 w1 = *(const LDS_AS f32x4*)(ss + 32 + 8 * grp + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ksc[j] = k0[j];
          ksc[4 + j] = k1[j];
          vsc[j] = w0[j];
          vsc[4 + j] = w1[j];
        }
        if (edge) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int t = tok0 + j;
            if (!(t >= lo_all && t < hi_all)) vsc[j] = 0.0f;
          }
        }
        float cmax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) cmax = fmaxf(cmax, vsc[j]);
        cmax = max_over_groups(cmax);
        const float vnew = fmaxf(vsmax, cmax);
        vratio = vnew > 0.0f ? vsmax / vnew : 1.0f;
        vinv = vnew > 0.0f ? 1.0f / vnew : 0.0f;
        vsmax = vnew;
      }

#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const f32x4 zz = {0.f, 0.f, 0.f, 0.f};
        f32x4 la = mfma_fp8_k128(KA, qhi8[cg], zz);
        f32x4 lb = mfma_fp8_k128(KB, qhi8[cg], zz);
        la = mfma_fp8_k128(KA, qlo8[cg], la);
        lb = mfma_fp8_k128(KB, qlo8[cg], lb);
        float lg[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lg[i] = la[i] * qfac[cg];
          lg[4 + i] = lb[i] * qfac[cg];
        }
        if (PER_TOKEN) {
#pragma unroll
          for (int j = 0; j < 8; ++j) lg[j] *= ksc[j];
        }
        if (!interior) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int t = tok0 + j;
            lg[j] = (t >= vis_lo[cg] && t < vis_hi[cg]) ? lg[j] : kNegInf;
          }
        }
        float cmax = fmaxf(fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3])), fmaxf(fmaxf(lg[4], lg[5]), fmaxf(lg[6], lg[7])));
        cmax = max_over_groups(cmax);
        const float mnew = fmaxf(m2[cg], cmax);
        const float muse = mnew == kNegInf ? 0.0f : mnew;
        const float alpha = __builtin_amdgcn_exp2f(m2[cg] - muse);
        m2[cg] = mnew;
        float pr[8];
        float psum = 0.0f;
        const float bias = 8.0f - muse;  // 256 * exp(l - m)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pr[j] = __builtin_amdgcn_exp2f(lg[j] + bias);
          psum += pr[j];
        }
        lsum[cg] = lsum[cg] * alpha + psum;
        if (PER_TOKEN) {
#pragma unroll
          for (int j = 0; j < 8; ++j) pr[j] *= vsc[j] * vinv;
        }
        long phi, plo;
        split8_fp8(pr, phi, plo);
        const float f = alpha * vratio;
        if (__ballot(f != 1.0f)) {
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[cg][j] *= f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          acc[cg][j] = mfma_fp8(V[j], phi, acc[cg][j]);
          acc[cg][j] = mfma_fp8(V[j], plo, acc[cg][j]);
        }
      }
    }
    if (MULTI) {
      // Slot z is complete (this wave owns it alone): write its partial and
      // fold it into the wave's running combination.
      const float vfin = PER_TOKEN ? vsmax : v_tensor_scale;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const float L = sum_over_groups(lsum[cg]);
        const float m = m2[cg];
        const int e = cg * 16 + c16;
        if (want_partials && e < eq) {
          const float sc = L > 0.0f ? vfin / L : 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) store_partial4(a, b, h, z, e, 16 * j + 4 * grp, acc[cg][j] * sc);
          if (grp == 0) store_stats(a, b, h, z, e, L * (1.0f / 256.0f), m * kLn2);
        }
        const float Mn = fmaxf(mC[cg], m);
        const float Mu = Mn == kNegInf ? 0.0f : Mn;
        const float fc = __builtin_amdgcn_exp2f(mC[cg] - Mu);
        const float fs = __builtin_amdgcn_exp2f(m - Mu);
        const float fsv = fs * vfin;
#pragma unroll
        for (int j = 0; j < 8; ++j) accC[cg][j] = accC[cg][j] * fc + acc[cg][j] * fsv;
        lC[cg] = lC[cg] * fc + L * fs;
        mC[cg] = Mn;
        m2[cg] = kNegInf;
        lsum[cg] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[cg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      vsmax = 0.0f;
    }
  }

  // ---------------- workgroup merge ----------------
  // Each wave publishes (max, sum, value-unit accumulator) per column; sets
  // of waves are then combined by log-sum-exp: each group of `wslot` waves
  // into its slot's partial (unless MULTI waves already wrote them), and,
  // for a workgroup that covers every slot, all waves into the output.
  const float vfin_end = PER_TOKEN ? vsmax : v_tensor_scale;
  float* mbuf = (float*)smem;             // [wave][16]
  float* lbuf = mbuf + kWaves * 16;       // [wave][16]
  float* abuf = lbuf + kWaves * 16;       // [wave][head dim][16]
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
      Mst = m2[cg];
      Lst = sum_over_groups(lsum[cg]);
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
        abuf[(wave * kHead + 16 * j + 4 * grp + i) * 16 + c16] = (MULTI ? accC[cg][j][i] : acc[cg][j][i]) * sc;
    __syncthreads();
    for (int idx = tid; idx < nsets * 256; idx += kThreads) {
      const int set = idx >> 8;
      const int col = (idx >> 4) & 15;
      const int d0 = (idx & 15) * 8;
      const int e = cg * 16 + col;
      if (e >= eq) continue;
      const int w0 = set < ngp ? set * wslot : 0;
      const int w1 = set < ngp ? w0 + wslot : kWaves;
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

template <int NCG, bool PT, bool BS16, bool MULTI>
hipError_t launch_partition(const pa_fp8_partition_args& a, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((pa_fp8_partition_kernel<NCG, PT, BS16, kStages, MULTI>), dim3(grid), dim3(kThreads), 0, s, a,
                     a.block_tables, a.kv_indptr, a.context_lengths, a.key_scale, a.value_scale);
  return hipGetLastError();
}

template <int NCG, bool MULTI>
hipError_t dispatch_ncg(const pa_fp8_partition_args& a, unsigned grid, hipStream_t s) {
  const bool pt = a.per_token_kv != 0;
  const bool bs16 = a.block_size == 16;
  if (pt)
    return bs16 ? launch_partition<NCG, true, true, MULTI>(a, grid, s)
                : launch_partition<NCG, true, false, MULTI>(a, grid, s);
  return bs16 ? launch_partition<NCG, false, true, MULTI>(a, grid, s)
              : launch_partition<NCG, false, false, MULTI>(a, grid, s);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

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
  if (a->head_size != kHead) return PA_ERR_HEAD_SIZE;
  const int bs = a->block_size;
  if (!(bs == 16 || (bs >= 32 && bs <= 1024 && (bs & (bs - 1)) == 0))) return PA_ERR_BLOCK_SIZE;
  if (a->num_seqs < 0 || a->num_kv_heads <= 0 || a->num_partitions <= 0 || a->query_length <= 0 ||
      a->query_group_size <= 0 || a->num_blocks <= 0 || a->max_blocks_per_seq <= 0 || a->sliding_window < 0)
    return PA_ERR_SHAPE;
  const int eq = a->query_length * a->query_group_size;
  if (eq > 64) return PA_ERR_GROUP;
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
  const int64_t grid = (int64_t)a->num_seqs * a->num_kv_heads * pa_cdiv(a->num_partitions, spw);
  if (grid == 0) return PA_OK;
  if (grid > 0x7fffffffLL) return PA_ERR_SHAPE;
  // A wave owns several slots only when a workgroup covers more slots than
  // it has waves; that form keeps a second accumulator set, built for one
  // 16-column group only.
  const bool multi = pa_min(spw, a->num_partitions) > kWaves;
  const int ncg = (eq + 15) / 16;
  if (multi && ncg > 1) return PA_ERR_GROUP;
  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
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
  if (a->head_size != kHead) return PA_ERR_HEAD_SIZE;
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
  hipLaunchKernelGGL(pa_fp8_lse_reduce_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, *a);
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? PA_OK : (int)err;
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
    case PA_ERR_HEAD_SIZE: return "unsupported head_size (only 128)";
    case PA_ERR_BLOCK_SIZE: return "unsupported block_size (16 or a power of two in [32, 1024])";
    case PA_ERR_GROUP: return "query_length * query_group_size must be in [1, 64]";
    case PA_ERR_DTYPE: return "unsupported dtype";
    case PA_ERR_SHAPE: return "invalid dimension";
    case PA_ERR_ALIGN: return "pointer or stride not 16-byte aligned";
    case PA_ERR_ABI: return "abi_version mismatch";
    default: return hipGetErrorString((hipError_t)code);
  }
}

}  // extern "C"
