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

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kHead = 128;
constexpr int kChunk = 32;                  // tokens per wave step
constexpr int kKBytes = kChunk * kHead;     // fp8 keys of one chunk
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

__device__ __forceinline__ void lds_dma16(const void* gsrc, LDS_AS void* ldst) {
  __builtin_amdgcn_global_load_lds(gsrc, ldst, 16, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= n only:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt and lgkmcnt at
// their maxima (7 and 15) so they are not waited on.
constexpr int vmcnt_only(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

// Write one slot's outputs for query column e (8 head dims per thread call).
__device__ __forceinline__ void store_partial8(const pa_fp8_partition_args& a, bool fused, int b, int h, int slot,
                                               int e, int d0, const float* v) {
  if (fused) {
    const int gqa = a.query_group_size;
    const int qi = e / gqa, g = e - qi * gqa;
    const int64_t off = (int64_t)(b * a.query_length + qi) * a.stride_out_tok +
                        (int64_t)(h * gqa + g) * a.stride_out_head + d0;
    if (a.output_dtype == PA_DTYPE_F32) {
      f32x4* p = (f32x4*)((float*)a.output + off);
      p[0] = f32x4{v[0], v[1], v[2], v[3]};
      p[1] = f32x4{v[4], v[5], v[6], v[7]};
    } else {
      const bool bf = a.output_dtype == PA_DTYPE_BF16;
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t lo16 = bf ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
        uint32_t hi16 = bf ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
        w[i] = lo16 | (hi16 << 16);
      }
      *(i32x4*)((uint16_t*)a.output + off) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
    return;
  }
  const int64_t off = (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head +
                      (int64_t)slot * a.stride_to_part + (int64_t)e * a.stride_to_group + d0;
  if (a.tmp_dtype == PA_DTYPE_F32) {
    f32x4* p = (f32x4*)((float*)a.tmp_out + off);
    p[0] = f32x4{v[0], v[1], v[2], v[3]};
    p[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_bf16_bits(v[2 * i]) | (f32_to_bf16_bits(v[2 * i + 1]) << 16);
    *(i32x4*)((uint16_t*)a.tmp_out + off) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

__device__ __forceinline__ void store_stats(const pa_fp8_partition_args& a, int b, int h, int slot, int e,
                                            float exp_sum, float max_logit) {
  const int64_t off = (int64_t)b * a.stride_es_seq + (int64_t)h * a.stride_es_head +
                      (int64_t)slot * a.stride_es_part + e;
  a.exp_sums[off] = exp_sum;
  a.max_logits[off] = max_logit;
}

// Block table, context lengths and scales come in as separate restrict
// pointers so that their wave-uniform loads become scalar (SMEM) loads:
// page lookups then count on lgkmcnt and never force a wait on the vmcnt
// of the direct-to-LDS data loads in flight.
template <int NCG, bool PER_TOKEN, bool BS16, int STAGES>
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
  int bid = blockIdx.x;
  const int slot = bid % P;
  bid /= P;
  const int h = bid % a.num_kv_heads;
  const int b = bid / a.num_kv_heads;

  const int ql = a.query_length;
  const int gqa = a.query_group_size;
  const int eq = ql * gqa;
  const int W = a.sliding_window;
  const int ctx = context_lengths[b];
  const bool fused = a.output != nullptr;

  int t0, t1, lo_all, hi_all, unused;
  pa_plan_slot_tokens(ctx, P, slot, W, ql, &t0, &t1);
  pa_plan_visible(ctx, 0, ql, W, &lo_all, &unused);
  pa_plan_visible(ctx, ql - 1, ql, W, &unused, &hi_all);
  const int a0 = pa_max(t0, lo_all);
  const int a1 = pa_min(t1, hi_all);

  // A sequence without pages in its block-table row reads nothing.
  const int bs_rows = kv_indptr ? kv_indptr[b + 1] - kv_indptr[b] : a.max_blocks_per_seq;
  if (a1 <= a0 || bs_rows <= 0) {
    // Empty slot: zero partial, zero sum, -inf max (reference empty-slot
    // semantics, kernels/pa_decode_swa.py:1493-1504).
    const float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int idx = tid; idx < eq * (kHead / 8); idx += kThreads) {
      const int e = idx / (kHead / 8);
      store_partial8(a, fused, b, h, slot, e, (idx % (kHead / 8)) * 8, z);
    }
    if (!fused)
      for (int e = tid; e < eq; e += kThreads) store_stats(a, b, h, slot, e, 0.0f, kNegInf);
    return;
  }

  // ---------------- query: load, scale, split into fp8 hi + lo ----------------
  long qhi[NCG][4], qlo[NCG][4];
  float qfac[NCG];   // base-2 logit factor per column
  int vis_lo[NCG], vis_hi[NCG];
  const float k_tensor_scale = PER_TOKEN ? 1.0f : key_scale[0];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    const int e = cg * 16 + c16;
    const bool valid = e < eq;
    float v[32];
    int qi = 0;
    if (valid) {
      qi = e / gqa;
      const int g = e - qi * gqa;
      const uint16_t* qp = (const uint16_t*)a.query + (int64_t)(b * ql + qi) * a.stride_q_tok +
                           (int64_t)(h * gqa + g) * a.stride_q_head;
      i32x4 x[4];
      x[0] = *(const i32x4*)(qp + 16 * grp);
      x[1] = *(const i32x4*)(qp + 16 * grp + 8);
      x[2] = *(const i32x4*)(qp + 16 * (grp + 4));
      x[3] = *(const i32x4*)(qp + 16 * (grp + 4) + 8);
      if (a.query_dtype == PA_DTYPE_F16) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t w = (uint32_t)x[i >> 2][i & 3];
          v[2 * i] = f16_bits_to_f32(w & 0xffffu);
          v[2 * i + 1] = f16_bits_to_f32(w >> 16);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t w = (uint32_t)x[i >> 2][i & 3];
          v[2 * i] = bf16_bits_to_f32(w & 0xffffu);
          v[2 * i + 1] = bf16_bits_to_f32(w >> 16);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) v[i] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, shfl_xor(amax, 16));
    amax = fmaxf(amax, shfl_xor(amax, 32));
    // Power-of-two scale putting amax into [128, 256): exact in fp32.
    int sexp = 261 - (int)((__float_as_uint(amax) >> 23) & 0xffu);
    sexp = sexp < 1 ? 1 : (sexp > 254 ? 254 : sexp);
    const float sq = amax > 0.0f ? __uint_as_float((uint32_t)sexp << 23) : 1.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float xs[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xs[i] = v[8 * s + i] * sq;
      split8_fp8(xs, qhi[cg][s], qlo[cg][s]);
    }
    qfac[cg] = a.softmax_scale * kLog2e * k_tensor_scale / sq;
    int lo = 0, hi = 0;
    if (valid) pa_plan_visible(ctx, qi, ql, W, &lo, &hi);
    vis_lo[cg] = lo;
    vis_hi[cg] = hi;
  }

  // ---------------- stream this wave's chunks ----------------
  const int cbeg = a0 & ~(kChunk - 1);
  const int nchunks = pa_cdiv(a1 - cbeg, kChunk);
  const int nmine = nchunks > wave ? (nchunks - wave + kWaves - 1) / kWaves : 0;

  const int bs = a.block_size;
  const int bs_shift = BS16 ? 4 : __builtin_ctz((unsigned)bs);
  const int64_t row_off = kv_indptr ? (int64_t)kv_indptr[b] : (int64_t)b * a.stride_bt_seq;
  const int row_len = kv_indptr ? kv_indptr[b + 1] - kv_indptr[b] : a.max_blocks_per_seq;
  const int32_t* bt_row = block_tables + row_off;
  const int last_page = pa_min(pa_cdiv(ctx, bs) - 1, row_len - 1);
  const int nblocks = a.num_blocks;
  // Block-table entries of the (one or two) pages of chunk k.  Reads past
  // the context reuse the last page (its tokens are masked).  The raw
  // entries are clamped into the cache only when used, one step later, so
  // the scalar loads overlap the current chunk's compute.
  auto fetch_pages = [&](int k, int& q0, int& q1) {
    const int lp0 = (cbeg + (wave + k * kWaves) * kChunk) >> bs_shift;
    q0 = bt_row[pa_min(lp0, last_page)];
    q1 = BS16 ? bt_row[pa_min(lp0 + 1, last_page)] : q0;
  };
  auto clamp_page = [&](int p) -> int {
    p = p < 0 ? 0 : p;
    return p < nblocks ? p : nblocks - 1;
  };

  const uint8_t* kbase = (const uint8_t*)a.key_cache + (int64_t)h * a.stride_k_head;
  const uint8_t* vbase = (const uint8_t*)a.value_cache + (int64_t)h * a.stride_v_head;
  const float* ksbase = PER_TOKEN ? key_scale + (int64_t)h * a.stride_ks_head : nullptr;
  const float* vsbase = PER_TOKEN ? value_scale + (int64_t)h * a.stride_ks_head : nullptr;

  LDS_AS unsigned char* ring = (LDS_AS unsigned char*)smem + wave * kWaveBytes;

  // Token order inside a chunk's LDS key image: slot r (0..15) of half t
  // holds chunk token 8*(r/4) + 4*t + r%4, so 16-row tile t of the QK
  // product reads slots 16t .. 16t+15 contiguously.
  const int kslot = lane & 31;
  const int ktok = 8 * ((kslot & 15) >> 2) + 4 * (kslot >> 4) + (kslot & 3);

  auto issue = [&](int k, int st, int raw0, int raw1) {
    const int p0 = clamp_page(raw0);
    const int p1 = BS16 ? clamp_page(raw1) : p0;
    const int tb = cbeg + (wave + k * kWaves) * kChunk;
    LDS_AS unsigned char* sk = ring + st * kStageBytes;
    LDS_AS unsigned char* sv = sk + kKBytes;
    const int s0 = BS16 ? 0 : (tb & (bs - 1));
    // keys: 4 x 1 KiB; lane -> (16-dim chunk c, token)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int c = 2 * ii + (lane >> 5);
      const uint8_t* src;
      if (BS16) {
        const int pg = ktok >= 16 ? p1 : p0;
        src = kbase + (int64_t)pg * a.stride_k_block + c * 256 + (ktok & 15) * 16;
      } else {
        src = kbase + (int64_t)p0 * a.stride_k_block + c * (bs * 16) + (s0 + ktok) * 16;
      }
      lds_dma16(src, sk + ii * 1024);
    }
    // values: 4 x 1 KiB; LDS image [16-token group][head dim][16 tokens]
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int off = ii * 1024 + lane * 16;
      const int tg = off >> 11;
      const int hd = (off >> 4) & (kHead - 1);
      const uint8_t* src;
      if (BS16) {
        src = vbase + (int64_t)(tg ? p1 : p0) * a.stride_v_block + hd * 16;
      } else {
        const int s = s0 + 16 * tg;
        src = a.trans_v ? vbase + (int64_t)p0 * a.stride_v_block + (s >> 4) * (kHead * 16) + hd * 16
                        : vbase + (int64_t)p0 * a.stride_v_block + hd * bs + s;
      }
      lds_dma16(src, sv + ii * 1024);
    }
    if (PER_TOKEN) {
      LDS_AS unsigned char* ss = sv + kVBytes;
      if (lane < 16) {
        const int tt = (lane & 7) * 4;
        const int pg = BS16 ? (tt >= 16 ? p1 : p0) : p0;
        const int s = BS16 ? (tt & 15) : s0 + tt;
        const float* base = lane < 8 ? ksbase : vsbase;
        lds_dma16(base + (int64_t)pg * a.stride_ks_block + s, ss);
      }
    }
  };

  float m2[NCG], lsum[NCG];
  f32x4 acc[NCG][8];
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    m2[cg] = kNegInf;
    lsum[cg] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[cg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float vsmax = 0.0f;  // running max of per-token value scales (per wave)

  // Pipeline: chunks k+1 .. k+STAGES-1 are in flight while chunk k is
  // computed; the page indices of the next chunk to issue are fetched one
  // step ahead so their scalar-load latency is hidden as well.
  int np0 = 0, np1 = 0;
#pragma unroll
  for (int k = 0; k < STAGES - 1; ++k)
    if (k < nmine) {
      fetch_pages(k, np0, np1);
      issue(k, k, np0, np1);
    }
  if (STAGES - 1 < nmine) fetch_pages(STAGES - 1, np0, np1);

  for (int k = 0; k < nmine; ++k) {
    const int st = k % STAGES;
    if (k + STAGES - 1 < nmine) {
      issue(k + STAGES - 1, (k + STAGES - 1) % STAGES, np0, np1);
      if (k + STAGES < nmine) fetch_pages(k + STAGES, np0, np1);
      // Loads retire in order: leave the newest chunks' loads in flight.
      constexpr int kLoadsPerChunk = 8 + (PER_TOKEN ? 1 : 0);
      __builtin_amdgcn_s_waitcnt(vmcnt_only(kLoadsPerChunk * (STAGES - 1)));
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    const int tb = cbeg + (wave + k * kWaves) * kChunk;
    const LDS_AS unsigned char* sk = ring + st * kStageBytes;
    const LDS_AS unsigned char* sv = sk + kKBytes;

    // key operands: tile 0 rows = slots 0..15, tile 1 rows = slots 16..31
    i32x4 ka0 = *(const LDS_AS i32x4*)(sk + grp * 512 + c16 * 16);
    i32x4 ka1 = *(const LDS_AS i32x4*)(sk + (grp + 4) * 512 + c16 * 16);
    i32x4 kb0 = *(const LDS_AS i32x4*)(sk + grp * 512 + (16 + c16) * 16);
    i32x4 kb1 = *(const LDS_AS i32x4*)(sk + (grp + 4) * 512 + (16 + c16) * 16);
    long KA[4], KB[4];
    KA[0] = (long)((uint64_t)(uint32_t)ka0[0] | ((uint64_t)(uint32_t)ka0[1] << 32));
    KA[1] = (long)((uint64_t)(uint32_t)ka0[2] | ((uint64_t)(uint32_t)ka0[3] << 32));
    KA[2] = (long)((uint64_t)(uint32_t)ka1[0] | ((uint64_t)(uint32_t)ka1[1] << 32));
    KA[3] = (long)((uint64_t)(uint32_t)ka1[2] | ((uint64_t)(uint32_t)ka1[3] << 32));
    KB[0] = (long)((uint64_t)(uint32_t)kb0[0] | ((uint64_t)(uint32_t)kb0[1] << 32));
    KB[1] = (long)((uint64_t)(uint32_t)kb0[2] | ((uint64_t)(uint32_t)kb0[3] << 32));
    KB[2] = (long)((uint64_t)(uint32_t)kb1[0] | ((uint64_t)(uint32_t)kb1[1] << 32));
    KB[3] = (long)((uint64_t)(uint32_t)kb1[2] | ((uint64_t)(uint32_t)kb1[3] << 32));

    // value operands: head dim 16j + c16, tokens 8*grp .. 8*grp+7
    long V[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      V[j] = *(const LDS_AS long*)(sv + (grp >> 1) * 2048 + (16 * j + c16) * 16 + 8 * (grp & 1));

    // This lane's 8 tokens: tb + 8*grp + j.
    const int tok0 = tb + 8 * grp;
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
      float cmax = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ksc[j] = k0[j];
        ksc[4 + j] = k1[j];
        vsc[j] = w0[j];
        vsc[4 + j] = w1[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = tok0 + j;
        if (!(t >= lo_all && t < hi_all)) vsc[j] = 0.0f;
        cmax = fmaxf(cmax, vsc[j]);
      }
      cmax = fmaxf(cmax, shfl_xor(cmax, 16));
      cmax = fmaxf(cmax, shfl_xor(cmax, 32));
      const float vnew = fmaxf(vsmax, cmax);
      vratio = vnew > 0.0f ? vsmax / vnew : 1.0f;
      vinv = vnew > 0.0f ? 1.0f / vnew : 0.0f;
      vsmax = vnew;
    }

#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      f32x4 la = {0.f, 0.f, 0.f, 0.f}, lb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        la = mfma_fp8(KA[s], qhi[cg][s], la);
        lb = mfma_fp8(KB[s], qhi[cg][s], lb);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        la = mfma_fp8(KA[s], qlo[cg][s], la);
        lb = mfma_fp8(KB[s], qlo[cg][s], lb);
      }
      float l[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        l[i] = la[i] * qfac[cg];
        l[4 + i] = lb[i] * qfac[cg];
      }
      float cmax = kNegInf;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (PER_TOKEN) l[j] *= ksc[j];
        const int t = tok0 + j;
        l[j] = (t >= vis_lo[cg] && t < vis_hi[cg]) ? l[j] : kNegInf;
        cmax = fmaxf(cmax, l[j]);
      }
      cmax = fmaxf(cmax, shfl_xor(cmax, 16));
      cmax = fmaxf(cmax, shfl_xor(cmax, 32));
      const float mnew = fmaxf(m2[cg], cmax);
      const float muse = mnew == kNegInf ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(m2[cg] - muse);
      m2[cg] = mnew;
      float p[8];
      float psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = __builtin_amdgcn_exp2f(l[j] - muse + 8.0f);  // 256 * exp(l - m)
        psum += p[j];
      }
      lsum[cg] = lsum[cg] * alpha + psum;
      if (PER_TOKEN) {
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] *= vsc[j] * vinv;
      }
      long phi, plo;
      split8_fp8(p, phi, plo);
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

  // ---------------- merge the four waves ----------------
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    lsum[cg] += shfl_xor(lsum[cg], 16);
    lsum[cg] += shfl_xor(lsum[cg], 32);
  }
  const float vfin = PER_TOKEN ? vsmax : value_scale[0];
  float* mbuf = (float*)smem;             // [wave][16]
  float* lbuf = mbuf + kWaves * 16;       // [wave][16]
  float* abuf = lbuf + kWaves * 16;       // [wave][head dim][16]
#pragma unroll
  for (int cg = 0; cg < NCG; ++cg) {
    __syncthreads();
    if (grp == 0) {
      mbuf[wave * 16 + c16] = m2[cg];
      lbuf[wave * 16 + c16] = lsum[cg];
    }
    __syncthreads();
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mbuf[w * 16 + c16]);
    const float Mu = M == kNegInf ? 0.0f : M;
    const float fself = __builtin_amdgcn_exp2f(m2[cg] - Mu) * vfin;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) abuf[(wave * kHead + 16 * j + 4 * grp + i) * 16 + c16] = acc[cg][j][i] * fself;
    __syncthreads();
    const int col = tid >> 4;
    const int d0 = (tid & 15) * 8;
    const int e = cg * 16 + col;
    if (e < eq) {
      float Mc = kNegInf;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) Mc = fmaxf(Mc, mbuf[w * 16 + col]);
      const float Mcu = Mc == kNegInf ? 0.0f : Mc;
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) L += lbuf[w * 16 + col] * __builtin_amdgcn_exp2f(mbuf[w * 16 + col] - Mcu);
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += abuf[(w * kHead + d0 + i) * 16 + col];
        o[i] = s * inv;
      }
      store_partial8(a, fused, b, h, slot, e, d0, o);
      if (!fused && (tid & 15) == 0) store_stats(a, b, h, slot, e, L * (1.0f / 256.0f), Mc * kLn2);
    }
  }
}

// One wave per (sequence, kv head, column); lane covers head dims 2l, 2l+1.
__global__ __launch_bounds__(256) void pa_fp8_lse_reduce_kernel(const pa_fp8_reduce_args a) {
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
  float M = kNegInf;
  for (int p = 0; p < P; ++p) M = fmaxf(M, a.max_logits[sbase + p * a.stride_es_part]);
  const int d = 2 * lane;
  float o0 = 0.0f, o1 = 0.0f;
  if (M != kNegInf) {
    float tot = 0.0f;
    const int64_t tbase = (int64_t)b * a.stride_to_seq + (int64_t)h * a.stride_to_head + (int64_t)e * a.stride_to_group + d;
    for (int p = 0; p < P; ++p) {
      const float mp = a.max_logits[sbase + p * a.stride_es_part];
      const float w = mp == kNegInf ? 0.0f : a.exp_sums[sbase + p * a.stride_es_part] * __expf(mp - M);
      tot += w;
      float x0, x1;
      if (a.tmp_dtype == PA_DTYPE_F32) {
        f32x2 t = *(const f32x2*)((const float*)a.tmp_out + tbase + p * a.stride_to_part);
        x0 = t[0];
        x1 = t[1];
      } else {
        const uint32_t t = *(const uint32_t*)((const uint16_t*)a.tmp_out + tbase + p * a.stride_to_part);
        x0 = bf16_bits_to_f32(t & 0xffffu);
        x1 = bf16_bits_to_f32(t >> 16);
      }
      o0 += w * x0;
      o1 += w * x1;
    }
    const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
    o0 *= inv;
    o1 *= inv;
  }
  const int gqa = a.query_group_size;
  const int qi = e / gqa, g = e - qi * gqa;
  const int64_t off = (int64_t)b * a.stride_out_seq + (int64_t)qi * a.stride_out_ql +
                      (int64_t)h * a.stride_out_kv_head + (int64_t)g * a.stride_out_group + d;
  if (a.output_dtype == PA_DTYPE_F32) {
    *(f32x2*)((float*)a.output + off) = f32x2{o0, o1};
  } else if (a.output_dtype == PA_DTYPE_F16) {
    *(uint32_t*)((uint16_t*)a.output + off) = f32_to_f16_bits(o0) | (f32_to_f16_bits(o1) << 16);
  } else {
    *(uint32_t*)((uint16_t*)a.output + off) = f32_to_bf16_bits(o0) | (f32_to_bf16_bits(o1) << 16);
  }
}

template <int NCG, bool PT, bool BS16>
hipError_t launch_partition(const pa_fp8_partition_args& a, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((pa_fp8_partition_kernel<NCG, PT, BS16, 2>), dim3(grid), dim3(kThreads), 0, s, a,
                     a.block_tables, a.kv_indptr, a.context_lengths, a.key_scale, a.value_scale);
  return hipGetLastError();
}

template <int NCG>
hipError_t dispatch_ncg(const pa_fp8_partition_args& a, unsigned grid, hipStream_t s) {
  const bool pt = a.per_token_kv != 0;
  const bool bs16 = a.block_size == 16;
  if (pt) return bs16 ? launch_partition<NCG, true, true>(a, grid, s) : launch_partition<NCG, true, false>(a, grid, s);
  return bs16 ? launch_partition<NCG, false, true>(a, grid, s) : launch_partition<NCG, false, false>(a, grid, s);
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
  const bool fused = a->output != nullptr;
  if (fused ? a->num_partitions != 1 : (!a->exp_sums || !a->max_logits || !a->tmp_out)) return PA_ERR_NULL_ARG;
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
  if (fused && a->output_dtype != PA_DTYPE_BF16 && a->output_dtype != PA_DTYPE_F16 && a->output_dtype != PA_DTYPE_F32)
    return PA_ERR_DTYPE;
  // 16-byte vector accesses: query rows, cache pages, scale rows, partials.
  if (!aligned16(a->query) || (a->stride_q_tok % 8) || (a->stride_q_head % 8)) return PA_ERR_ALIGN;
  if (!aligned16(a->key_cache) || !aligned16(a->value_cache) || (a->stride_k_block % 16) ||
      (a->stride_k_head % 16) || (a->stride_v_block % 16) || (a->stride_v_head % 16))
    return PA_ERR_ALIGN;
  if (a->per_token_kv &&
      (!aligned16(a->key_scale) || !aligned16(a->value_scale) || (a->stride_ks_block % 4) || (a->stride_ks_head % 4)))
    return PA_ERR_ALIGN;
  if (fused) {
    if (!aligned16(a->output) || (a->stride_out_tok % 8) || (a->stride_out_head % 8)) return PA_ERR_ALIGN;
  } else {
    if (!aligned16(a->tmp_out) || (a->stride_to_group % 8) || (a->stride_to_part % 8) || (a->stride_to_head % 8) ||
        (a->stride_to_seq % 8))
      return PA_ERR_ALIGN;
  }
  const int64_t grid = (int64_t)a->num_seqs * a->num_kv_heads * a->num_partitions;
  if (grid == 0) return PA_OK;
  if (grid > 0x7fffffffLL) return PA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  switch ((eq + 15) / 16) {
    case 1: err = dispatch_ncg<1>(*a, (unsigned)grid, s); break;
    case 2: err = dispatch_ncg<2>(*a, (unsigned)grid, s); break;
    case 3: err = dispatch_ncg<3>(*a, (unsigned)grid, s); break;
    default: err = dispatch_ncg<4>(*a, (unsigned)grid, s); break;
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
