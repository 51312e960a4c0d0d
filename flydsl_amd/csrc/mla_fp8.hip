// MLA (multi-head latent attention) fp8 decode for MI355X (gfx950): the
// persistent decode kernel, its log-sum-exp reduce, the host work-list
// planner and their C ABI (pa_fp8.h).
//
// Shape (kernels/mla_fwd_decode_m16x8_fp8_fp8.py:41-60): 128 query heads
// share one latent kv head; a token's key is its whole 576-byte fp8 row
// (512 latent + 64 rope dims) and its value is the first 512 bytes of the
// same row; page size 1.  Per token the decode does 128 x 1088 x 2 FLOP on
// 576 bytes, 484 FLOP/B -- just below the fp8 MFMA ridge of MI355X
// (5.0 PFLOP/s / 8 TB/s = 625 FLOP/B), so both the matrix cores and HBM
// must run near their peaks.
//
// Work decomposition.  One workgroup per worker (grid = number of workers,
// one per CU); it walks its works (work_indptr / work_info) and each work's
// kv range in 128-token blocks.  Eight waves (two per SIMD, so one wave's
// softmax runs beside the other's matrix products) split the heads (wave w:
// heads 16w .. 16w+15) and share each block through LDS: wave w DMAs tokens
// 16w .. 16w+15 of the block (gfx950 global_load_lds, 16 B per lane) into
// one of two 72 KiB stages while the block before is computed.
//
// LDS image of a stage: [4 token groups of 32][9 quads of 4 column units]
// [32 tokens][4 slots of 16 B], the slots XOR-swizzled by token.  Each DMA
// instruction fills one quad of 16 tokens, so every lane keeps one token
// (one page index) for the whole block, and both the key reads (16
// consecutive tokens of one unit) and the transposed value reads cover
// whole 256-byte runs.
//
// Arithmetic, all on v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3fn operands,
// unit scales):
//   * S^T = K Q^T per 16-token tile: A = 16 key rows x 128 dims (two 16-byte
//     LDS reads), B = Q^T of 16 heads, in registers; 4 latent blocks + 1
//     rope block (the key operand's upper 64 k-slots zero);
//   * the result lane (c, g) = (l % 16, l / 16) holds tokens 4g .. 4g+3 of
//     the tile for head c, which is exactly the B-operand slot order the
//     value product needs: dword T of P^T = the four probabilities of tile T;
//   * O^T = V^T P^T per 32 value dims: ds_read_b64_tr_b8 (gfx950 LDS
//     transpose read) gives lane (c, g) four tokens 16T+4g .. 16T+4g+3 of
//     value dims d0+c (low dword) and d0+16+c (high dword), i.e. the A
//     operands of two 16-dim row tiles with the same token order as P^T.
// The O^T accumulators are 16 heads x 512 dims per wave (128 AGPRs, the
// AGPR half of a wave's 256 registers at two waves per SIMD).
// Softmax is base 2 against a per-head reference exponent m0, set on a
// work's first block to the head's maximum + 40; the accumulators and the
// denominator stay in units of 2^m0.  Each half block's probabilities are
// p = 2^(x - e) <= 1 with e = ceil(max of the lane pair) and enter the value
// product with the e8m0 block scale 2^(e - m0), clamped to 2^-127 .. 2^127
// (logits more than 127 below m0 count as 2^-127 of m0, i.e. nothing).  A
// half block whose head maximum lies more than 64 above m0 (rare: it needs
// logits that grow by over 44 nats inside one work) first moves m0 to its
// maximum + 40 and multiplies the head's 128 accumulators and its sum by
// 2^(old - new), so e - m0 never exceeds 65 and nothing overflows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "mla_plan.h"
#include "pa_fp8.h"
#include "pa_check.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

#define LDS_AS __attribute__((address_space(3)))

constexpr int kHeads = 128;
constexpr int kQkDim = 576;
constexpr int kVDim = 512;
constexpr int kBlock = MLA_PLAN_BLOCK;       // tokens per LDS stage
constexpr int kQuadBytes = 32 * 64;         // four column units of a 32-token group
constexpr int kGroupBytes = 32 * kQkDim;     // one wave's 32 tokens
constexpr int kStageBytes = kBlock * kQkDim; // 73728
// Waves of a workgroup with NHT 16-head tiles per wave: 4 waves of 32 heads
// (one wave per SIMD, 256 accumulator registers each) or 8 waves of 16 heads
// (two waves per SIMD, 128 accumulator registers each).
template <int NHT>
struct Shape {
  static_assert(NHT == 1 || NHT == 2, "one or two head tiles per wave");
  static constexpr int waves = 8 / NHT;
  static constexpr int threads = 64 * waves;
  static constexpr int dma = kQkDim / 32 * NHT / 2;  // 1 KiB DMA instructions per wave and block
};
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kNegInf = -__builtin_inff();
// A head's block maximum this far (base 2) above its reference exponent m0
// moves m0 (the e8m0 block scales reach 2^127; accumulators and sums stay
// far from float overflow).
constexpr float kRescaleMargin = 64.f;
// Head tiles per wave of the build: 1 (eight waves of 16 heads, the
// default) or 2 (four waves of 32 heads; measured about 13% slower on
// B 128 x 8192, kept as a build option for comparison).
#ifndef MLA_HEAD_TILES
#define MLA_HEAD_TILES 1
#endif

static_assert(kGroupBytes * 4 == kStageBytes, "four 32-token groups per stage");
static_assert(kQuadBytes * (kQkDim / 64) == kGroupBytes, "9 quads per group");

// Value product into accumulators pinned to AGPRs, with e8m0 block scales
// (sa for the values: unit, sb for the probabilities of the lane's head and
// 32-token group).  The 256 accumulator registers of a wave fill the AGPR
// half of the register file; queries, logits and operands stay in VGPRs,
// which the compiler's own register-class choice for MFMA results does not
// achieve here.  The accumulate chain (same destination, same opcode back
// to back) is dependency-checked by the hardware; the only VALU reads of
// the accumulators (the epilogue) follow agpr_settle().
template <bool FIRST>
__device__ __forceinline__ void pv_mfma(f32x4& acc, const i32x8& a, const i32x8& b, int sa, int sb) {
  if (FIRST)
    asm volatile("s_nop 1\n\tv_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, 0, %3, %4" : "=&a"(acc) : "v"(a), "v"(b), "v"(sa), "v"(sb));
  else
    asm volatile("s_nop 1\n\tv_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4" : "+a"(acc) : "v"(a), "v"(b), "v"(sa), "v"(sb));
}
// Key product into logits in VGPRs (first: srcC = 0).  Compiler builtins,
// so the scheduler knows the MFMA latency and reads the next key operands
// from LDS while the products run, and the hazard recognizer covers the
// operand and result hazards.
template <bool FIRST>
__device__ __forceinline__ void qk_mfma(f32x4& acc, const i32x8& a, const i32x8& b) {
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, FIRST ? f32x4{0.f, 0.f, 0.f, 0.f} : acc, 0, 0, 0, 0,
                                                         0, 0);
}
// The compiler does not know that the inline-asm MFMAs of the value product
// are MFMAs, so the hazards it would cover are covered here (s_nop n waits
// n + 1 states):
//   * VALU write of an operand -> MFMA read: 2 wait states, the s_nop 1 in
//     front of every value-product MFMA;
//   * MFMA result -> first VALU read: agpr_settle() waits 24 states before
//     the accumulator reads.
// Orders the probability packing before the value product.
template <bool PRECISE>
__device__ __forceinline__ void probs_ready(i32x8 (&phi)[2], i32x8 (&plo)[2]) {
  if (PRECISE)
    asm volatile("" : "+v"(phi[0]), "+v"(phi[1]), "+v"(plo[0]), "+v"(plo[1]));
  else
    asm volatile("" : "+v"(phi[0]), "+v"(phi[1]));
}
template <bool PRECISE>
__device__ __forceinline__ void probs_ready(i32x8 (&phi)[1], i32x8 (&plo)[1]) {
  if (PRECISE)
    asm volatile("" : "+v"(phi[0]), "+v"(plo[0]));
  else
    asm volatile("" : "+v"(phi[0]));
}
// Accumulator tile -> VGPRs through explicit v_accvgpr_read (opaque to the
// compiler, so the epilogue's scaling cannot be hoisted ahead of its
// stores and keep every tile live at once).
__device__ __forceinline__ f32x4 read_acc(const f32x4& acc) {
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(r[i]) : "a"(acc[i]));
  return r;
}
__device__ __forceinline__ void agpr_settle() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// Rare path of the softmax: head tile ht's accumulators times f (a power of
// two, exact).  The scaled tiles go back to AGPRs; the asm statements that
// take them as in/out operands keep every write ahead of the next value
// product, whose MFMAs wait their own two states.
template <int NHT>
__device__ __forceinline__ void rescale_acc(f32x4 (&o)[16][2][NHT], int ht, float f) {
  agpr_settle();
#pragma unroll
  for (int db = 0; db < 16; ++db)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) o[db][rt][ht] = read_acc(o[db][rt][ht]) * f;
#pragma unroll
  for (int db = 0; db < 16; db += 4)
    asm volatile("s_nop 1"
                 : "+a"(o[db][0][ht]), "+a"(o[db][1][ht]), "+a"(o[db + 1][0][ht]), "+a"(o[db + 1][1][ht]),
                   "+a"(o[db + 2][0][ht]), "+a"(o[db + 2][1][ht]), "+a"(o[db + 3][0][ht]), "+a"(o[db + 3][1][ht]));
}

// 16 bytes per lane from global memory straight into LDS (M0 = the wave's
// LDS destination, lane l writing 16 l bytes past it), non-temporal: with
// the default cache policy the kernel fetches about 1.5x the bytes from
// HBM (measured with FETCH_SIZE), at no gain in time.
// Inline assembly rather than __builtin_amdgcn_global_load_lds: while the
// builtin's DMA is in flight, the compiler's wait insertion takes every LDS
// read to be unordered behind it and waits for each with lgkmcnt(0), which
// serialises the pipelined key reads.  The DMA is awaited explicitly
// (vmcnt(0) and a barrier before its stage is read).  The compiler sets M0
// (an input operand); an LDS DMA must not read M0 in the cycle after an
// SALU wrote it (the wait state hipcc puts between its own M0 write and
// such a load), which the compiler cannot see inside the statement, hence
// the s_nop.
__device__ __forceinline__ void lds_dma16(const void* gsrc, LDS_AS void* ldst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
               :
               : "v"(gsrc), "{m0}"((unsigned)(uintptr_t)ldst)
               : "memory");
}

constexpr int vmcnt_only(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Reductions over lanes c, c+16, c+32, c+48 (one head across the four
// 16-lane groups), VALU permlane swaps.
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

// Max over lanes l and l ^ 16 (lane groups {0,1} and {2,3}).
__device__ __forceinline__ float max_over_pair(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Value of lane l ^ 32.
__device__ __forceinline__ int other_half_wave(int v) { return __shfl_xor(v, 32, 64); }

// One work record, clamped into range; all fields wave-uniform.
struct Work {
  int qo;       // query row
  int pql;      // partial row, or -1: final output
  int kv0, kv1; // positions in kv_page_indices
  int nblk;     // 128-token blocks (1 for an empty range)
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, i>) for i = 0 .. N-1, each i a compile-time constant.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Lane index, recomputed where it is needed (volatile, so it is not hoisted
// into a register that lives through the whole loop and gets spilled).
__device__ __forceinline__ int lane_id() {
  int r;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(r));
  return r;
}

// Zero the compiler cannot see through (keeps two loads of one address
// apart).
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

__device__ __forceinline__ Work load_work(const pa_mla_decode_args& a, int wi) {
  const int32_t* w = a.work_info + 8 * (int64_t)wi;
  Work r;
  r.pql = uni(w[1]);
  r.qo = uni(w[2]);
  r.kv0 = uni(w[4]);
  r.kv1 = uni(w[5]);
  r.qo = min(max(r.qo, 0), a.num_rows - 1);
  if (r.pql >= a.num_partial) r.pql = a.num_partial - 1;
  if (r.pql < 0) r.pql = -1;
  r.kv0 = min(max(r.kv0, 0), a.num_page_indices);
  r.kv1 = min(max(r.kv1, r.kv0), a.num_page_indices);
  const int len = r.kv1 - r.kv0;
  r.nblk = len > 0 ? (len + kBlock - 1) / kBlock : 1;
  return r;
}

// Walks the (work, block) units of one worker.
struct Cursor {
  int wi, blk;
  Work w;
};

__device__ __forceinline__ bool valid(const Cursor& c, int we) { return c.wi < we; }

__device__ __forceinline__ void advance(const pa_mla_decode_args& a, Cursor& c, int we) {
  if (c.wi >= we) return;
  if (++c.blk < c.w.nblk) return;
  c.blk = 0;
  if (++c.wi < we) c.w = load_work(a, c.wi);
}

// Pages of the tokens this lane DMAs for unit c.  Four waves: wave w DMAs
// the 32-token group w, the lane tokens l / 4 and 16 + l / 4 of it.  Eight
// waves: wave w DMAs half w % 2 of group w / 2, the lane token
// 16 (w % 2) + l / 4 (returned twice).
template <int NHT>
__device__ __forceinline__ i32x2 unit_pages(const pa_mla_decode_args& a, const Cursor& c, int w) {
  if (c.w.kv1 <= c.w.kv0) return i32x2{0, 0};
  const int last = c.w.kv1 - 1;
  if constexpr (NHT == 2) {
    const int pos = c.w.kv0 + c.blk * kBlock + 32 * w + (lane_id() >> 2);
    return i32x2{a.kv_page_indices[min(pos, last)], a.kv_page_indices[min(pos + 16, last)]};
  } else {
    const int pos = c.w.kv0 + c.blk * kBlock + 16 * w + (lane_id() >> 2);
    const int p = a.kv_page_indices[min(pos, last)];
    return i32x2{p, p};
  }
}

// DMA of one wave's share of a block into a stage.  Group layout:
// [9 quads of 4 column units][32 tokens][4 slots of 16 B]; slot s of token t
// holds unit 4q + (s ^ swz(t)), swz(t) = (t >> 4 & 1) | (t >> 2 & 1) << 1:
// an XOR swizzle under which both the key reads (ds_read_b128, 16 rows of
// one unit) and the value transpose reads (ds_read_b64_tr_b8) run at the
// full LDS rate on gfx950 (measured against every XOR swizzle of the token
// bits; the lane grouping of a 16-byte read is not that of 16 consecutive
// lanes, and simpler swizzles cost a 2-way bank conflict).  Instruction n of a
// group fills quad n / 2 for tokens 16 (n % 2) .. +15: each lane reads 16 B
// and four lanes read 64 consecutive bytes of one row.  Four waves: wave w
// issues the 18 instructions of group w; eight waves: wave w issues the 9
// instructions n = 2k + w % 2 of group w / 2.
template <int NHT>
__device__ __forceinline__ void issue_block(const pa_mla_decode_args& a, LDS_AS unsigned char* stage, int w,
                                           i32x2 pages) {
  const int np = (int)(a.num_pages - 1);
  const int l = lane_id();
  const int sx0 = (l & 3) ^ (((l >> 4) & 1) << 1);  // tokens l / 4:      swz = 2 (l / 16 % 2)
  const unsigned char* kvb = (const unsigned char*)a.kv_buffer;
  if constexpr (NHT == 2) {
    const int sx1 = sx0 ^ 1;  // tokens 16 + l / 4: swz ^ 1
    const unsigned char* src0 = kvb + (int64_t)min(max(pages[0], 0), np) * kQkDim + 16 * sx0;
    const unsigned char* src1 = kvb + (int64_t)min(max(pages[1], 0), np) * kQkDim + 16 * sx1;
    LDS_AS unsigned char* dst = stage + w * kGroupBytes;
#pragma unroll
    for (int n = 0; n < Shape<NHT>::dma; ++n) lds_dma16(((n & 1) ? src1 : src0) + 64 * (n >> 1), dst + 1024 * n);
  } else {
    const int hf = w & 1;
    const unsigned char* src = kvb + (int64_t)min(max(pages[0], 0), np) * kQkDim + 16 * (sx0 ^ hf);
    LDS_AS unsigned char* dst = stage + (w >> 1) * kGroupBytes + 1024 * hf;
#pragma unroll
    for (int k = 0; k < Shape<NHT>::dma; ++k) lds_dma16(src + 64 * k, dst + 2048 * k);
  }
}

// Q^T B operands of the wave's 16-head tiles for query row qo: slot order
// per latent block kb: 16 dims at 128kb + 16g, then 16 at 128kb + 64 + 16g;
// the rope block's 16 dims 512 + 16g sit in both halves of its operand (the
// key operand's high half is zero, so the copy adds nothing).
template <int NHT>
struct QTile {
  i32x8 b[NHT][4];  // latent blocks
  i32x8 r[NHT];     // rope dims 512 + 16g .. +15, twice
};

template <int NHT>
__device__ __forceinline__ void load_query(const pa_mla_decode_args& a, int qo, int w, int c, int g, QTile<NHT>& q) {
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) {
    const unsigned char* row =
        (const unsigned char*)a.query + ((int64_t)qo * kHeads + 16 * NHT * w + 16 * ht + c) * kQkDim + 16 * g;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const i32x4 lo = *(const i32x4*)(row + 128 * kb);
      const i32x4 hi = *(const i32x4*)(row + 128 * kb + 64);
      q.b[ht][kb] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    // the rope dims loaded twice, straight into both halves: a register
    // copy would wait for the load (vmcnt counts in order, so also for the
    // next block's DMA in flight) at the end of every block
    const i32x4 r0 = *(const i32x4*)(row + 512);
    const i32x4 r1 = *(const i32x4*)(row + 512 + opaque_zero());
    q.r[ht] = i32x8{r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
  }
}

// A negative softmax scale: the queries' signs are flipped (exact in fp8)
// and the kernel scales by |softmax_scale|, so the softmax can take its
// maxima on the raw logits.  Applied after the loop top's wait (applied at
// the load it would wait there for the next block's DMA).
template <int NHT>
__device__ __forceinline__ void flip_query_signs(QTile<NHT>& q) {
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) q.b[ht][kb] ^= (int)0x80808080u;
    q.r[ht] ^= (int)0x80808080u;
  }
}

// ds_read_b64_tr_b8 as inline assembly: the compiler's own intrinsic makes it
// wait for every outstanding DMA (vmcnt(0)) before the read, which would
// serialise the next block's DMA with this block's value product.  The
// reads target the stage the DMA is not writing; their completion is
// awaited explicitly with lgkmcnt.
template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr8(unsigned addr) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}

// A operand of one 16-dim row tile: tiles 2k (low dword) and 2k+1 (high) of
// each 32-token group k.
template <int OFF>
__device__ __forceinline__ i32x8 read_tr_operand(const unsigned (&base)[4]) {
  const i32x2 r0 = lds_read_tr8<OFF>(base[0]);
  const i32x2 r1 = lds_read_tr8<OFF>(base[1]);
  const i32x2 r2 = lds_read_tr8<OFF>(base[2]);
  const i32x2 r3 = lds_read_tr8<OFF>(base[3]);
  return i32x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}


// O^T += V^T P^T over one 128-token block held at stage `sb`: per 32 value
// dims, eight transpose reads give the A operands of two 16-dim row tiles.
// Software pipelined by hand: the reads of block db + 1 are issued before
// the MFMAs of block db, which wait only for their own eight reads.
template <bool FIRST, bool PRECISE, int NHT>
__device__ __forceinline__ void pv_block(const LDS_AS unsigned char* sb, f32x4 (&o)[16][2][NHT],
                                         const i32x8 (&phi)[NHT], const i32x8 (&plo)[NHT], const int (&sbs)[NHT],
                                         const int (&sbl)[NHT], int sa, int vbase) {
  // unit u = 2db + rt sits in quad u / 4, slot (u % 4) ^ swz of the lane's
  // row 16(c / 8) + 4g + ..: swz = c / 8 + 2 (g % 2)
  const int l = lane_id();
  const int g = ((l >> 3) & 1) | (((l >> 4) & 1) << 1);
  unsigned base[4][4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl)
#pragma unroll
    for (int k = 0; k < 4; ++k) base[sl][k] = (unsigned)(uintptr_t)(sb + k * kGroupBytes + vbase + 16 * (sl ^ g));
  i32x8 va[2][2];
  auto load = [&](auto dbc, i32x8(&dst)[2]) {
    constexpr int db = decltype(dbc)::value;
    dst[0] = read_tr_operand<((2 * db) >> 2) * kQuadBytes>(base[(2 * db) & 3]);
    dst[1] = read_tr_operand<((2 * db + 1) >> 2) * kQuadBytes>(base[(2 * db + 1) & 3]);
  };
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  load(std::integral_constant<int, 0>{}, va[0]);
  static_for<16>([&](auto dbc) {
    constexpr int db = decltype(dbc)::value;
    if constexpr (db + 1 < 16) {
      load(std::integral_constant<int, db + 1>{}, va[(db + 1) & 1]);
      asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
    } else {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        pv_mfma<FIRST>(o[db][rt][ht], va[db & 1][rt], phi[ht], sa, sbs[ht]);
        if (PRECISE) pv_mfma<false>(o[db][rt][ht], va[db & 1][rt], plo[ht], sa, sbl[ht]);
      }
  });
}

template <bool PRECISE, int NHT>
__global__ __launch_bounds__(Shape<NHT>::threads, 1) void mla_fp8_decode_kernel(const pa_mla_decode_args a) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[2 * kStageBytes];
  LDS_AS unsigned char* lds = (LDS_AS unsigned char*)lds_raw;

  const int lane = threadIdx.x & 63;
  const int w = uni(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;

  int ws = uni(a.work_indptr[blockIdx.x]);
  int we = uni(a.work_indptr[blockIdx.x + 1]);
  ws = min(max(ws, 0), a.num_works);
  we = min(max(we, ws), a.num_works);
  if (ws >= we) return;

  // |scale| log2(e): a negative scale's sign is carried by the queries.  A
  // zero scale is taken as the smallest normal float, the same uniform
  // softmax, but masked logits stay -inf (-inf x 0 would be NaN).
  const float scale2 = fmaxf(__builtin_fabsf(a.softmax_scale) * kLog2e, 0x1p-126f);

  // Unit cursors: cur (computed now), c1 (DMA issued this step), c2 (page
  // index prefetched this step).
  Cursor cur;
  cur.wi = ws;
  cur.blk = 0;
  cur.w = load_work(a, ws);
  Cursor c1 = cur;
  advance(a, c1, we);
  Cursor c2 = c1;
  advance(a, c2, we);

  QTile<NHT> q;
  load_query(a, cur.w.qo, w, c, g, q);
  issue_block<NHT>(a, lds, w, unit_pages<NHT>(a, cur, w));
  i32x2 pg1 = valid(c1, we) ? unit_pages<NHT>(a, c1, w) : i32x2{0, 0};

  // O^T accumulators: [32-dim block][16-dim row tile][head tile].
  f32x4 o[16][2][NHT];
  float m0[NHT], lsum[NHT];
#pragma unroll
  for (int ht = 0; ht < NHT; ++ht) {
    m0[ht] = 0.f;    // reference exponent of each head (set on a work's first block)
    lsum[ht] = 0.f;  // this lane's share of the denominator, in units of 2^m0
  }

  // Lane bases inside a stage.  Keys: token row 16T + c, unit 8kb + g
  // (+4 for the upper 64 dims).  Values (transpose reads): lanes c < 8
  // address tile 2k, lanes c >= 8 tile 2k+1, row 4g + (c / 2) % 4 of the
  // tile, unit 2db + rt, byte 8 (c % 2); the low dword then holds tile 2k
  // and the high dword tile 2k+1 of value dim 32db + 16rt + c.
  // key rows 16(T % 2) + c: swz = T % 2 + 2 (c / 4 % 2)
  const int kbase0 = c * 64 + 16 * (g ^ (((c >> 2) & 1) << 1));
  const int kbase1 = c * 64 + 16 * (g ^ (((c >> 2) & 1) << 1) ^ 1);
  const int vbase = (16 * (c >> 3) + 4 * g + ((c >> 1) & 3)) * 64 + (c & 1) * 8;
  const int unit_scale = 127;  // e8m0 2^0

  int st = 0;
  while (true) {
    // vmcnt(0): this block's DMA (and the queries) have landed; lgkmcnt(0)
    // as a builtin also tells the compiler's wait insertion that no scalar
    // load is outstanding, so the key reads below are awaited by count
    // rather than with lgkmcnt(0).
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0) & ~(15 << 8));
    asm volatile("s_barrier" ::: "memory");
    if (a.softmax_scale < 0.f) flip_query_signs(q);
    if (valid(c1, we)) {
      issue_block<NHT>(a, lds + (st ^ 1) * kStageBytes, w, pg1);
      if (valid(c2, we)) pg1 = unit_pages<NHT>(a, c2, w);
    }
    const LDS_AS unsigned char* sb = lds + st * kStageBytes;

    // ---- S^T = K Q^T and softmax, in two halves of four 16-token tiles ----
    // The probabilities go into the value product with e8m0 block scales.
    // v_mfma_scale_f32_16x16x128_f8f6f4 scales k-slots in blocks of 32: the
    // low 16 bytes (tiles 0..3) of lane groups {0,1} form block 0, of {2,3}
    // block 1, the high 16 bytes (tiles 4..7) blocks 2 and 3, and lane
    // group j supplies the scale of block j.  So each half of the block has
    // one exponent per lane pair (g, g^1) and head: e = ceil(pair max), the
    // probabilities p = 2^(x - e) sit at the top of the fp8 range, and the
    // MFMA multiplies them back by 2^(e - m0).
    const bool first = cur.blk == 0;
    const bool last = cur.blk == cur.w.nblk - 1;
    const int len = cur.w.kv1 - cur.w.kv0 - cur.blk * kBlock;  // valid tokens from this block on
    i32x8 phi[NHT], plo[NHT];
    int kexp[2][NHT];     // [half][head tile]: block exponent - m0
    float hmax[2][NHT];   // [half][head tile]: the head's maximum raw logit
    float bexp[2][NHT];   // [half][head tile]: block exponent e of the lane pair
    float psum[2][NHT];   // [half][head tile]: the lane's sum of p = 2^(x - e)
    f32x4 s0[4][NHT], s1[4][NHT];

    // Key operand of product j = 5t + kb of a half block: tile
    // T = 4 half + t, latent block kb < 4 (two 16-byte reads), or kb = 4:
    // the rope dims in the low half, zeros in the high half.
    auto key_operand = [&](auto jc, int half, i32x8& dst) {
      constexpr int j = decltype(jc)::value, t = j / 5, kb = j % 5;
      const int T = 4 * half + t;
      const LDS_AS unsigned char* kr = sb + (T >> 1) * kGroupBytes + (T & 1) * 1024 + ((T & 1) ? kbase1 : kbase0);
      if constexpr (kb < 4) {
        const i32x4 lo = *(const LDS_AS i32x4*)(kr + 2 * kb * kQuadBytes);
        const i32x4 hi = *(const LDS_AS i32x4*)(kr + (2 * kb + 1) * kQuadBytes);
        dst = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      } else {
        const i32x4 r4 = *(const LDS_AS i32x4*)(kr + 8 * kQuadBytes);
        dst = i32x8{r4[0], r4[1], r4[2], r4[3], 0, 0, 0, 0};
      }
    };
    auto key_product = [&](auto jc, f32x4 (&s)[4][NHT], const i32x8& ka) {
      constexpr int j = decltype(jc)::value, t = j / 5, kb = j % 5;
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        if constexpr (kb == 0)
          qk_mfma<true>(s[t][ht], ka, q.b[ht][0]);
        else if constexpr (kb < 4)
          qk_mfma<false>(s[t][ht], ka, q.b[ht][kb]);
        else
          qk_mfma<false>(s[t][ht], ka, q.r[ht]);
      }
    };
    // Logits of positions past the range -> -inf (only a work's last block).
    auto mask = [&](f32x4 (&s)[4][NHT], int half) {
      if (len < (half + 1) * (kBlock / 2)) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool keep = 16 * (4 * half + t) + 4 * g + i < len;
#pragma unroll
            for (int ht = 0; ht < NHT; ++ht) s[t][ht][i] = keep ? s[t][ht][i] : kNegInf;
          }
      }
    };
    // Softmax, branch-free part: maxima of the raw logits (the scale is
    // positive), the lane pair's block exponent e = ceil(scaled pair max),
    // p = 2^(x scale - e) packed to fp8, and the lane's sum of p.
    auto softmax_probs = [&](const f32x4 (&s)[4][NHT], int half) {
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        float x = kNegInf;
#pragma unroll
        for (int t = 0; t < 4; ++t) x = fmaxf(x, fmaxf(fmaxf(s[t][ht][0], s[t][ht][1]), fmaxf(s[t][ht][2], s[t][ht][3])));
        hmax[half][ht] = max_over_groups(x);
        const float xp = max_over_pair(x);
        const float e = xp == kNegInf ? 0.f : __builtin_ceilf(xp * scale2);
        bexp[half][ht] = e;
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float pv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][ht][i], scale2, -e));
            acc += pv[i];
          }
          const uint32_t h = pack4_fp8(pv[0], pv[1], pv[2], pv[3]);
          phi[ht][4 * half + t] = (int)h;
          if (PRECISE) {
            const f32x2 b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, false);
            const f32x2 b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, true);
            // low terms carried x16 (scale 2^-4 in their MFMA), clear of
            // the e4m3fn subnormal range
            plo[ht][4 * half + t] = (int)pack4_fp8(16.f * (pv[0] - b0[0]), 16.f * (pv[1] - b0[1]),
                                                   16.f * (pv[2] - b1[0]), 16.f * (pv[3] - b1[1]));
          }
        }
        psum[half][ht] = acc;
      }
    };
    // Softmax, the rest: the reference exponent m0 (set on a work's first
    // block, moved in the rare case the head maximum outgrows it), the block
    // scale exponent e - m0 (clamped to the e8m0 range: a block more than 127
    // below m0 counts as 2^-127 of m0, i.e. nothing) and the denominator.
    auto softmax_scales = [&](int half) {
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        const float hm = hmax[half][ht] == kNegInf ? kNegInf : hmax[half][ht] * scale2;
        if (half == 0 && first) m0[ht] = hm == kNegInf ? 0.f : __builtin_ceilf(hm) + 40.f;
        const bool up = hm > m0[ht] + kRescaleMargin;
        if (__builtin_expect(__ballot(up) != 0, 0)) {
          // move m0: the denominator, the first half's block exponents and
          // (past the work's first block) the accumulators follow it
          const float mn = up ? __builtin_ceilf(hm) + 40.f : m0[ht];
          const float f = __builtin_amdgcn_exp2f(m0[ht] - mn);
          lsum[ht] *= f;
          if (half == 1) kexp[0][ht] = max(kexp[0][ht] + (int)(m0[ht] - mn), -127);
          m0[ht] = mn;
          if (!first) rescale_acc(o, ht, f);
        }
        kexp[half][ht] = (int)fminf(fmaxf(bexp[half][ht] - m0[ht], -127.f), 127.f);
        lsum[ht] += __builtin_ldexpf(psum[half][ht], kexp[half][ht]);
      }
    };

    // Key products of both halves, software pipelined: the reads of product
    // j + 2 are issued before product j (the scheduling barriers keep that
    // order; the compiler's own schedule reads each operand just before its
    // product and waits for it).  Interleaving the softmax VALU work into
    // these products measured slower: the other wave on the SIMD already
    // fills the matrix core's gaps.
    auto key_half = [&](int half, f32x4 (&s)[4][NHT]) {
      i32x8 kq[3];
      key_operand(std::integral_constant<int, 0>{}, half, kq[0]);
      key_operand(std::integral_constant<int, 1>{}, half, kq[1]);
      static_for<20>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if constexpr (j + 2 < 20) key_operand(std::integral_constant<int, j + 2>{}, half, kq[(j + 2) % 3]);
        __builtin_amdgcn_sched_barrier(0);
        key_product(jc, s, kq[j % 3]);
        __builtin_amdgcn_sched_barrier(0);
      });
    };
    key_half(0, s0);
    key_half(1, s1);
    mask(s0, 0);
    softmax_probs(s0, 0);
    softmax_scales(0);
    mask(s1, 1);
    softmax_probs(s1, 1);
    softmax_scales(1);
    // Scale VGPR of lane group g = exponent of block g: (half 0, pair {0,1}),
    // (half 0, pair {2,3}), (half 1, pair {0,1}), (half 1, pair {2,3}).
    int sbv[2][NHT];  // [hi, lo term][head tile]
#pragma unroll
    for (int ht = 0; ht < NHT; ++ht) {
      const int t0 = other_half_wave(kexp[0][ht]);  // group 1 <- group 3
      const int t1 = other_half_wave(kexp[1][ht]);  // group 2 <- group 0
      const int k = g == 0 ? kexp[0][ht] : g == 1 ? t0 : g == 2 ? t1 : kexp[1][ht];
      sbv[0][ht] = k + 127;
      sbv[1][ht] = max(k + 127 - 4, 0);
    }


    // ---- O^T += V^T P^T: 16 blocks of 32 value dims ----
    probs_ready<PRECISE>(phi, plo);
    if (first)
      pv_block<true, PRECISE, NHT>(sb, o, phi, plo, sbv[0], sbv[1], unit_scale, vbase);
    else
      pv_block<false, PRECISE, NHT>(sb, o, phi, plo, sbv[0], sbv[1], unit_scale, vbase);

    if (last) {
      // ---- epilogue: normalise and store the work's rows ----
      // One accumulator tile at a time (a scheduling barrier per tile): the
      // scaled tiles would otherwise all be formed before the stores.
      agpr_settle();
      const bool direct = cur.w.pql < 0;
#pragma unroll
      for (int ht = 0; ht < NHT; ++ht) {
        const float l = sum_over_groups(lsum[ht]);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int head = 16 * NHT * w + 16 * ht + c;
        const int64_t prow = direct ? (int64_t)cur.w.qo * kHeads + head : (int64_t)cur.w.pql * kHeads + head;
        // the lane's value dims 4g .. 4g+3 of each 16-dim tile: one pointer,
        // constant offsets per tile
        unsigned char* lrow = direct ? (unsigned char*)a.final_output + prow * (kVDim * 2) + 8 * g
                                     : (unsigned char*)(a.split_output + prow * kVDim) + 16 * g;
#pragma unroll
        for (int db = 0; db < 16; ++db)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            f32x4 v = read_acc(o[db][rt][ht]) * inv;
            // an empty range (l = 0) stores zeros whatever its page held
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = l > 0.f ? v[i] : 0.f;
            const int d0 = 32 * db + 16 * rt;
            if (direct) {
              const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
              const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
              *(i32x2*)(lrow + 2 * d0) = i32x2{(int)lo, (int)hi};
            } else {
              *(f32x4*)(lrow + 4 * d0) = v;
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        if (!direct && g == 0) a.split_lse[prow] = l > 0.f ? (m0[ht] + __builtin_amdgcn_logf(l)) * kLn2 : kNegInf;
        lsum[ht] = 0.f;
      }
    }

    if (!valid(c1, we)) break;
    // The queries of the next block's work are reloaded (from L2) after
    // every block rather than held in registers through the softmax and the
    // value product: that keeps the VGPRs within budget (no scratch spills,
    // whose reloads would wait on the in-flight DMA through vmcnt).  They
    // arrive with the next block's DMA, which the loop top waits for.
    load_query(a, c1.w.qo, w, c, g, q);
    cur = c1;
    c1 = c2;
    advance(a, c2, we);
    st ^= 1;
  }
}

// One wave per (group, head): lane l merges value dims 8l .. 8l+7.
__global__ __launch_bounds__(256) void mla_fp8_reduce_kernel(const pa_mla_reduce_args a) {
  const int gidx = blockIdx.x;
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  int p0 = a.reduce_indptr[gidx], p1 = a.reduce_indptr[gidx + 1];
  p0 = min(max(p0, 0), a.num_partial_map);
  p1 = min(max(p1, p0), a.num_partial_map);
  if (p0 >= p1) return;
  const int row0 = min(max(a.reduce_final_map[2 * gidx], 0), a.num_rows);
  const int row1 = min(max(a.reduce_final_map[2 * gidx + 1], row0), a.num_rows);
  // Pieces are merged in batches of kBatch whose loads (lse and the lane's
  // 8 value dims) are all in flight together, with an online log-sum-exp:
  // one round trip per batch instead of two per piece.  Pieces outside the
  // split buffers or with lse -inf (no visible key) are skipped.
  constexpr int kBatch = 8;
  for (int row = row0; row < row1; ++row) {
    const int r = row - row0;
    float mx = kNegInf, wsum = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i0 = p0; i0 < p1; i0 += kBatch) {
      int64_t prow[kBatch];
      bool ok[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int pr = i0 + k < p1 ? a.reduce_partial_map[i0 + k] + r : -1;
        ok[k] = pr >= 0 && pr < a.num_partial;
        prow[k] = (int64_t)(ok[k] ? pr : 0) * kHeads + head;
      }
      float l[kBatch];
      f32x4 x0[kBatch], x1[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        l[k] = kNegInf;
        x0[k] = x1[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (ok[k]) {  // wave-uniform
          const f32x4* src = (const f32x4*)(a.split_output + prow[k] * kVDim + 8 * lane);
          l[k] = a.split_lse[prow[k]];
          x0[k] = src[0];
          x1[k] = src[1];
        }
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (l[k] == kNegInf) continue;
        const float mn = fmaxf(mx, l[k]);
        const float fold = mx == kNegInf ? 0.f : __expf(mx - mn);
        const float w = __expf(l[k] - mn);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[j] = acc[j] * fold + w * x0[k][j];
          acc[4 + j] = acc[4 + j] * fold + w * x1[k][j];
        }
        wsum = wsum * fold + w;
        mx = mn;
      }
    }
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
    uint32_t packed[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      packed[k] = f32_to_bf16_bits(acc[2 * k] * inv) | (f32_to_bf16_bits(acc[2 * k + 1] * inv) << 16);
    unsigned char* orow = (unsigned char*)a.final_output + ((int64_t)row * kHeads + head) * (kVDim * 2);
    *(i32x4*)(orow + 16 * lane) = i32x4{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
    if (a.final_lse && lane == 0)
      a.final_lse[(int64_t)row * kHeads + head] = wsum > 0.f ? mx + __logf(wsum) : kNegInf;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// One e4m3fnuz byte to e4m3fn by value.  fnuz(x) = fn(x) / 2 for every
// non-special code, so a magnitude field >= 16 (exponent >= 2) loses one
// exponent step, exact; below 16 both formats are linear in the field
// (fnuz m * 2^-10, fn m * 2^-9), so the field halves, ties to even.
__device__ __forceinline__ uint32_t fnuz_byte_to_fn(uint32_t b) {
  const uint32_t mag = b & 0x7fu;
  const uint32_t half = (mag >> 1) + (mag & (mag >> 1) & 1u);
  const uint32_t out = (mag >= 16u ? mag - 8u : half) | (b & 0x80u);
  return b == 0x80u ? 0x7fu : out;
}

// Thread t converts 16 bytes: chunk t % (row_bytes / 16) of destination row
// t / (row_bytes / 16).
__global__ __launch_bounds__(256) void fnuz_to_fn_kernel(const unsigned char* __restrict__ src,
                                                         const int32_t* __restrict__ rows, int64_t num_rows,
                                                         int64_t num_src_rows, int64_t row_bytes,
                                                         unsigned char* __restrict__ dst) {
  const int64_t chunks = row_bytes >> 4;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= num_rows * chunks) return;
  const int64_t r = t / chunks, c = t - r * chunks;
  int64_t sr = rows ? (int64_t)rows[r] : r;
  pa_note(sr < 0 || sr >= num_src_rows, PA_VIOLATION_PAGE);
  sr = sr < 0 ? 0 : (sr >= num_src_rows ? num_src_rows - 1 : sr);
  const i32x4 v = *(const i32x4*)(src + sr * row_bytes + 16 * c);
  i32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t w = (uint32_t)v[k];
    o[k] = (int)(fnuz_byte_to_fn(w & 0xffu) | fnuz_byte_to_fn((w >> 8) & 0xffu) << 8 |
                 fnuz_byte_to_fn((w >> 16) & 0xffu) << 16 | fnuz_byte_to_fn(w >> 24) << 24);
  }
  *(i32x4*)(dst + r * row_bytes + 16 * c) = o;
}

#ifdef PA_FP8_CHECKED
// Checked builds: the decode's inputs against the ranges load_work and
// issue_block clamp them into -- the work records the workers walk and every
// page-list entry -- in a kernel of its own, run before the decode (the
// decode kernel has no registers to spare for the checks).
__global__ __launch_bounds__(256) void mla_check_kernel(const pa_mla_decode_args a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < a.num_page_indices) {
    const int p = a.kv_page_indices[i];
    pa_note(p < 0 || (int64_t)p >= a.num_pages, PA_VIOLATION_PAGE);
  }
  const int w0 = a.work_indptr[0], w1 = a.work_indptr[a.num_workers];
  if (i >= w0 && i < w1 && i < a.num_works) {
    const int32_t* w = a.work_info + 8 * i;
    const int pql = w[1], qo = w[2], kv0 = w[4], kv1 = w[5];
    pa_note(qo < 0 || qo >= a.num_rows || pql < -1 || pql >= a.num_partial || kv0 < 0 || kv1 < kv0 ||
                kv1 > a.num_page_indices,
            PA_VIOLATION_WORK);
  }
}
#endif

}  // namespace

PA_CHECK_DEFINE_TAKE(pa_violations_mla)

extern "C" int pa_fp8_fnuz_to_fn(const void* src, const int32_t* rows, int64_t num_rows, int64_t num_src_rows,
                                 int64_t row_bytes, void* dst, void* stream) {
  if (num_rows < 0 || num_src_rows < 0 || row_bytes <= 0 || row_bytes % 16) return PA_ERR_SHAPE;
  if (num_rows == 0) return 0;
  if (num_src_rows == 0) return PA_ERR_SHAPE;
  if (!src || !dst) return PA_ERR_NULL_ARG;
  if (!aligned16(src) || !aligned16(dst)) return PA_ERR_ALIGN;
  const int64_t threads = num_rows * (row_bytes / 16);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffLL) return PA_ERR_SHAPE;
  hipLaunchKernelGGL(fnuz_to_fn_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const unsigned char*)src, rows, num_rows, num_src_rows, row_bytes, (unsigned char*)dst);
  return (int)hipGetLastError();
}

extern "C" int pa_fp8_mla_decode(const pa_mla_decode_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (a->num_workers < 0 || a->num_works < 0 || a->num_rows < 0 || a->num_partial < 0 ||
      a->num_page_indices < 0 || a->num_pages < 0)
    return PA_ERR_SHAPE;
  if (a->num_workers == 0 || a->num_works == 0) return 0;
  if (a->num_rows == 0 || a->num_pages == 0) return PA_ERR_SHAPE;
  if (a->num_pages > 0x7fffffffLL) return PA_ERR_SHAPE;
  if (!a->query || !a->kv_buffer || !a->work_indptr || !a->work_info || !a->final_output) return PA_ERR_NULL_ARG;
  if (a->num_page_indices > 0 && !a->kv_page_indices) return PA_ERR_NULL_ARG;
  if (a->num_partial > 0 && (!a->split_output || !a->split_lse)) return PA_ERR_NULL_ARG;
  if (!aligned16(a->query) || !aligned16(a->kv_buffer) || !aligned16(a->final_output) ||
      (a->split_output && !aligned16(a->split_output)))
    return PA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
#ifdef PA_FP8_CHECKED
  {
    const int64_t n = a->num_page_indices > a->num_works ? a->num_page_indices : a->num_works;
    hipLaunchKernelGGL(mla_check_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, *a);
  }
#endif
  constexpr int kNht = MLA_HEAD_TILES;
  if (a->precise_p)
    hipLaunchKernelGGL((mla_fp8_decode_kernel<true, kNht>), dim3(a->num_workers), dim3(Shape<kNht>::threads), 0, s,
                       *a);
  else
    hipLaunchKernelGGL((mla_fp8_decode_kernel<false, kNht>), dim3(a->num_workers), dim3(Shape<kNht>::threads), 0, s,
                       *a);
  return (int)hipGetLastError();
}

extern "C" int pa_fp8_mla_reduce(const pa_mla_reduce_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (a->num_groups < 0 || a->num_partial < 0 || a->num_partial_map < 0 || a->num_rows < 0) return PA_ERR_SHAPE;
  if (a->num_groups == 0) return 0;
  if (!a->reduce_indptr || !a->reduce_final_map || !a->final_output) return PA_ERR_NULL_ARG;
  if (a->num_partial > 0 && (!a->split_output || !a->split_lse || !a->reduce_partial_map)) return PA_ERR_NULL_ARG;
  if (!aligned16(a->final_output) || (a->split_output && !aligned16(a->split_output))) return PA_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(mla_fp8_reduce_kernel, dim3(a->num_groups, kHeads / 4), dim3(256), 0, s, *a);
  return (int)hipGetLastError();
}

extern "C" int pa_fp8_mla_plan_sizes(int num_rows, int num_workers, int* max_works, int* max_partials) {
  if (num_rows < 0 || num_workers <= 0) return PA_ERR_SHAPE;
  if (!max_works || !max_partials) return PA_ERR_NULL_ARG;
  mla_plan_sizes(num_rows, num_workers, max_works, max_partials);
  return 0;
}

extern "C" int pa_fp8_mla_plan(const int32_t* qo_indptr, const int32_t* kv_indptr, int num_seqs, int num_workers,
                               int max_works, int max_partials, int32_t* work_indptr, int32_t* work_info,
                               int32_t* reduce_indptr, int32_t* reduce_final_map, int32_t* reduce_partial_map,
                               int* num_groups, int* num_partials) {
  if (!qo_indptr || !kv_indptr || !work_indptr || !reduce_indptr || !num_groups || !num_partials)
    return PA_ERR_NULL_ARG;
  if (num_seqs < 0 || num_workers <= 0 || max_works < 0 || max_partials < 0) return PA_ERR_SHAPE;
  if (max_works > 0 && !work_info) return PA_ERR_NULL_ARG;
  const int rows = qo_indptr[num_seqs] - qo_indptr[0];
  if (rows > 0 && !reduce_final_map) return PA_ERR_NULL_ARG;
  if (max_partials > 0 && !reduce_partial_map) return PA_ERR_NULL_ARG;
  const int n = mla_plan(qo_indptr, kv_indptr, num_seqs, num_workers, max_works, max_partials, work_indptr,
                         work_info, reduce_indptr, reduce_final_map, reduce_partial_map, num_groups, num_partials);
  return n < 0 ? PA_ERR_SHAPE : n;
}
