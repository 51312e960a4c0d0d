// KV-cache writer for MI355X (gfx950): NeoX RoPE on the new tokens' Q and K
// heads, and K / V scattered into the paged cache the decode kernels read,
// in one launch.  Behaviour follows kernels/fused_rope_cache_kernel.py
// (kernel :105-412, launch :420-512) and the reference test's torch
// semantics (tests/kernels/test_fused_rope_cache.py:162-237).
//
// Work decomposition.  A head row (one token, one Q or K head, head_dim D
// values) is held by D/8 lanes, 8 consecutive values (16 bytes) each, so a
// wave holds floor(64/(D/8)) rows at a time (lanes past the last whole row,
// when D/8 does not divide 64 -- D = 96: 5 rows of 12 lanes -- take no
// part): rows of Q heads of one token, or one
// K head's rows of consecutive tokens (which also carry the V rows and the
// cache writes; see the kernel).  The NeoX partner of value d (d +- D/2)
// sits in the lane D/16 further along the row and comes over with a lane
// shuffle.
//
// Arithmetic is the reference's: in the input precision (bf16 or f16),
// every product and the sum rounded to it (round to nearest even):
//   d <  D/2: out = r(r(x[d] cos[d]) - r(x[d+D/2] sin[d]))
//   d >= D/2: out = r(r(x[d] cos[d]) + r(x[d-D/2] sin[d]))
// with cos/sin[d] = row[d % (D/2)] when only the first half is stored.
// The fp8 cache holds e4m3fn(clamp(float(value) * (1/scale), +-448)); the
// reciprocal is the correctly rounded 1/scale, and finite values beyond the
// fp8 range saturate rather than becoming NaN.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_fp8.h"
#include "pa_check.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))

constexpr int kRcWaves = 4;
constexpr int kRcThreads = 64 * kRcWaves;
constexpr float kFp8Max = 448.0f;

__device__ __forceinline__ float h2f(uint32_t bits, bool bf) {
  if (bf) return __uint_as_float(bits << 16);
  _Float16 h;
  uint16_t s = (uint16_t)bits;
  __builtin_memcpy(&h, &s, 2);
  return (float)h;
}

// float -> bf16 / f16 bits, round to nearest even (NaN stays NaN); gfx950
// converts to bf16 in hardware (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f2h(float f, bool bf) {
  uint16_t s;
  if (bf) {
    const __bf16 h = (__bf16)f;
    __builtin_memcpy(&s, &h, 2);
  } else {
    const _Float16 h = (_Float16)f;
    __builtin_memcpy(&s, &h, 2);
  }
  return s;
}

// Round a float to the input precision and back.
__device__ __forceinline__ float rnd(float f, bool bf) {
  return bf ? (float)(__bf16)f : (float)(_Float16)f;
}

// Saturate at the e4m3fn range; NaN stays NaN.
__device__ __forceinline__ float sat_e4m3(float x) { return x > kFp8Max ? kFp8Max : (x < -kFp8Max ? -kFp8Max : x); }

// Four floats -> four e4m3fn bytes (round to nearest even), saturating.
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  a = sat_e4m3(a);
  b = sat_e4m3(b);
  c = sat_e4m3(c);
  d = sat_e4m3(d);
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

// Low 32 bits of element t of an int32 or int64 index tensor (the reference
// reads int64 positions and slots as their low words).  t is wave-uniform:
// read through the constant address space, a scalar load.
__device__ __forceinline__ int load_index(const void* p, int64_t t, bool i64) {
  const __attribute__((address_space(4))) int32_t* c = (const __attribute__((address_space(4))) int32_t*)p;
  return i64 ? c[2 * t] : c[t];
}

// Rotated values o[0..7] of this lane's 8 dims (reference rounding).
template <bool BF16>
__device__ __forceinline__ void rotate8(const i32x4& x, const i32x4& xp, const i32x4& cs, const i32x4& sn, bool first,
                                        float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int sh = (i & 1) * 16;
    const float xv = h2f(((uint32_t)x[i >> 1] >> sh) & 0xffffu, BF16);
    const float pv = h2f(((uint32_t)xp[i >> 1] >> sh) & 0xffffu, BF16);
    const float cv = h2f(((uint32_t)cs[i >> 1] >> sh) & 0xffffu, BF16);
    const float sv = h2f(((uint32_t)sn[i >> 1] >> sh) & 0xffffu, BF16);
    const float xc = rnd(xv * cv, BF16);
    const float ps = rnd(pv * sv, BF16);
    o[i] = rnd(first ? xc - ps : xc + ps, BF16);
  }
}

template <bool BF16>
__device__ __forceinline__ i32x4 pack8(const float (&o)[8]) {
  i32x4 ob;
#pragma unroll
  for (int i = 0; i < 4; ++i) ob[i] = (int)(f2h(o[2 * i], BF16) | (f2h(o[2 * i + 1], BF16) << 16));
  return ob;
}

// Tokens of one cache page sub-block that the value transpose writes whole.
constexpr int kSub = 16;
// LDS of a K/V workgroup: value rows [tokens][D] (2048 elements of at most
// 2 bytes whatever D) and the tokens' slots.
constexpr int kRcLdsElems = 2048;
constexpr int kRcMaxGroup = 128;
// Q wave-units per wave (four rows' loads in flight per lane).
constexpr int kRcQUnits = 4;

// Two kinds of workgroups in one launch.
//
// Q workgroups (blockIdx.x < nq): wave-unit u covers Q rows rs*rpw ..
// rs*rpw + rpw - 1 of token u / ceil(QH / rpw); a wave takes kRcQUnits
// consecutive units.  Token positions are scalar loads; the cos/sin rows
// they select and the head rows are all issued before anything waits.
//
// K/V workgroups: one kv head over a group of G = 4 * rpw consecutive
// tokens, wave w holding tokens w*rpw .. w*rpw + rpw - 1 (one per row).
// Each row is rotated, written to K_out and to the key cache.  Value rows
// go through LDS: a 16-token sub-block whose slots fill 16 consecutive
// positions of one page (the prefill case) is written transposed, 8 tokens
// of one value dim per thread, as whole 8- or 16-byte stores, instead of
// 128 single-element stores per token into as many cache lines; other
// tokens (decode, ragged slots) are written one by one.
template <bool BF16, int LAYOUT, bool SCALE>
__global__ __launch_bounds__(kRcThreads) void pa_rope_cache_kernel(const pa_fp8_rope_cache_args a) {
  // one LDS array: value rows, then the group's slots
  __shared__ __attribute__((aligned(16))) unsigned char lds[kRcLdsElems * 2 + kRcMaxGroup * 4];
  LDS_AS unsigned char* const lds_v = (LDS_AS unsigned char*)lds;
  LDS_AS int* const lds_slot = (LDS_AS int*)(lds_v + kRcLdsElems * 2);

  const int D = a.head_dim;
  const int lpr = D >> 3;                 // lanes per head row
  const int rpw = 64 / lpr;               // head rows per wave
  const int half = lpr >> 1;              // lanes per half row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = lane / lpr;              // row within the wave
  const bool dead = rw >= rpw;            // past the wave's last whole row
  const int l = lane - rw * lpr;          // lane within the row
  const bool first = l < half;
  const int partner = rw * lpr + (first ? l + half : l - half);
  const int cidx = a.reuse_freqs_front_part ? (8 * l) % (D >> 1) : 8 * l;
  const int QH = a.num_q_heads;
  const int KH = a.num_kv_heads;
  const int T = a.num_tokens;
  const bool i64 = a.index_i64 != 0;
  const uint32_t qwpt = (QH + rpw - 1) / rpw;  // Q wave-units per token
  const uint32_t qunits = (uint32_t)T * qwpt;   // < 2^31 (checked at launch)
  const uint32_t nq = (qunits + kRcWaves * kRcQUnits - 1) / (kRcWaves * kRcQUnits);

  if (blockIdx.x < nq) {
    // ---------------- Q rows: kRcQUnits wave-units per wave ----------------
    // Loads are unconditional (a dead lane reads a valid row and drops it),
    // so nothing branches between the loads and their first use.
    i32x4 x[kRcQUnits], cs[kRcQUnits], sn[kRcQUnits];
    uint32_t tq[kRcQUnits];
    int rq[kRcQUnits];
    bool lq[kRcQUnits];
#pragma unroll
    for (int j = 0; j < kRcQUnits; ++j) {
      const uint32_t u = (blockIdx.x * kRcWaves + wave) * kRcQUnits + j;
      const uint32_t t = u / qwpt;
      const int row = (int)(u - t * qwpt) * rpw + rw;
      tq[j] = t;
      rq[j] = row;
      lq[j] = u < qunits && row < QH && !dead;
      const uint32_t tc = __builtin_amdgcn_readfirstlane(u < qunits ? t : (uint32_t)T - 1);
      const int rc = row < QH ? row : QH - 1;
      int p = load_index(a.positions, tc, i64);
      pa_note(lq[j] && (p < 0 || p >= a.max_pos), PA_VIOLATION_POSITION);
      p = p < 0 ? 0 : (p >= a.max_pos ? a.max_pos - 1 : p);  // never read outside the tables
      cs[j] = *(const i32x4*)((const uint16_t*)a.cos_cache + (int64_t)p * a.stride_cos_pos + cidx);
      sn[j] = *(const i32x4*)((const uint16_t*)a.sin_cache + (int64_t)p * a.stride_sin_pos + cidx);
      x[j] = __builtin_nontemporal_load((const i32x4*)((const uint16_t*)a.q + (int64_t)tc * a.stride_q_tok + (int64_t)rc * a.stride_q_head + 8 * l));
    }
    asm volatile("" ::: "memory");  // every load above is issued before the first wait
#pragma unroll
    for (int j = 0; j < kRcQUnits; ++j) {
      i32x4 xp;
#pragma unroll
      for (int i = 0; i < 4; ++i) xp[i] = __shfl(x[j][i], partner, 64);
      if (!lq[j]) continue;
      float o[8];
      rotate8<BF16>(x[j], xp, cs[j], sn[j], first, o);
      *(i32x4*)((uint16_t*)a.q_out + (int64_t)tq[j] * a.stride_qo_tok + (int64_t)rq[j] * a.stride_qo_head + 8 * l) =
          pack8<BF16>(o);
    }
    return;
  }

  // ---------------- K / V rows ----------------
  const int G = kRcWaves * rpw;  // tokens per workgroup
  const uint32_t b = blockIdx.x - nq;
  const uint32_t g = b / KH;
  const int kh = (int)(b - g * KH);
  const int gi = wave * rpw + rw;         // token within the group
  const int tok = (int)g * G + gi;        // this row's token
  const bool live = tok < T && !dead;  // a dead lane's gi aliases the next row
  const int d0 = 8 * l;

  float krcp = 1.0f, vrcp = 1.0f;
  if (SCALE) {
    krcp = 1.0f / ((const __attribute__((address_space(4))) float*)a.k_scale)[0];
    vrcp = 1.0f / ((const __attribute__((address_space(4))) float*)a.v_scale)[0];
  }
  int p = 0, slot = -1;
  if (live) {
    p = i64 ? ((const int32_t*)a.positions)[2 * (int64_t)tok] : ((const int32_t*)a.positions)[tok];
    slot = i64 ? ((const int32_t*)a.slot_mapping)[2 * (int64_t)tok] : ((const int32_t*)a.slot_mapping)[tok];
  }
  i32x4 x = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
  if (live) {  // rows are read once (non-temporal); the tables stay cached for other rows
    x = __builtin_nontemporal_load((const i32x4*)((const uint16_t*)a.k + (int64_t)tok * a.stride_k_tok + (int64_t)kh * a.stride_k_head + d0));
    vv = __builtin_nontemporal_load((const i32x4*)((const uint16_t*)a.v + (int64_t)tok * a.stride_v_tok + (int64_t)kh * a.stride_v_head + d0));
  }
  asm volatile("" ::: "memory");  // row loads issued before the tables wait on the positions
  pa_note(live && (p < 0 || p >= a.max_pos), PA_VIOLATION_POSITION);
  p = p < 0 ? 0 : (p >= a.max_pos ? a.max_pos - 1 : p);
  const i32x4 cs = *(const i32x4*)((const uint16_t*)a.cos_cache + (int64_t)p * a.stride_cos_pos + cidx);
  const i32x4 sn = *(const i32x4*)((const uint16_t*)a.sin_cache + (int64_t)p * a.stride_sin_pos + cidx);
  i32x4 xp;
#pragma unroll
  for (int i = 0; i < 4; ++i) xp[i] = __shfl(x[i], partner, 64);
  float o[8];
  rotate8<BF16>(x, xp, cs, sn, first, o);
  const i32x4 ob = pack8<BF16>(o);
  const int bs = a.block_size;
  const int64_t bi = slot >= 0 ? slot / bs : 0;
  const int bp = slot >= 0 ? slot - (int)bi * bs : 0;
  const bool cached = live && slot >= 0 && bi < a.num_blocks;
  pa_note(live && slot >= 0 && bi >= a.num_blocks, PA_VIOLATION_SLOT);

  // value cache elements of this lane's 8 dims when fp8
  uint32_t v8[2] = {0, 0};
  if (SCALE) {
    float vf[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vf[i] = h2f(((uint32_t)vv[i >> 1] >> ((i & 1) * 16)) & 0xffffu, BF16) * vrcp;
    v8[0] = pack4_e4m3(vf[0], vf[1], vf[2], vf[3]);
    v8[1] = pack4_e4m3(vf[4], vf[5], vf[6], vf[7]);
  }

  if (live)
    *(i32x4*)((uint16_t*)a.k_out + (int64_t)tok * a.stride_ko_tok + (int64_t)kh * a.stride_ko_head + d0) = ob;
  if (cached) {
    int64_t k_off;
    if (LAYOUT == PA_CACHE_FLASH)  // [NB, bs, KH, D]
      k_off = ((bi * bs + bp) * KH + kh) * D + d0;
    else  // [NB, KH, D/16, bs, 16]
      k_off = (((bi * KH + kh) * (D >> 4) + (d0 >> 4)) * bs + bp) * 16 + (d0 & 15);
    if (SCALE) {
      const uint32_t k0 = pack4_e4m3(o[0] * krcp, o[1] * krcp, o[2] * krcp, o[3] * krcp);
      const uint32_t k1 = pack4_e4m3(o[4] * krcp, o[5] * krcp, o[6] * krcp, o[7] * krcp);
      *(i32x2*)((uint8_t*)a.key_cache + k_off) = i32x2{(int)k0, (int)k1};
    } else {
      *(i32x4*)((uint16_t*)a.key_cache + k_off) = ob;
    }
    if (LAYOUT == PA_CACHE_FLASH) {  // value rows are contiguous in this layout
      if (SCALE)
        *(i32x2*)((uint8_t*)a.value_cache + k_off) = i32x2{(int)v8[0], (int)v8[1]};
      else
        *(i32x4*)((uint16_t*)a.value_cache + k_off) = vv;
    }
  }
  if (LAYOUT == PA_CACHE_FLASH) return;

  // value rows -> LDS [token in group][D] (element = 1 or 2 bytes), slots
  if (!dead) {
    if (SCALE)
      *(LDS_AS i32x2*)(lds_v + gi * D + d0) = i32x2{(int)v8[0], (int)v8[1]};
    else
      *(LDS_AS i32x4*)(lds_v + (gi * D + d0) * 2) = vv;
    if (l == 0) lds_slot[gi] = cached ? slot : -1;
  }
  __syncthreads();

  // a 16-token sub-block is written whole when its slots are one page's
  // positions bp0 .. bp0 + 15 in order (bp0 a multiple of 16)
  auto whole = [&](int m) -> bool {
    const int s0 = lds_slot[m * kSub];
    if (s0 < 0 || (bs % kSub) != 0 || ((s0 % bs) % kSub) != 0) return false;
    for (int i = 1; i < kSub; ++i)
      if (lds_slot[m * kSub + i] != s0 + i) return false;
    return true;
  };
  const int nsub = G / kSub;  // 0 when D = 256 (8 tokens per group)
  // transposed writes: item = (sub-block m, value dim d, token half h)
  for (int item = threadIdx.x; item < nsub * D * 2; item += kRcThreads) {
    const int m = item / (2 * D);
    const int d = (item >> 1) - m * D;
    const int h = item & 1;
    if (!whole(m)) continue;
    const int s0 = lds_slot[m * kSub];
    const int64_t sb = s0 / bs;
    const int sp = s0 - (int)sb * bs + 8 * h;  // page position of the first of the 8 tokens
    int64_t v_off;
    if (LAYOUT == PA_CACHE_ATOM)  // [NB, KH, D, bs]
      v_off = ((sb * KH + kh) * D + d) * bs + sp;
    else  // [NB, KH, bs/16, D, 16]
      v_off = ((sb * KH + kh) * (bs >> 4) + (sp >> 4)) * (int64_t)D * 16 + (int64_t)d * 16 + (sp & 15);
    const int r0 = m * kSub + 8 * h;
    if (SCALE) {
      uint32_t w[2] = {0, 0};
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k >> 2] |= (uint32_t)lds_v[(r0 + k) * D + d] << (8 * (k & 3));
      *(i32x2*)((uint8_t*)a.value_cache + v_off) = i32x2{(int)w[0], (int)w[1]};
    } else {
      uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 8; ++k)
        w[k >> 1] |= (uint32_t)((LDS_AS uint16_t*)lds_v)[(r0 + k) * D + d] << (16 * (k & 1));
      *(i32x4*)((uint16_t*)a.value_cache + v_off) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
  }

  // tokens outside whole sub-blocks: one element per value dim
  if (!cached || (gi / kSub < nsub && whole(gi / kSub))) return;
  int64_t v_off, v_step;
  if (LAYOUT == PA_CACHE_ATOM) {  // [NB, KH, D, bs]
    v_off = ((bi * KH + kh) * D + d0) * bs + bp;
    v_step = bs;
  } else {  // [NB, KH, bs/16, D, 16]
    v_off = ((bi * KH + kh) * (bs >> 4) + (bp >> 4)) * (int64_t)D * 16 + (int64_t)d0 * 16 + (bp & 15);
    v_step = 16;
  }
  if (SCALE) {
    uint8_t* vd = (uint8_t*)a.value_cache + v_off;
#pragma unroll
    for (int i = 0; i < 8; ++i) vd[i * v_step] = (uint8_t)((v8[i >> 2] >> (8 * (i & 3))) & 0xffu);
  } else {
    uint16_t* vd = (uint16_t*)a.value_cache + v_off;
#pragma unroll
    for (int i = 0; i < 8; ++i) vd[i * v_step] = (uint16_t)(((uint32_t)vv[i >> 1] >> ((i & 1) * 16)) & 0xffffu);
  }
}

template <bool BF16, int LAYOUT, bool SCALE>
hipError_t launch_rope_cache(const pa_fp8_rope_cache_args& a, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((pa_rope_cache_kernel<BF16, LAYOUT, SCALE>), dim3(grid), dim3(kRcThreads), 0, s, a);
  return hipGetLastError();
}

template <bool BF16>
hipError_t dispatch_rope_cache(const pa_fp8_rope_cache_args& a, unsigned grid, hipStream_t s) {
  const bool sc = a.apply_scale != 0;
  switch (a.cache_layout) {
    case PA_CACHE_FLASH:
      return sc ? launch_rope_cache<BF16, PA_CACHE_FLASH, true>(a, grid, s)
                : launch_rope_cache<BF16, PA_CACHE_FLASH, false>(a, grid, s);
    case PA_CACHE_ATOM:
      return sc ? launch_rope_cache<BF16, PA_CACHE_ATOM, true>(a, grid, s)
                : launch_rope_cache<BF16, PA_CACHE_ATOM, false>(a, grid, s);
    default:
      return sc ? launch_rope_cache<BF16, PA_CACHE_ATOM_TRANS_V, true>(a, grid, s)
                : launch_rope_cache<BF16, PA_CACHE_ATOM_TRANS_V, false>(a, grid, s);
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

PA_CHECK_DEFINE_TAKE(pa_violations_rope_cache)

extern "C" int pa_fp8_rope_cache(const pa_fp8_rope_cache_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (a->num_tokens < 0 || a->num_q_heads < 0 || a->num_kv_heads < 0 || a->block_size <= 0 || a->num_blocks < 0 ||
      a->max_pos <= 0)
    return PA_ERR_SHAPE;
  const int D = a->head_dim;
  // 8 values per lane, a half row a whole number of lanes, a row in a wave
  if (D < 16 || D > 512 || (D & 15)) return PA_ERR_HEAD_SIZE;
  if (a->dtype != PA_DTYPE_BF16 && a->dtype != PA_DTYPE_F16) return PA_ERR_DTYPE;
  if (a->cache_layout != PA_CACHE_FLASH && a->cache_layout != PA_CACHE_ATOM && a->cache_layout != PA_CACHE_ATOM_TRANS_V)
    return PA_ERR_SHAPE;
  if (a->cache_layout == PA_CACHE_ATOM_TRANS_V && (a->block_size & 15)) return PA_ERR_BLOCK_SIZE;
  const int rows = a->num_q_heads + a->num_kv_heads;
  if (a->num_tokens == 0 || rows == 0) return PA_OK;
  if (!a->q_out || !a->positions || !a->cos_cache || !a->sin_cache || (a->num_q_heads > 0 && !a->q))
    return PA_ERR_NULL_ARG;
  if (a->num_kv_heads > 0 && (!a->k || !a->v || !a->k_out || !a->slot_mapping || !a->key_cache || !a->value_cache))
    return PA_ERR_NULL_ARG;
  if (a->apply_scale && (!a->k_scale || !a->v_scale)) return PA_ERR_NULL_ARG;
  // 16-byte vectors: 8 values per lane
  const int64_t strides[] = {a->stride_q_tok, a->stride_q_head, a->stride_k_tok,  a->stride_k_head,
                             a->stride_v_tok, a->stride_v_head, a->stride_qo_tok, a->stride_qo_head,
                             a->stride_ko_tok, a->stride_ko_head, a->stride_cos_pos, a->stride_sin_pos};
  for (int64_t st : strides)
    if (st % 8) return PA_ERR_ALIGN;
  if (!al16(a->q) || !al16(a->k) || !al16(a->v) || !al16(a->q_out) || !al16(a->k_out) || !al16(a->cos_cache) ||
      !al16(a->sin_cache) || !al16(a->key_cache) || !al16(a->value_cache))
    return PA_ERR_ALIGN;
  const int rpw = 64 / (D >> 3);
  const int64_t qunits = (int64_t)((a->num_q_heads + rpw - 1) / rpw) * a->num_tokens;
  if (qunits > 0x7fffffffLL) return PA_ERR_SHAPE;
  const int G = kRcWaves * rpw;  // tokens per K/V workgroup
  const int64_t grid = (qunits + kRcWaves * kRcQUnits - 1) / (kRcWaves * kRcQUnits) +
                       (int64_t)((a->num_tokens + G - 1) / G) * a->num_kv_heads;
  if (grid > 0x7fffffffLL) return PA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const hipError_t err = a->dtype == PA_DTYPE_BF16 ? dispatch_rope_cache<true>(*a, (unsigned)grid, s)
                                                   : dispatch_rope_cache<false>(*a, (unsigned)grid, s);
  return err == hipSuccess ? PA_OK : (int)err;
}
