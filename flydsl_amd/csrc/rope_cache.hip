// KV-cache writer for MI355X (gfx950): NeoX RoPE on the new tokens' Q and K
// heads, and K / V scattered into the paged cache the decode kernels read,
// in one launch.  Behaviour follows kernels/fused_rope_cache_kernel.py
// (kernel :105-412, launch :420-512) and the reference test's torch
// semantics (tests/kernels/test_fused_rope_cache.py:162-237).
//
// Work decomposition.  A head row (one token, one Q or K head, head_dim D
// values) is held by D/8 lanes, 8 consecutive values (16 bytes) each, so a
// wave holds 64/(D/8) rows and a 256-thread workgroup 4x that.  Rows
// 0 .. QH-1 of a token are its Q heads, rows QH .. QH+KH-1 its K heads; a
// K row also loads the matching V head and writes both to the cache.  The
// NeoX partner of value d (d +- D/2) sits in the lane D/16 further along the
// row and comes over with a lane shuffle.  All global accesses are 16-byte
// vectors except the cache layouts whose value dimension is strided.
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

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

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

// float -> bf16 / f16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t f2h(float f, bool bf) {
  if (bf) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  }
  _Float16 h = (_Float16)f;
  uint16_t s;
  __builtin_memcpy(&s, &h, 2);
  return s;
}

// Round a float to the input precision and back.
__device__ __forceinline__ float rnd(float f, bool bf) { return h2f(f2h(f, bf), bf); }

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
// reads int64 positions and slots as their low words).
__device__ __forceinline__ int load_index(const void* p, int64_t t, bool i64) {
  return i64 ? ((const int32_t*)p)[2 * t] : ((const int32_t*)p)[t];
}

template <bool BF16, int LAYOUT, bool SCALE>
__global__ __launch_bounds__(kRcThreads) void pa_rope_cache_kernel(const pa_fp8_rope_cache_args a) {
  const int D = a.head_dim;
  const int lpr = D >> 3;                 // lanes per head row
  const int rpw = 64 / lpr;               // head rows per wave
  const int half = lpr >> 1;              // lanes per half row
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rw = lane / lpr;              // row within the wave
  const int l = lane - rw * lpr;          // lane within the row
  const int rows = a.num_q_heads + a.num_kv_heads;
  const int wg_per_token = (rows + rpw * kRcWaves - 1) / (rpw * kRcWaves);
  const int64_t t = blockIdx.x / wg_per_token;
  const int row = (int)(blockIdx.x - t * wg_per_token) * rpw * kRcWaves + wave * rpw + rw;
  const bool live = rw < rpw && row < rows && t < a.num_tokens;
  const bool is_q = row < a.num_q_heads;
  const int kh = row - a.num_q_heads;

  // this lane's 8 values of the row (dims 8l .. 8l+7)
  i32x4 x = {0, 0, 0, 0};
  if (live) {
    const uint16_t* src = is_q ? (const uint16_t*)a.q + t * a.stride_q_tok + (int64_t)row * a.stride_q_head
                               : (const uint16_t*)a.k + t * a.stride_k_tok + (int64_t)kh * a.stride_k_head;
    x = *(const i32x4*)(src + 8 * l);
  }
  // NeoX partner values from the lane half a row away (every lane takes
  // part in the shuffle; rows beyond the wave's last read their own lane).
  const bool first = l < half;
  const int partner = rw < rpw ? rw * lpr + (first ? l + half : l - half) : lane;
  i32x4 xp;
#pragma unroll
  for (int i = 0; i < 4; ++i) xp[i] = __shfl(x[i], partner, 64);
  if (!live) return;

  int pos = load_index(a.positions, t, a.index_i64 != 0);
  pos = pos < 0 ? 0 : (pos >= a.max_pos ? a.max_pos - 1 : pos);  // never read outside the tables
  const int cidx = a.reuse_freqs_front_part ? (8 * l) % (D >> 1) : 8 * l;
  const i32x4 cs = *(const i32x4*)((const uint16_t*)a.cos_cache + (int64_t)pos * a.stride_cos_pos + cidx);
  const i32x4 sn = *(const i32x4*)((const uint16_t*)a.sin_cache + (int64_t)pos * a.stride_sin_pos + cidx);

  float o[8];
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
  i32x4 ob;
#pragma unroll
  for (int i = 0; i < 4; ++i) ob[i] = (int)(f2h(o[2 * i], BF16) | (f2h(o[2 * i + 1], BF16) << 16));
  uint16_t* dst = is_q ? (uint16_t*)a.q_out + t * a.stride_qo_tok + (int64_t)row * a.stride_qo_head
                       : (uint16_t*)a.k_out + t * a.stride_ko_tok + (int64_t)kh * a.stride_ko_head;
  *(i32x4*)(dst + 8 * l) = ob;
  if (is_q) return;

  // ---------------- cache write (K rows) ----------------
  const int slot = load_index(a.slot_mapping, t, a.index_i64 != 0);
  if (slot < 0) return;  // padding token: nothing cached
  const int bs = a.block_size;
  const int64_t bi = slot / bs;
  const int bp = slot - (int)bi * bs;
  if (bi >= a.num_blocks) return;  // outside the cache: nothing written
  const i32x4 vv = *(const i32x4*)((const uint16_t*)a.v + t * a.stride_v_tok + (int64_t)kh * a.stride_v_head + 8 * l);
  const int KH = a.num_kv_heads;
  const int d0 = 8 * l;

  // element offsets (cache element = 1 byte fp8 or 2 bytes bf16/f16)
  int64_t k_off, v_off, v_step;
  if (LAYOUT == PA_CACHE_FLASH) {  // [NB, bs, KH, D] both
    k_off = ((bi * bs + bp) * KH + kh) * D + d0;
    v_off = k_off;
    v_step = 1;
  } else {
    // K [NB, KH, D/16, bs, 16]
    k_off = (((bi * KH + kh) * (D >> 4) + (d0 >> 4)) * bs + bp) * 16 + (d0 & 15);
    if (LAYOUT == PA_CACHE_ATOM) {  // V [NB, KH, D, bs]
      v_off = ((bi * KH + kh) * D + d0) * bs + bp;
      v_step = bs;
    } else {  // V [NB, KH, bs/16, D, 16]
      v_off = ((bi * KH + kh) * (bs >> 4) + (bp >> 4)) * (int64_t)D * 16 + (int64_t)d0 * 16 + (bp & 15);
      v_step = 16;
    }
  }

  if (SCALE) {
    const float krcp = 1.0f / a.k_scale[0];
    const float vrcp = 1.0f / a.v_scale[0];
    float vf[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vf[i] = h2f(((uint32_t)vv[i >> 1] >> ((i & 1) * 16)) & 0xffffu, BF16) * vrcp;
    const uint32_t k0 = pack4_e4m3(o[0] * krcp, o[1] * krcp, o[2] * krcp, o[3] * krcp);
    const uint32_t k1 = pack4_e4m3(o[4] * krcp, o[5] * krcp, o[6] * krcp, o[7] * krcp);
    *(i32x2*)((uint8_t*)a.key_cache + k_off) = i32x2{(int)k0, (int)k1};
    const uint32_t v0 = pack4_e4m3(vf[0], vf[1], vf[2], vf[3]);
    const uint32_t v1 = pack4_e4m3(vf[4], vf[5], vf[6], vf[7]);
    uint8_t* vd = (uint8_t*)a.value_cache + v_off;
    if (LAYOUT == PA_CACHE_FLASH) {
      *(i32x2*)vd = i32x2{(int)v0, (int)v1};
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) vd[i * v_step] = (uint8_t)(((i < 4 ? v0 : v1) >> (8 * (i & 3))) & 0xffu);
    }
  } else {
    *(i32x4*)((uint16_t*)a.key_cache + k_off) = ob;
    uint16_t* vd = (uint16_t*)a.value_cache + v_off;
    if (LAYOUT == PA_CACHE_FLASH) {
      *(i32x4*)vd = vv;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) vd[i * v_step] = (uint16_t)(((uint32_t)vv[i >> 1] >> ((i & 1) * 16)) & 0xffffu);
    }
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

extern "C" int pa_fp8_rope_cache(const pa_fp8_rope_cache_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  if (a->num_tokens < 0 || a->num_q_heads < 0 || a->num_kv_heads < 0 || a->block_size <= 0 || a->num_blocks < 0 ||
      a->max_pos <= 0)
    return PA_ERR_SHAPE;
  const int D = a->head_dim;
  if (D < 16 || D > 256 || (D & 15)) return PA_ERR_HEAD_SIZE;
  if (64 % (D >> 3) != 0) return PA_ERR_HEAD_SIZE;  // whole head rows per wave
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
  const int64_t wg_per_token = (rows + rpw * kRcWaves - 1) / (rpw * kRcWaves);
  const int64_t grid = wg_per_token * a->num_tokens;
  if (grid > 0x7fffffffLL) return PA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const hipError_t err = a->dtype == PA_DTYPE_BF16 ? dispatch_rope_cache<true>(*a, (unsigned)grid, s)
                                                   : dispatch_rope_cache<false>(*a, (unsigned)grid, s);
  return err == hipSuccess ? PA_OK : (int)err;
}
