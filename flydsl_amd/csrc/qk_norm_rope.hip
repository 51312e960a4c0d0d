// Fused per-token RMSNorm + GPT-J RoPE + optional fp8 quantisation of the
// query heads and the single KV row of each token, for MI355X (gfx950), and
// its C ABI (pa_fp8_qk_norm_rope_quant, declared in pa_fp8.h).
//
// Semantics follow kernels/qk_norm_rope_quant.py (kernel :259-640): the
// RMSNorm statistic of the unweighted row, the optional per-channel weight,
// GPT-J rotation of the last RD elements, and the rstd-cancelling fp8
// algebra with float32 or e8m0 group scales.
//
// Work decomposition.  Rows are (token, head) pairs in token-major order,
// head H being the KV row.  One wave owns kRowsPerWave consecutive rows and
// issues every global load of all of them (row, cos/sin, position) before
// computing any, so each wave keeps kRowsPerWave x 64 x 16 B in flight --
// the kernel is HBM-bound (per row: 2D bytes in, D or 2D bytes out).  Lane l
// holds elements [l*VEC, l*VEC + VEC) of the row (VEC = D / 64), so the
// row's square sum is one wave reduction and a quant group of G elements is
// G / VEC adjacent lanes.  No LDS, no barriers.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_fp8.h"

namespace {

constexpr int kRowsPerWave = 4;
constexpr int kWavesPerGroup = 4;
constexpr float kMaxOverSqrt2 = 316.78383797157f;  // float32(448 / sqrt(2))
constexpr float kInvMaxSqrt2 = 0.0031567461f;      // float32(sqrt(2) / 448)
constexpr float kSqrt2 = 1.41421356237f;            // float32(sqrt(2))
constexpr int kE8m0Headroom = 7;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// VEC bf16 values as VEC / 2 dwords, one vector load.
template <int VEC>
struct Raw {
  uint32_t w[VEC / 2];
};

template <int VEC>
__device__ __forceinline__ Raw<VEC> load_raw(const void* p) {
  Raw<VEC> r;
  if constexpr (VEC == 8) {
    const u32x4 v = *(const u32x4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.w[i] = v[i];
  } else if constexpr (VEC == 4) {
    const u32x2 v = *(const u32x2*)p;
    r.w[0] = v[0];
    r.w[1] = v[1];
  } else {
    r.w[0] = *(const uint32_t*)p;
  }
  return r;
}

// Half of the pairs' cos (or sin) values: VEC / 2 bf16.
template <int VEC>
struct Half {
  uint32_t w[VEC / 4 > 0 ? VEC / 4 : 1];
};

template <int VEC>
__device__ __forceinline__ Half<VEC> load_half(const uint16_t* p) {
  Half<VEC> r;
  if constexpr (VEC == 8) {
    const u32x2 v = *(const u32x2*)p;
    r.w[0] = v[0];
    r.w[1] = v[1];
  } else if constexpr (VEC == 4) {
    r.w[0] = *(const uint32_t*)p;
  } else {
    r.w[0] = *p;  // one bf16
  }
  return r;
}

__device__ __forceinline__ float bf16_at(const uint32_t* w, int i) {
  const uint32_t x = w[i >> 1];
  return __uint_as_float((i & 1) ? (x & 0xffff0000u) : (x << 16));
}

// Round to nearest even (finite inputs; NaN keeps a quiet payload).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Maximum over the 2^lg adjacent lanes of a quant group.
__device__ __forceinline__ float group_max(float v, int lg) {
#pragma unroll
  for (int s = 0; s < 6; ++s)
    if (s < lg) v = fmaxf(v, __shfl_xor(v, 1 << s, 64));
  return v;
}

// fp8 e4m3fn of a and b (round to nearest even) into bytes 2*hi, 2*hi + 1 of
// old; values in (-2^-8, 0) become +0 first, as the reference's store does.
template <bool HI>
__device__ __forceinline__ int pack2_fp8(float a, float b, int old) {
  a = (a < 0.0f && a > -0.00390625f) ? 0.0f : a;
  b = (b < 0.0f && b > -0.00390625f) ? 0.0f : b;
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, HI);
}

template <int VEC, bool QUANT, bool E8M0>
__global__ __launch_bounds__(64 * kWavesPerGroup) void pa_qk_norm_rope_kernel(const pa_qk_norm_rope_args a,
                                                                             int tpg_log2) {
  constexpr int D = 64 * VEC;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * kWavesPerGroup + (threadIdx.x >> 6);
  const int H = a.num_q_heads;
  const uint32_t hp = (uint32_t)H + 1;
  const uint32_t rows = (uint32_t)a.num_tokens * hp;
  const int rd = a.rope_head_dim;
  const int rope_lo = (D - rd) / VEC;  // first lane of the rotated part
  const bool is_rope = lane >= rope_lo;
  const int half_off = (lane - rope_lo) * (VEC / 2);  // this lane's first pair
  const uint16_t* cos_tab = (const uint16_t*)a.cos_cache;
  const uint16_t* sin_tab = (const uint16_t*)a.sin_cache;

  // Per-channel weights of this lane's elements (loaded once per wave).
  const Raw<VEC> kvw = load_raw<VEC>((const uint16_t*)a.kv_weight + lane * VEC);
  Raw<VEC> qw;
  const bool q_weighted = a.q_weight != nullptr;
  if (q_weighted) qw = load_raw<VEC>((const uint16_t*)a.q_weight + lane * VEC);

  // ---- every load of the wave's rows first ----
  Raw<VEC> x[kRowsPerWave];
  Half<VEC> cs[kRowsPerWave], sn[kRowsPerWave];
  uint32_t tok[kRowsPerWave], head[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const uint32_t r = wave * kRowsPerWave + i;
    const uint32_t rr = r < rows ? r : rows - 1;  // rows past the end repeat the last (not stored)
    tok[i] = rr / hp;
    head[i] = rr - tok[i] * hp;
    const uint16_t* src = head[i] < (uint32_t)H
                              ? (const uint16_t*)a.q + (int64_t)tok[i] * a.stride_q_tok + (int64_t)head[i] * D
                              : (const uint16_t*)a.kv + (int64_t)tok[i] * a.stride_kv_tok;
    x[i] = load_raw<VEC>(src + lane * VEC);
    // int64 position read as its low word; outside the table the rotation
    // reads zeros, like the reference's range-checked buffer loads.
    const int pos = (int)(uint32_t)(uint64_t)a.positions[tok[i]];
    const bool inside = pos >= 0 && pos < a.max_pos;
    if (is_rope && inside) {
      cs[i] = load_half<VEC>(cos_tab + (int64_t)pos * (rd / 2) + half_off);
      sn[i] = load_half<VEC>(sin_tab + (int64_t)pos * (rd / 2) + half_off);
    } else {
#pragma unroll
      for (int k = 0; k < (VEC / 4 > 0 ? VEC / 4 : 1); ++k) {
        cs[i].w[k] = 0;
        sn[i].w[k] = 0;
      }
    }
  }

  // ---- compute and store each row ----
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const uint32_t r = wave * kRowsPerWave + i;
    if (r >= rows) break;  // wave-uniform
    const bool isq = head[i] < (uint32_t)H;
    const bool weighted = isq ? q_weighted : true;
    float xv[VEC], xw[VEC];
    float sq = 0.0f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      xv[v] = bf16_at(x[i].w, v);
      sq += xv[v] * xv[v];
      const float wv = isq ? (q_weighted ? bf16_at(qw.w, v) : 1.0f) : bf16_at(kvw.w, v);
      xw[v] = weighted ? xv[v] * wv : xv[v];
    }
    sq = wave_sum(sq);
    const float rstd = __builtin_amdgcn_rsqf(sq * (1.0f / D) + 1e-6f);
    float y[VEC];
    if (QUANT) {
      float am = 0.0f;
#pragma unroll
      for (int v = 0; v < VEC; ++v) am = fmaxf(am, fabsf(xw[v]));
      am = fmaxf(group_max(am, tpg_log2), 1e-12f);
      float factor;
      uint32_t e8 = 0;
      float scale32 = 0.0f;
      if (E8M0) {
        const float post = am * rstd * kSqrt2;
        const uint32_t bits = (__float_as_uint(post) + 0x400000u) & 0xff800000u;
        int e = (int)(bits >> 23) - kE8m0Headroom;
        e = e < 0 ? 0 : (e > 255 ? 255 : e);
        e8 = (uint32_t)e;
        factor = rstd * __uint_as_float((uint32_t)(254 - e) << 23);
      } else {
        factor = kMaxOverSqrt2 * __builtin_amdgcn_rcpf(am);
        scale32 = am * rstd * kInvMaxSqrt2;
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) y[v] = xw[v] * factor;
      if ((lane & ((1 << tpg_log2) - 1)) == 0) {
        const int ng = D / (VEC << tpg_log2);
        const int64_t srow = isq ? ((int64_t)tok[i] * H + head[i]) * ng : (int64_t)tok[i] * ng;
        const int g = lane >> tpg_log2;
        if (E8M0)
          ((uint8_t*)(isq ? a.q_scale : a.kv_scale))[srow + g] = (uint8_t)e8;
        else
          ((float*)(isq ? a.q_scale : a.kv_scale))[srow + g] = scale32;
      }
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) y[v] = xw[v] * rstd;
    }
    if (is_rope) {
#pragma unroll
      for (int k = 0; k < VEC / 2; ++k) {
        const float c = bf16_at(cs[i].w, k), s = bf16_at(sn[i].w, k);
        const float e = y[2 * k], o = y[2 * k + 1];
        y[2 * k] = e * c - o * s;
        y[2 * k + 1] = e * s + o * c;
      }
    }
    const int64_t orow = isq ? ((int64_t)tok[i] * H + head[i]) * D : (int64_t)tok[i] * D;
    void* out = isq ? a.q_out : a.kv_out;
    if (QUANT) {
      uint8_t* o8 = (uint8_t*)out + orow + lane * VEC;
      if constexpr (VEC == 8) {
        const int w0 = pack2_fp8<true>(y[2], y[3], pack2_fp8<false>(y[0], y[1], 0));
        const int w1 = pack2_fp8<true>(y[6], y[7], pack2_fp8<false>(y[4], y[5], 0));
        *(u32x2*)o8 = u32x2{(uint32_t)w0, (uint32_t)w1};
      } else if constexpr (VEC == 4) {
        *(uint32_t*)o8 = (uint32_t)pack2_fp8<true>(y[2], y[3], pack2_fp8<false>(y[0], y[1], 0));
      } else {
        *(uint16_t*)o8 = (uint16_t)pack2_fp8<false>(y[0], y[1], 0);
      }
    } else {
      uint16_t* o16 = (uint16_t*)out + orow + lane * VEC;
      uint32_t w[VEC / 2];
#pragma unroll
      for (int k = 0; k < VEC / 2; ++k) w[k] = f32_to_bf16(y[2 * k]) | (f32_to_bf16(y[2 * k + 1]) << 16);
      if constexpr (VEC == 8)
        *(u32x4*)o16 = u32x4{w[0], w[1], w[2], w[3]};
      else if constexpr (VEC == 4)
        *(u32x2*)o16 = u32x2{w[0], w[1]};
      else
        *(uint32_t*)o16 = w[0];
    }
  }
}

template <int VEC, bool QUANT, bool E8M0>
hipError_t launch(const pa_qk_norm_rope_args& a, int tpg_log2, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((pa_qk_norm_rope_kernel<VEC, QUANT, E8M0>), dim3(grid), dim3(64 * kWavesPerGroup), 0, s, a,
                     tpg_log2);
  return hipGetLastError();
}

template <int VEC>
hipError_t dispatch(const pa_qk_norm_rope_args& a, int tpg_log2, unsigned grid, hipStream_t s) {
  if (!a.quant) return launch<VEC, false, false>(a, tpg_log2, grid, s);
  return a.scale_e8m0 ? launch<VEC, true, true>(a, tpg_log2, grid, s) : launch<VEC, true, false>(a, tpg_log2, grid, s);
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

}  // namespace

extern "C" int pa_fp8_qk_norm_rope_quant(const pa_qk_norm_rope_args* a, void* stream) {
  if (!a) return PA_ERR_NULL_ARG;
  if (a->abi_version != PA_FP8_ABI_VERSION) return PA_ERR_ABI;
  const int D = a->head_dim;
  if (D != 128 && D != 256 && D != 512) return PA_ERR_HEAD_SIZE;
  const int vec = D / 64;
  const int rd = a->rope_head_dim;
  if (a->num_tokens < 0 || a->num_q_heads < 0 || a->max_pos <= 0 || rd < 0 || rd > D || (rd & 1) || rd % vec)
    return PA_ERR_SHAPE;
  const int g = a->quant ? a->group_size : D;
  if (g <= 0 || D % g || g % vec) return PA_ERR_SHAPE;
  const int tpg = g / vec;
  if (tpg & (tpg - 1)) return PA_ERR_SHAPE;
  const int64_t rows = (int64_t)a->num_tokens * (a->num_q_heads + 1);
  if (rows >= ((int64_t)1 << 31)) return PA_ERR_SHAPE;
  if (rows == 0) return PA_OK;
  if (!a->kv || !a->kv_weight || (rd > 0 && (!a->cos_cache || !a->sin_cache)) || !a->positions || !a->kv_out ||
      (a->num_q_heads > 0 && (!a->q || !a->q_out)))
    return PA_ERR_NULL_ARG;
  if (a->quant && (!a->kv_scale || (a->num_q_heads > 0 && !a->q_scale))) return PA_ERR_NULL_ARG;
  // Vector accesses: VEC bf16 in, VEC (fp8) or 2 VEC bytes out per lane.
  const uintptr_t in_al = 2 * vec, out_al = a->quant ? vec : 2 * vec, half_al = vec;
  if (!aligned(a->q, in_al) || !aligned(a->kv, in_al) || !aligned(a->kv_weight, in_al) ||
      (a->q_weight && !aligned(a->q_weight, in_al)) || !aligned(a->q_out, out_al) || !aligned(a->kv_out, out_al) ||
      !aligned(a->cos_cache, half_al) || !aligned(a->sin_cache, half_al) || !aligned(a->positions, 8))
    return PA_ERR_ALIGN;
  if (a->stride_q_tok % vec || a->stride_kv_tok % vec || (rd / 2) % (vec / 2 > 0 ? vec / 2 : 1)) return PA_ERR_ALIGN;
  if (a->scale_e8m0 && !a->quant) return PA_ERR_DTYPE;
  const int64_t waves = (rows + kRowsPerWave - 1) / kRowsPerWave;
  const unsigned grid = (unsigned)((waves + kWavesPerGroup - 1) / kWavesPerGroup);
  const int lg = __builtin_ctz((unsigned)tpg);
  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  switch (vec) {
    case 2: err = dispatch<2>(*a, lg, grid, s); break;
    case 4: err = dispatch<4>(*a, lg, grid, s); break;
    default: err = dispatch<8>(*a, lg, grid, s); break;
  }
  return err == hipSuccess ? PA_OK : (int)err;
}
