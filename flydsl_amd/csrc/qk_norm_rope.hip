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
// head H being the KV row.  A wave owns kBatch consecutive rows and issues
// every load of them (rows, cos/sin; positions are scalar loads, one per
// token) before computing any; many short waves keep the GPU full.  The
// kernel is HBM-bound (per row 2D bytes in, D or 2D out) when its VALU work
// per row is small: lane l holds elements [l*VEC, l*VEC + VEC) of the row
// (VEC = D / 64), the row's square sum and a quant group's maximum are DPP /
// permlane reductions, and the per-channel weights are read once per wave.
// No LDS, no barriers.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_fp8.h"
#include "pa_check.h"

namespace {

constexpr int kBatch = 2;  // rows per load batch
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

// DPP lane exchanges (gfx9 encodings): quad_perm [1,0,3,2] and [2,3,0,1]
// pair lanes l ^ 1 and l ^ 2; row_half_mirror pairs lane i of an 8-lane
// half-row with 7 - i, row_mirror lane i of a 16-lane row with 15 - i.
// After the quad steps every lane holds its quad's value, so the mirrors
// complete reductions over 8 and 16 lanes; gfx950's permlane swaps then pair
// lanes l ^ 16 and l ^ 32.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swap16(float v, bool maxop) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return maxop ? fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) : __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32(float v, bool maxop) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return maxop ? fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) : __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v = swap16(v, false);
  return swap32(v, false);
}

// Maximum over the 2^lg adjacent lanes of a quant group (lg wave-uniform).
// v >= 0, so the float order is the unsigned order of the bits and the DPP
// steps fuse into v_max_u32_dpp.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float group_max(float f, int lg) {
  uint32_t v = __float_as_uint(f);
  if (lg >= 1) v = max(v, dpp_u<0xB1>(v));
  if (lg >= 2) v = max(v, dpp_u<0x4E>(v));
  if (lg >= 3) v = max(v, dpp_u<0x141>(v));
  if (lg >= 4) v = max(v, dpp_u<0x140>(v));
  f = __uint_as_float(v);
  if (lg >= 5) f = swap16(f, true);
  if (lg >= 6) f = swap32(f, true);
  return f;
}

// fp8 e4m3fn of a and b (round to nearest even) into bytes 2*hi, 2*hi + 1 of
// old; values in (-2^-8, 0) become +0 first, as the reference's store does.
template <bool HI>
__device__ __forceinline__ int pack2_fp8(float a, float b, int old) {
  a = (a < 0.0f && a > -0.00390625f) ? 0.0f : a;
  b = (b < 0.0f && b > -0.00390625f) ? 0.0f : b;
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, HI);
}

template <int VEC, bool QUANT, bool E8M0, bool QW>
__global__ __launch_bounds__(64 * kWavesPerGroup) void pa_qk_norm_rope_kernel(const pa_qk_norm_rope_args a,
                                                                             int tpg_log2, int rows_per_wave) {
  constexpr int D = 64 * VEC;
  constexpr int NH = VEC / 4 > 0 ? VEC / 4 : 1;  // dwords of a lane's cos (or sin) values
  const int lane = threadIdx.x & 63;
  // Wave-uniform (readfirstlane), so the row walk and the position reads
  // are scalar and never wait on the vector loads in flight.
  const uint32_t wave = blockIdx.x * kWavesPerGroup + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.num_q_heads;
  const uint32_t hp = (uint32_t)H + 1;
  const uint32_t rows = (uint32_t)a.num_tokens * hp;
  const uint32_t r0 = wave * (uint32_t)rows_per_wave;
  if (r0 >= rows) return;
  const uint32_t r1 = r0 + rows_per_wave < rows ? r0 + rows_per_wave : rows;
  const int rd = a.rope_head_dim;
  const int rope_lo = (D - rd) / VEC;  // first lane of the rotated part
  const bool is_rope = lane >= rope_lo;
  const int half_off = is_rope ? (lane - rope_lo) * (VEC / 2) : 0;  // this lane's first pair
  const uint16_t* cos_tab = (const uint16_t*)a.cos_cache;
  const uint16_t* sin_tab = (const uint16_t*)a.sin_cache;
  const int ng = D / (VEC << tpg_log2);  // quant groups per row
  const int grp = lane >> tpg_log2;      // this lane's quant group

  // Per-channel weights of this lane's elements (loaded once per wave).
  float kvw[VEC], qw[VEC];
  {
    const Raw<VEC> w = load_raw<VEC>((const uint16_t*)a.kv_weight + lane * VEC);
#pragma unroll
    for (int v = 0; v < VEC; ++v) kvw[v] = bf16_at(w.w, v);
  }
  if (QW) {
    const Raw<VEC> w = load_raw<VEC>((const uint16_t*)a.q_weight + lane * VEC);
#pragma unroll
    for (int v = 0; v < VEC; ++v) qw[v] = bf16_at(w.w, v);
  }

  // Row cursor (token lt, head lh) of the next row to load, with the
  // token's position (read once per token).
  uint32_t lt = r0 / hp, lh = r0 - lt * hp;
  int lpos = (int)(uint32_t)(uint64_t)a.positions[lt];
  struct Batch {
    Raw<VEC> x[kBatch];
    Half<VEC> cs[kBatch], sn[kBatch];
    uint32_t tok[kBatch], head[kBatch];
  };
  Batch b0;
  auto load_batch = [&](Batch& b, uint32_t rb) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      b.tok[i] = lt;
      b.head[i] = lh;
      if (rb + i < r1) {  // wave-uniform
        const uint16_t* src = lh < (uint32_t)H
                                  ? (const uint16_t*)a.q + (int64_t)lt * a.stride_q_tok + (int64_t)lh * D
                                  : (const uint16_t*)a.kv + (int64_t)lt * a.stride_kv_tok;
        b.x[i] = load_raw<VEC>(src + lane * VEC);
        // int64 position read as its low word; outside the table the
        // rotation reads zeros, like the reference's range-checked loads.
        // With a rotated part (rd > 0, wave-uniform; the tables may be empty
        // or NULL otherwise) every lane loads, in bounds -- row clamped into
        // the table, offset 0 outside the rotated lanes, rd / 2 >= VEC / 2 --
        // and rows outside the table keep zeros: a select, not a branch
        // around the loads.  (Lanes outside the rotated part select their
        // unrotated values after the rotation, which keeps signed zeros.)
        const bool inside = lpos >= 0 && lpos < a.max_pos;
        pa_note(rd > 0 && !inside, PA_VIOLATION_POSITION);
        if (rd > 0) {
          const int64_t crow = (int64_t)(inside ? lpos : 0) * (rd / 2) + half_off;
          b.cs[i] = load_half<VEC>(cos_tab + crow);
          b.sn[i] = load_half<VEC>(sin_tab + crow);
#pragma unroll
          for (int k = 0; k < NH; ++k) {
            b.cs[i].w[k] = inside ? b.cs[i].w[k] : 0u;
            b.sn[i].w[k] = inside ? b.sn[i].w[k] : 0u;
          }
        }
        if (++lh == hp) {
          lh = 0;
          if (++lt < (uint32_t)a.num_tokens) lpos = (int)(uint32_t)(uint64_t)a.positions[lt];
        }
      }
    }
  };

  auto compute_row = [&](const Raw<VEC>& xr, const Half<VEC>& cs, const Half<VEC>& sn, uint32_t t, uint32_t h) {
    const bool isq = h < (uint32_t)H;  // wave-uniform
    float xv[VEC], xw[VEC];
    float sq = 0.0f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      xv[v] = bf16_at(xr.w, v);
      sq += xv[v] * xv[v];
    }
    if (!isq) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xw[v] = xv[v] * kvw[v];
    } else if (QW) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xw[v] = xv[v] * qw[v];
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xw[v] = xv[v];
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
      if (E8M0) {
        const float post = am * rstd * kSqrt2;
        const uint32_t bits = (__float_as_uint(post) + 0x400000u) & 0xff800000u;
        int e = (int)(bits >> 23) - kE8m0Headroom;
        e = e < 0 ? 0 : (e > 255 ? 255 : e);
        factor = rstd * __uint_as_float((uint32_t)(254 - e) << 23);
        // every lane of the group stores the same byte
        const int64_t srow = isq ? ((int64_t)t * H + h) * ng : (int64_t)t * ng;
        ((uint8_t*)(isq ? a.q_scale : a.kv_scale))[srow + grp] = (uint8_t)e;
      } else {
        factor = kMaxOverSqrt2 * __builtin_amdgcn_rcpf(am);
        const int64_t srow = isq ? ((int64_t)t * H + h) * ng : (int64_t)t * ng;
        ((float*)(isq ? a.q_scale : a.kv_scale))[srow + grp] = am * rstd * kInvMaxSqrt2;
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) y[v] = xw[v] * factor;
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) y[v] = xw[v] * rstd;
    }
    if (rd > 0) {
#pragma unroll
      for (int k = 0; k < VEC / 2; ++k) {
        const float c = bf16_at(cs.w, k), s = bf16_at(sn.w, k);
        const float e = y[2 * k], o = y[2 * k + 1];
        const float ne = e * c - o * s, no = e * s + o * c;
        y[2 * k] = is_rope ? ne : e;
        y[2 * k + 1] = is_rope ? no : o;
      }
    }
    const int64_t orow = isq ? ((int64_t)t * H + h) * D : (int64_t)t * D;
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
  };

  auto compute_batch = [&](const Batch& b, uint32_t rb) {
    if (rb + kBatch <= r1) {  // a full batch: no per-row checks
#pragma unroll
      for (int i = 0; i < kBatch; ++i) compute_row(b.x[i], b.cs[i], b.sn[i], b.tok[i], b.head[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        if (rb + i < r1) compute_row(b.x[i], b.cs[i], b.sn[i], b.tok[i], b.head[i]);
    }
  };

  // One batch per wave: every load first, then the rows; many short waves
  // keep the GPU full.  Measured on the 8192-token, 16-head prefill
  // (kernel us): 1 row per wave 66, 2 rows 56, 4 rows 59, 8 rows 67; runs
  // of several double-buffered batches per wave 77-83 (fewer waves fit per
  // SIMD and the runs end unevenly).
  load_batch(b0, r0);
  compute_batch(b0, r0);
}

template <int VEC, bool QUANT, bool E8M0>
hipError_t launch(const pa_qk_norm_rope_args& a, int tpg_log2, int rpw, unsigned grid, hipStream_t s) {
  if (a.q_weight)
    hipLaunchKernelGGL((pa_qk_norm_rope_kernel<VEC, QUANT, E8M0, true>), dim3(grid), dim3(64 * kWavesPerGroup), 0, s,
                       a, tpg_log2, rpw);
  else
    hipLaunchKernelGGL((pa_qk_norm_rope_kernel<VEC, QUANT, E8M0, false>), dim3(grid), dim3(64 * kWavesPerGroup), 0,
                       s, a, tpg_log2, rpw);
  return hipGetLastError();
}

template <int VEC>
hipError_t dispatch(const pa_qk_norm_rope_args& a, int tpg_log2, int rpw, unsigned grid, hipStream_t s) {
  if (!a.quant) return launch<VEC, false, false>(a, tpg_log2, rpw, grid, s);
  return a.scale_e8m0 ? launch<VEC, true, true>(a, tpg_log2, rpw, grid, s)
                      : launch<VEC, true, false>(a, tpg_log2, rpw, grid, s);
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

}  // namespace

PA_CHECK_DEFINE_TAKE(pa_violations_qk_norm_rope)

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
  const int64_t rpw = kBatch;  // rows per wave
  const int64_t waves = (rows + rpw - 1) / rpw;
  const unsigned grid = (unsigned)((waves + kWavesPerGroup - 1) / kWavesPerGroup);
  const int lg = __builtin_ctz((unsigned)tpg);
  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  switch (vec) {
    case 2: err = dispatch<2>(*a, lg, (int)rpw, grid, s); break;
    case 4: err = dispatch<4>(*a, lg, (int)rpw, grid, s); break;
    default: err = dispatch<8>(*a, lg, (int)rpw, grid, s); break;
  }
  return err == hipSuccess ? PA_OK : (int)err;
}
