#include <hip/hip_runtime.h>
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i8v __attribute__((ext_vector_type(8)));
extern "C" __global__ void p0(const i8v* a, const i8v* b, f4* out) {
  int l = threadIdx.x;
  f4 acc = {0,0,0,0};
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[l], b[l], acc, 0, 0, 0, 0, 0, 0);
  out[l] = acc;
}
extern "C" __global__ void p127(const i8v* a, const i8v* b, f4* out) {
  int l = threadIdx.x;
  f4 acc = {0,0,0,0};
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[l], b[l], acc, 0, 0, 0, 127, 0, 127);
  out[l] = acc;
}
extern "C" __global__ void p2(float* out) {
  int l = threadIdx.x;
  float v = out[l];
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  out[l] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
