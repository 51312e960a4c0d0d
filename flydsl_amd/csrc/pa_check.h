// Checked builds of the library (compiled with -DPA_FP8_CHECKED).
//
// The kernels clamp every index they read from caller data into its range
// before using it as an address -- page indices from block_tables and
// kv_page_indices, MLA work records, rope positions, cache slots -- so a bad
// value never leaves the buffers it points into.  A release build clamps in
// silence.  A checked build also records each clamped value as a violation
// bit in a device word of its translation unit (relaxed device-scope atomic
// OR; nothing traps or waits), and pa_fp8_debug_violations() reads and clears
// the bits of every unit.  Release builds compile pa_note() to nothing, so
// their code is unchanged.
#pragma once

#include <hip/hip_runtime.h>

#include "pa_fp8.h"

#ifdef PA_FP8_CHECKED

// The violation bits of this translation unit (each unit its own word).
static __device__ unsigned int pa_violation_bits;

__device__ __forceinline__ void pa_note(bool bad, unsigned int bit) {
  if (bad) __hip_atomic_fetch_or(&pa_violation_bits, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Host side: ORs the unit's bits since the last call (PA_VIOLATION_*) into
// *bits and clears them; returns 0 or the HIP error of the copy.
// Synchronises the current device.
#define PA_CHECK_DEFINE_TAKE(fn)                                                            \
  int fn(unsigned int* bits) {                                                              \
    unsigned int b = 0, zero = 0;                                                           \
    hipError_t e = hipDeviceSynchronize();                                                  \
    if (e == hipSuccess) e = hipMemcpyFromSymbol(&b, HIP_SYMBOL(pa_violation_bits), 4);     \
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(pa_violation_bits), &zero, 4);     \
    if (e == hipSuccess) *bits |= b;                                                        \
    return (int)e;                                                                          \
  }

#else

__device__ __forceinline__ void pa_note(bool, unsigned int) {}

#define PA_CHECK_DEFINE_TAKE(fn) \
  int fn(unsigned int*) { return 0; }

#endif

// The per-unit readers (one per source file of the library).
int pa_violations_paged(unsigned int* bits);
int pa_violations_mla(unsigned int* bits);
int pa_violations_rope_cache(unsigned int* bits);
int pa_violations_qk_norm_rope(unsigned int* bits);
