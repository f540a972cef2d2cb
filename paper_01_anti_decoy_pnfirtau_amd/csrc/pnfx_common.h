// Shared device/host helpers for the pn_fir_tau HIP library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pnfx.h"

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace pnfx {

// ---------------------------------------------------------------- host-side error state
void set_error(const char* fmt, ...);
int launch_status(const char* what);  // checks hipGetLastError after a launch

#define PNFX_REQUIRE(cond, ...)            \
  do {                                     \
    if (!(cond)) {                         \
      ::pnfx::set_error(__VA_ARGS__);      \
      return PNFX_EINVAL;                  \
    }                                      \
  } while (0)

// ---------------------------------------------------------------- element conversion
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }  // RNE

// ---------------------------------------------------------------- wave helpers (wave64)
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------- MFMA wrappers
// v_mfma_f32_16x16x32_bf16: lane l holds A[row l%16][k-slots of group l/16],
// B[k-slots of group l/16][col l%16]; D[row 4*(l/16)+i][col l%16], i = 0..3.
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 zero_bf16x8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
  return z;
}

__device__ __forceinline__ bf16x8 pack8(float a0, float a1, float a2, float a3, float b0, float b1,
                                        float b2, float b3) {
  bf16x8 v;
  v[0] = (bf16)a0; v[1] = (bf16)a1; v[2] = (bf16)a2; v[3] = (bf16)a3;
  v[4] = (bf16)b0; v[5] = (bf16)b1; v[6] = (bf16)b2; v[7] = (bf16)b3;
  return v;
}

template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) { return *p; }

}  // namespace pnfx
