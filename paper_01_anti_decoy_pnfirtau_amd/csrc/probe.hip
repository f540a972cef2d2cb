// Diagnostic, not on the attention path: how far the matrix (MFMA) and vector (VALU) pipes of
// a gfx950 SIMD overlap.  A register-only loop issues NM independent MFMAs (each into its own
// accumulator) and NV independent fp32 FMAs per iteration; the loop is timed with MFMAs only,
// with FMAs only, and with both.  Overlap = (t_mfma + t_valu - t_both) / min(t_mfma, t_valu):
// 0 when the pipes serialise, 1 when the shorter stream hides entirely under the longer.
// The attention kernels' backward interleaves the two the same way (S and dW MFMAs, then the
// power chain on the VALU, then the dK/dV or dQ MFMAs), so this bounds what scheduling can win.
#include "pnfx_common.h"

namespace pnfx {
namespace {

typedef __attribute__((ext_vector_type(16))) float f32x16;

template <int NM, int NV, bool BIG>
__global__ __launch_bounds__(512) void pipe_probe_kernel(float* out, int iters, float a, float b) {
  const int tid = threadIdx.x;
  bf16x8 x, y;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = (bf16)(a * (float)(tid + e));
    y[e] = (bf16)(b * (float)(tid - e));
  }
  constexpr int NS = NM > 0 ? NM : 1, NB = NM / 2 > 0 ? NM / 2 : 1;
  f32x4 c[NS];
  f32x16 C[NB];
#pragma unroll
  for (int m = 0; m < NS; ++m) c[m] = f32x4{0.f, 0.f, 0.f, (float)m};
#pragma unroll
  for (int m = 0; m < NB; ++m) {
#pragma unroll
    for (int i = 0; i < 16; ++i) C[m][i] = i == 3 ? (float)m : 0.f;
  }
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = a * (float)(i + tid);
  for (int it = 0; it < iters; ++it) {
    if constexpr (BIG) {  // equal FLOPs: NM/2 32x32x16 MFMAs
#pragma unroll
      for (int m = 0; m < NM / 2; ++m) C[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, C[m], 0, 0, 0);
    } else {
#pragma unroll
      for (int m = 0; m < NM; ++m) c[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, c[m], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j % 32] = __builtin_fmaf(v[j % 32], a, b);
  }
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < NS; ++m) s += c[m][0] + c[m][3];
#pragma unroll
  for (int m = 0; m < NB; ++m) s += C[m][0] + C[m][15];
#pragma unroll
  for (int i = 0; i < 32; ++i) s += v[i];
  out[blockIdx.x * blockDim.x + tid] = s;  // keeps every stream live
}

constexpr int kProbeBlocks = 256;  // one workgroup per CU

template <int NM, int NV, bool BIG>
int time_probe(float* out, int threads, int iters, hipStream_t st, float* ms) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    set_error("probe_pipe_overlap: hipEventCreate failed");
    return PNFX_ELAUNCH;
  }
  // warm-up launch, then the timed one
  hipLaunchKernelGGL((pipe_probe_kernel<NM, NV, BIG>), dim3(kProbeBlocks), dim3(threads), 0, st,
                     out, iters, 0.999f, 0.001f);
  (void)hipEventRecord(e0, st);
  hipLaunchKernelGGL((pipe_probe_kernel<NM, NV, BIG>), dim3(kProbeBlocks), dim3(threads), 0, st,
                     out, iters, 0.999f, 0.001f);
  (void)hipEventRecord(e1, st);
  const hipError_t e = hipEventSynchronize(e1);
  float t = 0.f;
  if (e == hipSuccess) (void)hipEventElapsedTime(&t, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) {
    set_error("probe_pipe_overlap: %s", hipGetErrorString(e));
    return PNFX_ELAUNCH;
  }
  *ms = t;
  return launch_status("pnfx_probe_pipe_overlap");
}

// MFMA only, VALU only, both: into ms[0..2].
template <int NM, int NV, bool BIG>
int probe_triple(float* out, int threads, int iters, hipStream_t st, float* ms) {
  int rc = time_probe<NM, 0, BIG>(out, threads, iters, st, ms + 0);
  if (!rc) rc = time_probe<0, NV, BIG>(out, threads, iters, st, ms + 1);
  if (!rc) rc = time_probe<NM, NV, BIG>(out, threads, iters, st, ms + 2);
  return rc;
}

template <bool BIG>
int probe_mix(int nm, int nv, float* out, int threads, int iters, hipStream_t st, float* ms) {
  if (nm == 8 && nv == 32) return probe_triple<8, 32, BIG>(out, threads, iters, st, ms);
  if (nm == 8 && nv == 64) return probe_triple<8, 64, BIG>(out, threads, iters, st, ms);
  if (nm == 16 && nv == 64) return probe_triple<16, 64, BIG>(out, threads, iters, st, ms);
  set_error("probe_pipe_overlap: (mfma, valu) per iteration must be (8, 32), (8, 64) or (16, 64)");
  return PNFX_EINVAL;
}

}  // namespace
}  // namespace pnfx

extern "C" int pnfx_probe_pipe_overlap(int waves_per_simd, int mfma_32x32, int mfma_per_iter,
                                       int valu_per_iter, int iters, float* out, float* ms,
                                       void* stream) {
  using namespace pnfx;
  PNFX_REQUIRE(waves_per_simd == 1 || waves_per_simd == 2,
               "probe_pipe_overlap: waves_per_simd must be 1 or 2");
  PNFX_REQUIRE(iters >= 1 && iters <= (1 << 20), "probe_pipe_overlap: iters in 1 .. 2^20");
  PNFX_REQUIRE(out != nullptr && ms != nullptr, "probe_pipe_overlap: null buffer");
  const int threads = 256 * waves_per_simd;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return mfma_32x32 ? probe_mix<true>(mfma_per_iter, valu_per_iter, out, threads, iters, st, ms)
                    : probe_mix<false>(mfma_per_iter, valu_per_iter, out, threads, iters, st, ms);
}
