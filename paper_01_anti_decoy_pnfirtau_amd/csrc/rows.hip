// Row-fused rectified power-norm score -> weight (the materialised-score path of pn_fir_tau).
//
// One wave64 per score row; any row length.  Forward makes two passes over the row:
// pass 1 accumulates the row peak and the power mass (lane-local, then a wave butterfly),
// pass 2 re-reads the row (L1/L2 resident), counts peak ties and writes the weights.
// Backward mirrors it: pass 1 forms <dW, w_hat>, pass 2 writes dScores and the row's
// tau partial.
//
// Semantics follow src/triton_pnfirtau.py:141-212 (forward) and :214-303 (backward):
// s = fma(raw, scale, -tau); u = relu(s) on valid columns (col <= t when causal,
// t = row % N); pw = u^p; Z = sum pw + 1e-12; gate = peak/(peak + gamma);
// w = pw * (gate / Z); silent rows (peak <= 0) short-circuit to zeros.
#include "pnfx_common.h"

namespace pnfx {
namespace {

struct RowsArgs {
  const void* raw;
  int64_t raw_rs;
  const void* dw;
  int64_t dw_rs;
  void* out;  // w (forward) or d_raw (backward)
  int64_t out_rs;
  float* M;
  float* Z;
  int32_t* Nmax;
  float* dtau_rows;
  int64_t R, N;
  const float* tau;
  float scale, p, gamma;
  int has_gamma, causal;
};

template <int PMODE>
__device__ __forceinline__ float pow_p(float u, float p) {
  if (PMODE == 10) {
    const float u2 = u * u;
    const float u4 = u2 * u2;
    return u4 * u4 * u2;
  } else if (PMODE == 2) {
    return u * u;
  } else {
    return u > 0.0f ? expf(logf(u) * p) : 0.0f;
  }
}

template <typename T, int PMODE>
__global__ __launch_bounds__(256) void pn_rows_fwd_kernel(RowsArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= a.R) return;
  const int64_t t = r % a.N;
  const int64_t limit = a.causal ? t + 1 : a.N;
  const T* row = reinterpret_cast<const T*>(a.raw) + r * a.raw_rs;
  T* wrow = reinterpret_cast<T*>(a.out) + r * a.out_rs;
  const float ntau = -a.tau[0];

  float peak = 0.0f, mass = 0.0f;
  for (int64_t c = lane; c < limit; c += 64) {
    const float s = __builtin_fmaf(to_f32(row[c]), a.scale, ntau);
    const float u = s > 0.0f ? s : 0.0f;
    peak = fmaxf(peak, u);
    mass += pow_p<PMODE>(u, a.p);
  }
  peak = wave_max(peak);
  mass = wave_sum(mass);

  if (peak <= 0.0f) {
    for (int64_t c = lane; c < a.N; c += 64) wrow[c] = from_f32<T>(0.0f);
    if (lane == 0) {
      a.M[r] = 0.0f;
      a.Z[r] = 1e-12f;
      a.Nmax[r] = 0;
    }
    return;
  }
  const float z = mass + 1e-12f;
  const float gate = a.has_gamma ? peak / (peak + a.gamma) : 1.0f;
  const float coef = gate / z;
  int cnt = 0;
  for (int64_t c = lane; c < a.N; c += 64) {
    float w = 0.0f;
    if (c < limit) {
      const float s = __builtin_fmaf(to_f32(row[c]), a.scale, ntau);
      const float u = s > 0.0f ? s : 0.0f;
      w = pow_p<PMODE>(u, a.p) * coef;
      cnt += (u == peak) ? 1 : 0;
    }
    wrow[c] = from_f32<T>(w);
  }
  cnt = wave_sum_i(cnt);
  if (lane == 0) {
    a.M[r] = peak;
    a.Z[r] = z;
    a.Nmax[r] = cnt;
  }
}

template <typename T, int PMODE>
__global__ __launch_bounds__(256) void pn_rows_bwd_kernel(RowsArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= a.R) return;
  T* drow = reinterpret_cast<T*>(a.out) + r * a.out_rs;
  const float peak = a.M[r];
  if (peak <= 0.0f) {
    for (int64_t c = lane; c < a.N; c += 64) drow[c] = from_f32<T>(0.0f);
    if (lane == 0) a.dtau_rows[r] = 0.0f;
    return;
  }
  const int64_t t = r % a.N;
  const int64_t limit = a.causal ? t + 1 : a.N;
  const T* row = reinterpret_cast<const T*>(a.raw) + r * a.raw_rs;
  const T* dyrow = reinterpret_cast<const T*>(a.dw) + r * a.dw_rs;
  const float ntau = -a.tau[0];
  const float z = a.Z[r];
  const float nmax = (float)a.Nmax[r];

  float dot = 0.0f;
  for (int64_t c = lane; c < limit; c += 64) {
    const float s = __builtin_fmaf(to_f32(row[c]), a.scale, ntau);
    const float u = s > 0.0f ? s : 0.0f;
    dot += to_f32(dyrow[c]) * (pow_p<PMODE>(u, a.p) / z);
  }
  dot = wave_sum(dot);

  float gate = 1.0f, gterm = 0.0f;
  if (a.has_gamma) {
    gate = peak / (peak + a.gamma);
    const float dgate = a.gamma / ((peak + a.gamma) * (peak + a.gamma));
    gterm = dot * dgate / nmax;
  }
  const float coef = a.p * gate / z;
  float acc = 0.0f;
  for (int64_t c = lane; c < a.N; c += 64) {
    float du = 0.0f;
    if (c < limit) {
      const float s = __builtin_fmaf(to_f32(row[c]), a.scale, ntau);
      const float u = s > 0.0f ? s : 0.0f;
      float upm1;
      if (PMODE == 10) {
        const float u2 = u * u;
        const float u4 = u2 * u2;
        upm1 = u4 * u4 * u;
      } else if (PMODE == 2) {
        upm1 = u;
      } else {
        upm1 = u > 0.0f ? expf(logf(u) * (a.p - 1.0f)) : 0.0f;
      }
      const float dy = to_f32(dyrow[c]);
      const float du_norm = coef * upm1 * (dy - dot);
      const float du_gate = (a.has_gamma && u == peak) ? gterm : 0.0f;
      du = u > 0.0f ? du_norm + du_gate : 0.0f;
      acc += du;
    }
    drow[c] = from_f32<T>(du * a.scale);
  }
  acc = wave_sum(acc);
  if (lane == 0) a.dtau_rows[r] = -acc;
}

template <typename T, bool BWD>
int launch_rows(const RowsArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.R + 3) / 4)), block(256);
  const int pm = a.p == 10.0f ? 10 : (a.p == 2.0f ? 2 : 0);
  if (BWD) {
    if (pm == 10) hipLaunchKernelGGL((pn_rows_bwd_kernel<T, 10>), grid, block, 0, st, a);
    else if (pm == 2) hipLaunchKernelGGL((pn_rows_bwd_kernel<T, 2>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((pn_rows_bwd_kernel<T, 0>), grid, block, 0, st, a);
  } else {
    if (pm == 10) hipLaunchKernelGGL((pn_rows_fwd_kernel<T, 10>), grid, block, 0, st, a);
    else if (pm == 2) hipLaunchKernelGGL((pn_rows_fwd_kernel<T, 2>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((pn_rows_fwd_kernel<T, 0>), grid, block, 0, st, a);
  }
  return launch_status(BWD ? "pnfx_pn_rows_bwd" : "pnfx_pn_rows_fwd");
}

template <bool BWD>
int rows_dispatch(const RowsArgs& a, int dtype, hipStream_t st) {
  if (a.R == 0 || a.N == 0) return PNFX_OK;
  if (dtype == PNFX_BF16) return launch_rows<bf16, BWD>(a, st);
  if (dtype == PNFX_F32) return launch_rows<float, BWD>(a, st);
  set_error("pn_rows: unsupported dtype %d", dtype);
  return PNFX_EUNSUPPORTED;
}

}  // namespace
}  // namespace pnfx

extern "C" int pnfx_pn_rows_fwd(const void* raw, int64_t raw_rs, void* w, int64_t w_rs, float* M,
                                float* Z, int32_t* Nmax, int64_t R, int64_t N, const float* tau,
                                float scale, float p, float gamma, int has_gamma, int causal,
                                int dtype, void* stream) {
  PNFX_REQUIRE(raw && w && M && Z && Nmax && tau, "pn_rows_fwd: null pointer");
  PNFX_REQUIRE(R >= 0 && N >= 0, "pn_rows_fwd: bad shape");
  pnfx::RowsArgs a{raw, raw_rs, nullptr, 0, w, w_rs, M, Z, Nmax, nullptr, R, N, tau, scale, p,
                   gamma, has_gamma, causal};
  return pnfx::rows_dispatch<false>(a, dtype, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pnfx_pn_rows_bwd(const void* dw, int64_t dw_rs, const void* raw, int64_t raw_rs,
                                const float* M, const float* Z, const int32_t* Nmax, void* draw,
                                int64_t draw_rs, float* dtau_rows, int64_t R, int64_t N,
                                const float* tau, float scale, float p, float gamma, int has_gamma,
                                int causal, int dtype, void* stream) {
  PNFX_REQUIRE(dw && raw && M && Z && Nmax && draw && dtau_rows && tau,
               "pn_rows_bwd: null pointer");
  PNFX_REQUIRE(R >= 0 && N >= 0, "pn_rows_bwd: bad shape");
  pnfx::RowsArgs a{raw, raw_rs, dw, dw_rs, draw, draw_rs, const_cast<float*>(M),
                   const_cast<float*>(Z), const_cast<int32_t*>(Nmax), dtau_rows, R, N, tau,
                   scale, p, gamma, has_gamma, causal};
  return pnfx::rows_dispatch<true>(a, dtype, reinterpret_cast<hipStream_t>(stream));
}
