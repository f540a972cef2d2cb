// Row-fused rectified power-norm score -> weight (the materialised-score path of pn_fir_tau).
//
// One wave64 per score row; any row length.  Forward makes two passes over the row:
// pass 1 accumulates the row peak and the power mass (lane-local, then a wave butterfly),
// pass 2 counts peak ties and writes the weights from the register-held scores (re-reading
// only what did not fit).  Backward mirrors it: pass 1 forms <dW, w_hat>, pass 2 writes
// dScores and the row's tau partial.
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

// V consecutive elements of a row, converted to fp32: V = 16 bytes / element size when the
// rows are 16-byte aligned and N is a multiple of V (one dwordx4 access per lane), else 1.
template <typename T, int V>
struct RowIO;
template <typename T>
struct RowIO<T, 1> {
  __device__ static void load(const T* p, float (&x)[1]) { x[0] = to_f32(p[0]); }
  __device__ static void store(T* p, const float (&x)[1]) { p[0] = from_f32<T>(x[0]); }
};
template <>
struct RowIO<bf16, 8> {
  __device__ static void load(const bf16* p, float (&x)[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = __uint_as_float(w[j] << 16);
      x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ static void store(bf16* p, const float (&x)[8]) {
    bf16x8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (bf16)x[j];
    *reinterpret_cast<bf16x8*>(p) = v;
  }
};
template <>
struct RowIO<float, 4> {
  __device__ static void load(const float* p, float (&x)[4]) {
    const f32x4 q = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = q[j];
  }
  __device__ static void store(float* p, const float (&x)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  }
};

// Lane l owns columns [l*V, l*V + V) of every 64*V-column chunk.  The first CH chunks of a
// row stay in registers between the two passes (u, and dW in the backward); columns beyond
// them are re-read in pass 2.  CH = 1 for rows of one chunk (512 bf16 / 256 fp32 entries),
// which keeps the register count low enough for 8 waves per SIMD -- the bytes in flight
// that a one-load-per-lane row needs to approach HBM bandwidth.
template <typename T, int PMODE, int V, int CH>
__global__ __launch_bounds__(256, CH == 1 ? 8 : 2) void pn_rows_fwd_kernel(RowsArgs a) {
  using IO = RowIO<T, V>;
  constexpr int64_t SPAN = 64 * V;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= a.R) return;
  const int64_t t = r % a.N;
  const int64_t limit = a.causal ? t + 1 : a.N;
  const T* row = reinterpret_cast<const T*>(a.raw) + r * a.raw_rs;
  T* wrow = reinterpret_cast<T*>(a.out) + r * a.out_rs;
  const float ntau = -a.tau[0];
  const int64_t cl = (int64_t)lane * V;

  float u[CH][V];
  float peak = 0.0f, mass = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t c0 = k * SPAN + cl;
    float x[V] = {};
    if (c0 < limit) IO::load(row + c0, x);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float s = __builtin_fmaf(x[j], a.scale, ntau);
      u[k][j] = (c0 + j < limit && s > 0.0f) ? s : 0.0f;
      peak = fmaxf(peak, u[k][j]);
      mass += pow_p<PMODE>(u[k][j], a.p);
    }
  }
  for (int64_t c0 = CH * SPAN + cl; c0 - cl < limit; c0 += SPAN) {
    if (c0 >= limit) continue;
    float x[V];
    IO::load(row + c0, x);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float s = __builtin_fmaf(x[j], a.scale, ntau);
      const float uj = (c0 + j < limit && s > 0.0f) ? s : 0.0f;
      peak = fmaxf(peak, uj);
      mass += pow_p<PMODE>(uj, a.p);
    }
  }
  peak = wave_max(peak);
  mass = wave_sum(mass);

  if (peak <= 0.0f) {
    const float zero[V] = {};
    for (int64_t c0 = cl; c0 < a.N; c0 += SPAN) IO::store(wrow + c0, zero);
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
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t c0 = k * SPAN + cl;
    if (c0 < a.N) {
      float w[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        w[j] = pow_p<PMODE>(u[k][j], a.p) * coef;
        cnt += (u[k][j] == peak) ? 1 : 0;
      }
      IO::store(wrow + c0, w);
    }
  }
  for (int64_t c0 = CH * SPAN + cl; c0 - cl < a.N; c0 += SPAN) {
    if (c0 >= a.N) continue;
    float x[V] = {}, w[V];
    if (c0 < limit) IO::load(row + c0, x);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float s = __builtin_fmaf(x[j], a.scale, ntau);
      const float uj = (c0 + j < limit && s > 0.0f) ? s : 0.0f;
      w[j] = pow_p<PMODE>(uj, a.p) * coef;
      cnt += (uj == peak) ? 1 : 0;
    }
    IO::store(wrow + c0, w);
  }
  cnt = wave_sum_i(cnt);
  if (lane == 0) {
    a.M[r] = peak;
    a.Z[r] = z;
    a.Nmax[r] = cnt;
  }
}

template <int PMODE>
__device__ __forceinline__ float pow_pm1(float u, float p) {
  if (PMODE == 10) {
    const float u2 = u * u;
    const float u4 = u2 * u2;
    return u4 * u4 * u;
  } else if (PMODE == 2) {
    return u;
  } else {
    return u > 0.0f ? expf(logf(u) * (p - 1.0f)) : 0.0f;
  }
}

template <typename T, int PMODE, int V, int CH>
__global__ __launch_bounds__(256, CH == 1 ? (sizeof(T) == 2 ? 6 : 8) : 2) void pn_rows_bwd_kernel(RowsArgs a) {
  using IO = RowIO<T, V>;
  constexpr int64_t SPAN = 64 * V;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= a.R) return;
  T* drow = reinterpret_cast<T*>(a.out) + r * a.out_rs;
  const int64_t cl = (int64_t)lane * V;
  const float peak = a.M[r];
  if (peak <= 0.0f) {
    const float zero[V] = {};
    for (int64_t c0 = cl; c0 < a.N; c0 += SPAN) IO::store(drow + c0, zero);
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

  float u[CH][V], dy[CH][V];
  float dot = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t c0 = k * SPAN + cl;
    float x[V] = {}, g[V] = {};
    if (c0 < limit) {
      IO::load(row + c0, x);
      IO::load(dyrow + c0, g);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float s = __builtin_fmaf(x[j], a.scale, ntau);
      u[k][j] = (c0 + j < limit && s > 0.0f) ? s : 0.0f;
      dy[k][j] = g[j];
      dot += g[j] * (pow_p<PMODE>(u[k][j], a.p) / z);
    }
  }
  for (int64_t c0 = CH * SPAN + cl; c0 - cl < limit; c0 += SPAN) {
    if (c0 >= limit) continue;
    float x[V], g[V];
    IO::load(row + c0, x);
    IO::load(dyrow + c0, g);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float s = __builtin_fmaf(x[j], a.scale, ntau);
      const float uj = (c0 + j < limit && s > 0.0f) ? s : 0.0f;
      dot += g[j] * (pow_p<PMODE>(uj, a.p) / z);
    }
  }
  dot = wave_sum(dot);

  float gate = 1.0f, gterm = 0.0f;
  if (a.has_gamma) {
    gate = peak / (peak + a.gamma);
    const float dgate = a.gamma / ((peak + a.gamma) * (peak + a.gamma));
    gterm = dot * dgate / nmax;
  }
  const float coef = a.p * gate / z;
  // du for one entry; u == 0 covers both masked columns and the relu's dead side.
  auto du_of = [&](float uj, float g) {
    const float du_norm = coef * pow_pm1<PMODE>(uj, a.p) * (g - dot);
    const float du_gate = (a.has_gamma && uj == peak) ? gterm : 0.0f;
    return uj > 0.0f ? du_norm + du_gate : 0.0f;
  };
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int64_t c0 = k * SPAN + cl;
    if (c0 < a.N) {
      float d[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float du = du_of(u[k][j], dy[k][j]);
        acc += du;
        d[j] = du * a.scale;
      }
      IO::store(drow + c0, d);
    }
  }
  for (int64_t c0 = CH * SPAN + cl; c0 - cl < a.N; c0 += SPAN) {
    if (c0 >= a.N) continue;
    float x[V] = {}, g[V] = {}, d[V];
    if (c0 < limit) {
      IO::load(row + c0, x);
      IO::load(dyrow + c0, g);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float s = __builtin_fmaf(x[j], a.scale, ntau);
      const float uj = (c0 + j < limit && s > 0.0f) ? s : 0.0f;
      const float du = du_of(uj, g[j]);
      acc += du;
      d[j] = du * a.scale;
    }
    IO::store(drow + c0, d);
  }
  acc = wave_sum(acc);
  if (lane == 0) a.dtau_rows[r] = -acc;
}

template <typename T, int V, int CH, bool BWD>
void launch_rows_v(const RowsArgs& a, int pm, dim3 grid, dim3 block, hipStream_t st) {
  if (BWD) {
    if (pm == 10) hipLaunchKernelGGL((pn_rows_bwd_kernel<T, 10, V, CH>), grid, block, 0, st, a);
    else if (pm == 2) hipLaunchKernelGGL((pn_rows_bwd_kernel<T, 2, V, CH>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((pn_rows_bwd_kernel<T, 0, V, CH>), grid, block, 0, st, a);
  } else {
    if (pm == 10) hipLaunchKernelGGL((pn_rows_fwd_kernel<T, 10, V, CH>), grid, block, 0, st, a);
    else if (pm == 2) hipLaunchKernelGGL((pn_rows_fwd_kernel<T, 2, V, CH>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((pn_rows_fwd_kernel<T, 0, V, CH>), grid, block, 0, st, a);
  }
}

template <typename T, bool BWD>
int launch_rows(const RowsArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.R + 3) / 4)), block(256);
  const int pm = a.p == 10.0f ? 10 : (a.p == 2.0f ? 2 : 0);
  constexpr int V = 16 / (int)sizeof(T);
  auto aligned = [](const void* ptr, int64_t rs) {
    return ((uintptr_t)ptr % 16 == 0) && rs % V == 0;
  };
  const bool vec = a.N % V == 0 && aligned(a.raw, a.raw_rs) && aligned(a.out, a.out_rs) &&
                   (!BWD || aligned(a.dw, a.dw_rs));
  if (vec && a.N <= 64 * V) launch_rows_v<T, V, 1, BWD>(a, pm, grid, block, st);
  else if (vec) launch_rows_v<T, V, 4, BWD>(a, pm, grid, block, st);
  else launch_rows_v<T, 1, 8, BWD>(a, pm, grid, block, st);
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
