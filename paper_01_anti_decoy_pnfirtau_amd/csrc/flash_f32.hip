// Flash pn_fir_tau attention for fp32 tensors (the reference's TF32-off parity path).
//
// Scalar fp32 FMA kernels: one lane per query row (forward, dQ) or per key (dK/dV), 64-row
// tiles of the other operand staged in LDS and read as broadcasts.  Dot products are a
// sequential fma chain over the head dimension in the same order in every kernel, so the
// backward reproduces the forward's scores bit for bit (the u == peak tie test relies on
// it).  Same math, statistics, tile mask and workspace layout as the bf16 MFMA kernels; the
// dQ kernel counts the peak ties itself with one extra sweep of the scores.
#include "flash.h"

namespace pnfx {
namespace {

constexpr int TB = 64;

__device__ __forceinline__ float pow10f_(float u) {
  const float u2 = u * u;
  const float u4 = u2 * u2;
  return u4 * u4 * u2;
}

template <int D>
__device__ __forceinline__ void stage(float (*dst)[D], const float* src, int64_t sn, int row0, int N) {
  for (int idx = threadIdx.x; idx < TB * D; idx += TB) {
    const int r = idx / D, d = idx % D;
    dst[r][d] = (row0 + r < N) ? src[(int64_t)(row0 + r) * sn + d] : 0.f;
  }
}

template <int D, bool CAUSAL, bool HAS_GAMMA>
__global__ __launch_bounds__(64) void f32_fwd_kernel(FwdParams p) {
  __shared__ float Ks[TB][D], Vs[TB][D];
  const int lane = threadIdx.x, N = p.N;
  const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
  const int row = blockIdx.x * TB + lane;
  const bool has = row < N;
  const float* Q = static_cast<const float*>(p.q) + b * p.qsb + h * p.qsh;
  const float* K = static_cast<const float*>(p.k) + b * p.ksb + h * p.ksh;
  const float* V = static_cast<const float*>(p.v) + b * p.vsb + h * p.vsh;
  const float ntau = -p.tau[0];
  float q[D], acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = has ? Q[(int64_t)row * p.qsn + d] : 0.f;
    acc[d] = 0.f;
  }
  float m = 0.f, mass = 0.f;
  int cnt = 0;
  const int kv_end = CAUSAL ? min((int)(blockIdx.x + 1) * TB, N) : N;
  const int ntiles = (kv_end + TB - 1) / TB;
  const int g0 = 2 * blockIdx.x;
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * TB;
    __syncthreads();
    stage<D>(Ks, K, p.ksn, n0, N);
    stage<D>(Vs, V, p.vsn, n0, N);
    __syncthreads();
    bool act = false;
    const int jmax = min(TB, N - n0);
    for (int j = 0; j < jmax; ++j) {
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) s = __builtin_fmaf(q[d], Ks[j][d], s);
      const float sv = __builtin_fmaf(s, p.scale, ntau);
      float u = sv > 0.f ? sv : 0.f;
      if (!has || (CAUSAL && n0 + j > row)) u = 0.f;
      act |= u > 0.f;
      if (u > m) {
        m = u;
        cnt = 1;
      } else if (u == m) {
        ++cnt;
      }
      const float pw = pow10f_(u);
      mass += pw;
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(pw, Vs[j][d], acc[d]);
    }
    const uint64_t bal = __ballot(act);
    if (p.mask && lane == 0) {
      if (g0 < p.nq32) p.mask[((int64_t)bh * p.nq32 + g0) * p.nk64 + t] = (bal & 0xffffffffull) ? 1 : 0;
      if (g0 + 1 < p.nq32) p.mask[((int64_t)bh * p.nq32 + g0 + 1) * p.nk64 + t] = (bal >> 32) ? 1 : 0;
    }
  }
  if (p.mask && lane == 0) {
    for (int t = ntiles; t < p.nk64; ++t) {
      if (g0 < p.nq32) p.mask[((int64_t)bh * p.nq32 + g0) * p.nk64 + t] = 0;
      if (g0 + 1 < p.nq32) p.mask[((int64_t)bh * p.nq32 + g0 + 1) * p.nk64 + t] = 0;
    }
  }
  if (!has) return;
  const float gate = m > 0.f ? (HAS_GAMMA ? m / (m + p.gamma) : 1.f) : 0.f;
  const float z = mass + 1e-12f;
  const float so = gate / z;
  float* O = static_cast<float*>(p.o) + b * p.osb + h * p.osh + (int64_t)row * p.osn;
#pragma unroll
  for (int d = 0; d < D; ++d) O[d] = acc[d] * so;
  const int64_t si = (int64_t)bh * N + row;
  p.M[si] = m;
  p.Z[si] = z;
  if (p.Nmax) p.Nmax[si] = m > 0.f ? cnt : 0;
}

template <int D, bool HAS_GAMMA>
__global__ __launch_bounds__(256) void f32_bwd_pre_kernel(BwdParams p) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= (int64_t)p.B * p.H * p.N) return;
  const int64_t bh = row / p.N, i = row % p.N, b = bh / p.H, h = bh % p.H;
  const float* O = static_cast<const float*>(p.o) + b * p.osb + h * p.osh + i * p.osn;
  const float* dO = static_cast<const float*>(p.dout) + b * p.dosb + h * p.dosh + i * p.dosn;
  float dot = 0.f;
  for (int d = 0; d < D; ++d) dot = __builtin_fmaf(dO[d], O[d], dot);
  const float M = p.M[row], Z = p.Z[row];
  const float g = M > 0.f ? (HAS_GAMMA ? M / (M + p.gamma) : 1.f) : 0.f;
  const float Dv = g > 0.f ? dot / g : 0.f;
  float Gu = 0.f;  // the whole row's peak-tie du; the dQ kernel divides it by Nmax
  if (HAS_GAMMA && M > 0.f) Gu = Dv * (p.gamma / ((M + p.gamma) * (M + p.gamma)));
  float* rc = p.rc + 8 * row;
  rc[0] = M;
  rc[1] = g / Z;
  rc[2] = 10.f * g / Z * p.scale;  // dS = du scale, for the dK/dV kernel
  rc[3] = Dv;
  rc[4] = Gu * p.scale;  // the dQ kernel replaces it by its share G/Nmax
  rc[5] = 10.f * g / Z;  // du, for the dQ kernel (its sum is the tau gradient)
  rc[6] = Gu;
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(64) void f32_bwd_dq_kernel(BwdParams p) {
  __shared__ float Ks[TB][D], Vs[TB][D];
  const int lane = threadIdx.x, N = p.N;
  const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
  const int row = blockIdx.x * TB + lane;
  const bool has = row < N;
  const float* Q = static_cast<const float*>(p.q) + b * p.qsb + h * p.qsh;
  const float* K = static_cast<const float*>(p.k) + b * p.ksb + h * p.ksh;
  const float* V = static_cast<const float*>(p.v) + b * p.vsb + h * p.vsh;
  const float* dO = static_cast<const float*>(p.dout) + b * p.dosb + h * p.dosh;
  const float ntau = -p.tau[0];
  float q[D], gdo[D], dq[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = has ? Q[(int64_t)row * p.qsn + d] : 0.f;
    gdo[d] = has ? dO[(int64_t)row * p.dosn + d] : 0.f;
    dq[d] = 0.f;
  }
  float* rcp = p.rc + 8 * ((int64_t)bh * N + (has ? row : 0));
  const float rM = rcp[0], rcoef = rcp[5], rD = rcp[3];
  const int kv_end = CAUSAL ? min((int)(blockIdx.x + 1) * TB, N) : N;
  const int ntiles = (kv_end + TB - 1) / TB;
  // Count the keys tied at the peak (the forward leaves Nmax to the backward): one sweep of
  // the scores, computed exactly as below, so G/Nmax is known before dQ accumulates.
  int nmax = 0;
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * TB;
    __syncthreads();
    stage<D>(Ks, K, p.ksn, n0, N);
    __syncthreads();
    if (!has || rM <= 0.f) continue;
    const int jmax = min(TB, N - n0);
    for (int j = 0; j < jmax; ++j) {
      if (CAUSAL && n0 + j > row) break;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) s = __builtin_fmaf(q[d], Ks[j][d], s);
      const float sv = __builtin_fmaf(s, p.scale, ntau);
      nmax += (sv > 0.f ? sv : 0.f) == rM ? 1 : 0;
    }
  }
  const float rG = nmax > 0 ? rcp[6] / (float)nmax : 0.f;  // du share of a tied key
  __syncthreads();
  if (has) rcp[4] = rG * p.scale;  // dS share, read by the dK/dV kernel
  const int grp = row >> 5;
  double dsum = 0.0;  // this row's sum of du; per-tile fp32 sums are added in fp64
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * TB;
    __syncthreads();
    stage<D>(Ks, K, p.ksn, n0, N);
    stage<D>(Vs, V, p.vsn, n0, N);
    __syncthreads();
    if (!has) continue;
    if (p.mask && p.mask[((int64_t)bh * p.nq32 + grp) * p.nk64 + t] == 0) continue;
    const int jmax = min(TB, N - n0);
    float tsum = 0.f;
    for (int j = 0; j < jmax; ++j) {
      if (CAUSAL && n0 + j > row) break;
      float s = 0.f, dw = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = __builtin_fmaf(q[d], Ks[j][d], s);
        dw = __builtin_fmaf(gdo[d], Vs[j][d], dw);
      }
      const float sv = __builtin_fmaf(s, p.scale, ntau);
      const float u = sv > 0.f ? sv : 0.f;
      const float u2 = u * u, u4 = u2 * u2;
      const float u9 = u4 * u4 * u;
      float du = rcoef * u9 * (dw - rD);
      if (u == rM && u > 0.f) du += rG;
      tsum += du;
      const float ds = du * p.scale;
#pragma unroll
      for (int d = 0; d < D; ++d) dq[d] = __builtin_fmaf(ds, Ks[j][d], dq[d]);
    }
    dsum += (double)tsum;
  }
  dsum = wave_sum_d(dsum);
  if (lane == 0) p.partials[(int64_t)bh * gridDim.x + blockIdx.x] = dsum;
  if (!has) return;
  float* dQ = static_cast<float*>(p.dq) + b * p.dqsb + h * p.dqsh + (int64_t)row * p.dqsn;
#pragma unroll
  for (int d = 0; d < D; ++d) dQ[d] = dq[d];
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(64) void f32_bwd_dkdv_kernel(BwdParams p) {
  __shared__ float Qs[TB][D], dOs[TB][D], RC[TB][8];
  const int lane = threadIdx.x, N = p.N;
  const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
  const int key = blockIdx.x * TB + lane;
  const bool has = key < N;
  const float* Q = static_cast<const float*>(p.q) + b * p.qsb + h * p.qsh;
  const float* K = static_cast<const float*>(p.k) + b * p.ksb + h * p.ksh;
  const float* V = static_cast<const float*>(p.v) + b * p.vsb + h * p.vsh;
  const float* dO = static_cast<const float*>(p.dout) + b * p.dosb + h * p.dosh;
  const float ntau = -p.tau[0];
  float k[D], v[D], dk[D], dv[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    k[d] = has ? K[(int64_t)key * p.ksn + d] : 0.f;
    v[d] = has ? V[(int64_t)key * p.vsn + d] : 0.f;
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  const int nqt = (N + TB - 1) / TB;
  const int qt0 = CAUSAL ? blockIdx.x : 0;
  for (int qt = qt0; qt < nqt; ++qt) {
    const int m0 = qt * TB;
    __syncthreads();
    stage<D>(Qs, Q, p.qsn, m0, N);
    stage<D>(dOs, dO, p.dosn, m0, N);
    for (int idx = lane; idx < TB * 8; idx += TB) {
      const int r = idx / 8, c = idx % 8;
      RC[r][c] = (m0 + r < N) ? p.rc[8 * ((int64_t)bh * N + m0 + r) + c] : 0.f;
    }
    __syncthreads();
    if (p.mask) {
      const int r32 = m0 >> 5;
      const bool a0 = p.mask[((int64_t)bh * p.nq32 + r32) * p.nk64 + blockIdx.x] != 0;
      const bool a1 = (r32 + 1 < p.nq32) && p.mask[((int64_t)bh * p.nq32 + r32 + 1) * p.nk64 + blockIdx.x] != 0;
      if (!a0 && !a1) continue;
    }
    if (!has) continue;
    const int imax = min(TB, N - m0);
    for (int i = 0; i < imax; ++i) {
      if (CAUSAL && m0 + i < key) continue;
      float s = 0.f, dw = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = __builtin_fmaf(Qs[i][d], k[d], s);
        dw = __builtin_fmaf(dOs[i][d], v[d], dw);
      }
      const float sv = __builtin_fmaf(s, p.scale, ntau);
      const float u = sv > 0.f ? sv : 0.f;
      const float u2 = u * u, u4 = u2 * u2, u8 = u4 * u4;
      const float w = u8 * u2 * RC[i][1];
      float ds = RC[i][2] * (u8 * u) * (dw - RC[i][3]);
      if (u == RC[i][0] && u > 0.f) ds += RC[i][4];
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dv[d] = __builtin_fmaf(w, dOs[i][d], dv[d]);
        dk[d] = __builtin_fmaf(ds, Qs[i][d], dk[d]);
      }
    }
  }
  if (!has) return;
  float* dK = static_cast<float*>(p.dk) + b * p.dksb + h * p.dksh + (int64_t)key * p.dksn;
  float* dV = static_cast<float*>(p.dv) + b * p.dvsb + h * p.dvsh + (int64_t)key * p.dvsn;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    dK[d] = dk[d];
    dV[d] = dv[d];
  }
}

// dtau = -(sum of the du partials), in fp64 and a fixed order.
__global__ __launch_bounds__(256) void f32_dtau_kernel(const double* partials, int64_t n,
                                                       float* dtau) {
  __shared__ double red[256];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 256) acc += partials[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) dtau[0] = (float)(-red[0]);
}

template <int D>
int fwd_d(const FwdParams& fp, bool causal, bool has_gamma, hipStream_t st) {
  const dim3 grid((unsigned)((fp.N + TB - 1) / TB), (unsigned)(fp.B * fp.H)), block(TB);
  if (causal) {
    if (has_gamma) hipLaunchKernelGGL((f32_fwd_kernel<D, true, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((f32_fwd_kernel<D, true, false>), grid, block, 0, st, fp);
  } else {
    if (has_gamma) hipLaunchKernelGGL((f32_fwd_kernel<D, false, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((f32_fwd_kernel<D, false, false>), grid, block, 0, st, fp);
  }
  return launch_status("pnfx_flash_fwd(f32)");
}

template <int D>
int bwd_d(const BwdParams& bp, bool causal, bool has_gamma, int stages, hipStream_t st) {
  const unsigned nb = (unsigned)((bp.N + TB - 1) / TB);
  const dim3 grid(nb, (unsigned)(bp.B * bp.H)), block(TB);
  if (stages & PNFX_BWD_PREPARE) {
    const int64_t rows = (int64_t)bp.B * bp.H * bp.N;
    const dim3 gpre((unsigned)((rows + 255) / 256));
    if (has_gamma) hipLaunchKernelGGL((f32_bwd_pre_kernel<D, true>), gpre, dim3(256), 0, st, bp);
    else hipLaunchKernelGGL((f32_bwd_pre_kernel<D, false>), gpre, dim3(256), 0, st, bp);
    const int rc = launch_status("pnfx_flash_bwd(f32 prepare)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DQ) {
    if (causal) hipLaunchKernelGGL((f32_bwd_dq_kernel<D, true>), grid, block, 0, st, bp);
    else hipLaunchKernelGGL((f32_bwd_dq_kernel<D, false>), grid, block, 0, st, bp);
    hipLaunchKernelGGL(f32_dtau_kernel, dim3(1), dim3(256), 0, st, bp.partials,
                       (int64_t)bp.B * bp.H * nb, bp.dtau);
    const int rc = launch_status("pnfx_flash_bwd(f32 dq)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DKDV) {  // reads the G/Nmax the dQ stage wrote
    if (causal) hipLaunchKernelGGL((f32_bwd_dkdv_kernel<D, true>), grid, block, 0, st, bp);
    else hipLaunchKernelGGL((f32_bwd_dkdv_kernel<D, false>), grid, block, 0, st, bp);
    const int rc = launch_status("pnfx_flash_bwd(f32 dkdv)");
    if (rc) return rc;
  }
  return PNFX_OK;
}

}  // namespace

int flash_fwd_f32(const FwdParams& fp, int64_t D, bool causal, bool has_gamma, hipStream_t st) {
  switch (D) {
    case 16: return fwd_d<16>(fp, causal, has_gamma, st);
    case 32: return fwd_d<32>(fp, causal, has_gamma, st);
    case 64: return fwd_d<64>(fp, causal, has_gamma, st);
    case 128: return fwd_d<128>(fp, causal, has_gamma, st);
  }
  set_error("flash(f32): head dim %lld not in {16, 32, 64, 128}", (long long)D);
  return PNFX_EUNSUPPORTED;
}

int flash_bwd_f32(const BwdParams& bp, int64_t D, bool causal, bool has_gamma, int stages,
                  hipStream_t st) {
  switch (D) {
    case 16: return bwd_d<16>(bp, causal, has_gamma, stages, st);
    case 32: return bwd_d<32>(bp, causal, has_gamma, stages, st);
    case 64: return bwd_d<64>(bp, causal, has_gamma, stages, st);
    case 128: return bwd_d<128>(bp, causal, has_gamma, stages, st);
  }
  set_error("flash(f32): head dim %lld not in {16, 32, 64, 128}", (long long)D);
  return PNFX_EUNSUPPORTED;
}

}  // namespace pnfx
