// Causal depthwise FIR along the sequence axis (keys of pn_fir_tau), forward and adjoint.
//
// Streaming, HBM-bound.  Each thread owns one 16-byte channel chunk of RUN = 8 consecutive
// sequence rows of one (b, h) slice: it issues all RUN + K - 1 row loads up front (the
// K - 1 row causal halo is served by L2: the neighbouring run of the same wave reads those
// rows at the same time), evaluates the fp32 fused multiply-add chains in lag order, one
// input row at a time (each row widened to fp32 once and fed to every output that uses it),
// and writes RUN 16-byte rows with non-temporal stores (the output is streamed, not re-read
// by this kernel).  Eight consecutive lanes cover one 128-byte row of a d = 64 bf16 head, so
// every load and store instruction moves whole cache lines.  Of the variants measured on
// MI355X (runs of 2..64 rows, an LDS-staged 64-row tile, non-temporal loads, stores issued as
// soon as each output is complete), this one is the fastest; on the 32 MiB benchmark tensor
// it takes about 0.96x the time of the runtime's device copy of the same bytes.  At that size
// every workgroup is resident at once, so the arithmetic (about 9.5 VALU operations per
// output element, 7 of them the FMA chain) lies between the loads and the stores: widening
// every input element once per use instead of once per row took 1.2x as long.
//
// Numerics follow src/triton_pnfirtau.py:72-84 (forward) and :120-132 (adjoint):
// acc = x[n] * h0; acc = fma(x[n -/+ u], h_u, acc) for u = 1..K-1 while in range;
// h_u = taps[K-1-u] in fp32; one rounding to the storage type at the store.
#include <type_traits>

#include "pnfx_common.h"

namespace pnfx {
namespace {

constexpr int RUN = 8;
constexpr int KMAX = 16;

template <typename T>
struct Chunk {
  static constexpr int VEC = 16 / sizeof(T);
};

// A 16-byte chunk is kept raw (4 dwords) and widened to fp32 on use.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ float chunk_elem(const u32x4& r, int e);
template <>
__device__ __forceinline__ float chunk_elem<bf16>(const u32x4& r, int e) {
  const uint32_t d = r[e >> 1];
  return __uint_as_float((e & 1) ? (d & 0xffff0000u) : (d << 16));
}
template <>
__device__ __forceinline__ float chunk_elem<float>(const u32x4& r, int e) {
  return __uint_as_float(r[e]);
}

template <typename T>
__device__ __forceinline__ void store_chunk(T* p, const float* in);
template <>
__device__ __forceinline__ void store_chunk<bf16>(bf16* p, const float* in) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (bf16)in[e];
  __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(p));
}
template <>
__device__ __forceinline__ void store_chunk<float>(float* p, const float* in) {
  f32x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = in[e];
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}

struct FirArgs {
  const void* x;
  int64_t sb, sh, sn;
  void* y;
  int64_t B, H, N, C;
  const float* taps;
  int64_t taps_rows;
  int K;
};

// KT is the compile-time bound on the tap count (K <= KT); KT == 7 is the pn_fir_tau case.
// grid.x covers the (run, chunk) pairs of one (b, h) slice, grid.y = b * H + h; all index
// arithmetic except the final address is 32-bit (sizes are checked on the host).
template <typename T, int KT, bool ADJ>
__global__ __launch_bounds__(256) void fir_vec_kernel(FirArgs a) {
  constexpr int VEC = Chunk<T>::VEC;
  constexpr int WIN = RUN + KT - 1;
  const int CH = (int)a.C / VEC;
  const int N = (int)a.N;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= ((N + RUN - 1) / RUN) * CH) return;
  const int ch = t % CH;
  const int run = t / CH;
  const int bh = blockIdx.y;
  const int H = (int)a.H;
  const int b = bh / H, hh = bh % H;
  const int K = KT == 7 ? 7 : a.K;

  float h[KT];
  const float* tp = a.taps + (a.taps_rows == 1 ? 0 : hh) * K;
#pragma unroll
  for (int u = 0; u < KT; ++u) h[u] = u < K ? tp[K - 1 - u] : 0.0f;

  const T* xs = reinterpret_cast<const T*>(a.x) + (int64_t)b * a.sb + (int64_t)hh * a.sh + ch * VEC;
  const int n0 = run * RUN;
  // Window row w holds sequence row m = base + w.
  const int base = ADJ ? n0 : n0 - (KT - 1);
  u32x4 win[WIN];
  // Loads in the order the chain below uses the rows (loads complete in order, so the first
  // terms can start while the rest are in flight).
#pragma unroll
  for (int i = 0; i < WIN; ++i) {
    const int w = ADJ ? i : WIN - 1 - i;
    const int m = base + w;
    if (m >= 0 && m < N) {
      win[w] = *reinterpret_cast<const u32x4*>(xs + (int64_t)m * a.sn);
    } else {
      win[w] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  T* ys = reinterpret_cast<T*>(a.y) + ((int64_t)bh * N + n0) * a.C + ch * VEC;
  // Window rows in the order of increasing lag (newest first for the forward, oldest first
  // for the adjoint): each row is widened to fp32 once and feeds every output of the run
  // that uses it, as that output's next term.  Output j (row n = n0 + j) sits at window
  // index w0 = j + KT - 1 (forward) or j (adjoint) and takes lag u from window row w0 -/+ u,
  // so it still sees its terms in lag order u = 0, 1, ..., K - 1: the same chain and the same
  // roundings as one output at a time, with the widening done once per row instead of once
  // per use.
  float acc[RUN][VEC];
  // Away from the sequence ends every lag of every output of the run is in range; only runs
  // within K - 1 rows of an end take the per-term range test (wave-uniform in practice).
  const bool interior = ADJ ? (n0 + RUN + KT - 2 < N) : (n0 >= KT - 1);
  const auto chain = [&](auto checked) {
#pragma unroll
    for (int i = 0; i < WIN; ++i) {
      const int w = ADJ ? i : WIN - 1 - i;
      float xe[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) xe[e] = chunk_elem<T>(win[w], e);
#pragma unroll
      for (int j = 0; j < RUN; ++j) {
        const int w0 = ADJ ? j : j + KT - 1;
        const int u = ADJ ? w - w0 : w0 - w;  // lag of window row w for output j
        if (u < 0 || u >= KT) continue;       // compile-time after unrolling
        const int n = n0 + j;
        if (u == 0) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[j][e] = xe[e] * h[0];
        } else if ((KT == 7 || u < K) &&
                   (!decltype(checked)::value || (ADJ ? (n + u < N) : (n - u >= 0)))) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[j][e] = __builtin_fmaf(xe[e], h[u], acc[j][e]);
        }
      }
    }
  };
  if (interior) chain(std::integral_constant<bool, false>{});
  else chain(std::integral_constant<bool, true>{});
#pragma unroll
  for (int j = 0; j < RUN; ++j)
    if (n0 + j < N) store_chunk<T>(ys + (int64_t)j * a.C, acc[j]);
}

// One thread per output element; any channel stride / alignment.
template <typename T, bool ADJ>
__global__ __launch_bounds__(256) void fir_scalar_kernel(FirArgs a, int64_t sc) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.B * a.H * a.N * a.C) return;
  const int64_t c = t % a.C;
  const int64_t n = (t / a.C) % a.N;
  const int64_t bh = t / (a.C * a.N);
  const int64_t b = bh / a.H, hh = bh % a.H;
  const float* tp = a.taps + (a.taps_rows == 1 ? 0 : hh) * a.K;
  const T* xs = reinterpret_cast<const T*>(a.x) + b * a.sb + hh * a.sh + c * sc;
  float acc = to_f32(xs[n * a.sn]) * tp[a.K - 1];
  for (int u = 1; u < a.K; ++u) {
    const int64_t m = ADJ ? n + u : n - u;
    if (m < 0 || m >= a.N) break;
    acc = __builtin_fmaf(to_f32(xs[m * a.sn]), tp[a.K - 1 - u], acc);
  }
  reinterpret_cast<T*>(a.y)[(bh * a.N + n) * a.C + c] = from_f32<T>(acc);
}

template <typename T, bool ADJ>
int launch_fir(const FirArgs& a, hipStream_t st) {
  constexpr int VEC = Chunk<T>::VEC;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(a.x) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) && a.C % VEC == 0 &&
                      a.sb % VEC == 0 && a.sh % VEC == 0 && a.sn % VEC == 0;
  const int64_t per_slice = ((a.N + RUN - 1) / RUN) * (a.C / VEC);
  if (vec_ok && per_slice < (1ll << 30) && a.B * a.H < 65536 && a.N < (1ll << 30)) {
    const dim3 grid((unsigned)((per_slice + 255) / 256), (unsigned)(a.B * a.H));
    if (a.K == 7)
      hipLaunchKernelGGL((fir_vec_kernel<T, 7, ADJ>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((fir_vec_kernel<T, KMAX, ADJ>), grid, dim3(256), 0, st, a);
  } else {
    const int64_t total = a.B * a.H * a.N * a.C;
    hipLaunchKernelGGL((fir_scalar_kernel<T, ADJ>), dim3((total + 255) / 256), dim3(256), 0, st,
                       a, (int64_t)1);
  }
  return launch_status(ADJ ? "pnfx_fir_bwd" : "pnfx_fir_fwd");
}

int fir_entry(bool adj, const void* x, int64_t sb, int64_t sh, int64_t sn, void* y, int64_t B,
              int64_t H, int64_t N, int64_t C, const float* taps, int64_t taps_rows, int K,
              int dtype, void* stream) {
  PNFX_REQUIRE(x && y && taps, "fir: null pointer");
  PNFX_REQUIRE(B >= 0 && H >= 1 && N >= 0 && C >= 0, "fir: bad shape B=%lld H=%lld N=%lld C=%lld",
               (long long)B, (long long)H, (long long)N, (long long)C);
  PNFX_REQUIRE(K >= 1 && K <= KMAX, "fir: K=%d outside [1, %d]", K, KMAX);
  PNFX_REQUIRE(taps_rows == 1 || taps_rows == H, "fir: taps_rows=%lld must be 1 or H=%lld",
               (long long)taps_rows, (long long)H);
  if (B * H * N * C == 0) return PNFX_OK;
  FirArgs a{x, sb, sh, sn, y, B, H, N, C, taps, taps_rows, K};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == PNFX_BF16) return adj ? launch_fir<bf16, true>(a, st) : launch_fir<bf16, false>(a, st);
  if (dtype == PNFX_F32) return adj ? launch_fir<float, true>(a, st) : launch_fir<float, false>(a, st);
  set_error("fir: unsupported dtype %d", dtype);
  return PNFX_EUNSUPPORTED;
}

}  // namespace
}  // namespace pnfx

extern "C" int pnfx_fir_fwd(const void* x, int64_t sb, int64_t sh, int64_t sn, void* y, int64_t B,
                            int64_t H, int64_t N, int64_t C, const float* taps, int64_t taps_rows,
                            int K, int dtype, void* stream) {
  return pnfx::fir_entry(false, x, sb, sh, sn, y, B, H, N, C, taps, taps_rows, K, dtype, stream);
}

extern "C" int pnfx_fir_bwd(const void* gy, int64_t sb, int64_t sh, int64_t sn, void* gx,
                            int64_t B, int64_t H, int64_t N, int64_t C, const float* taps,
                            int64_t taps_rows, int K, int dtype, void* stream) {
  return pnfx::fir_entry(true, gy, sb, sh, sn, gx, B, H, N, C, taps, taps_rows, K, dtype, stream);
}
