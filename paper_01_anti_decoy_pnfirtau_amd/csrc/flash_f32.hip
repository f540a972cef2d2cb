// Flash pn_fir_tau attention for fp32 tensors (the reference's TF32-off parity path) on the
// MFMA units: scores on v_mfma_f64_16x16x4_f64, the other products on v_mfma_f32_16x16x4_f32.
//
// Math (src/triton_pnfirtau.py:313-621): s = fma(q.k, scale, -tau), u = relu(s), P = u^10,
// Z = sum P + 1e-12, M = max u, Nmax = #(u == M); O = (sum P v) gate / Z.  Nothing is
// rounded below fp32.  The score's dot product q.k is formed in fp64 (the fp32 inputs'
// products are exact there) and rounded to fp32 once: u^9 in the gradient multiplies the
// score's relative error by nine, and an fp32 sum of the d products, where they cancel, put
// single gradient elements past 1e-5 of the tensor's scale on random inputs.
//
// MFMA mapping.  Lane l = 16 g + r of a wave holds A[row r][k-slot g] and B[k-slot g][col r];
// a dot product over the head dimension runs D/4 chained MFMAs, and in step s k-slot g carries
// head column g (D/4) + s, in every kernel.  The fp32 MFMA returns D[4 g + i][r] in register i,
// the fp64 MFMA D[g + 4 i][r].  The forward and the dQ kernel form S^T = K Q^T (K as A, Q as B:
// a lane holds one query, keys g + 4 i of each 16-key block); the dK/dV kernel forms
// S = Q K^T (a lane holds one key, queries g + 4 i).  On gfx950 the fp64 MFMA is bitwise
// transpose-symmetric (swapping the A and B values gives exactly the transposed result), so
// every kernel recomputes the forward's scores bit for bit and the backward's peak-tie test
// u == M sees the forward's ties.  dW = dO V^T runs on the fp32 MFMA with its A rows taken in
// the 4x4-transposed order perm4(r), so that its register i holds the same key (or query)
// g + 4 i as the score's.  The score registers then feed the second product directly:
// register i is k-slot g of MFMA i, i.e. keys (or queries) 4 i .. 4 i + 3 of the block.
//
// Workgroups of four waves own 32 query rows (forward, dQ) or 32 keys (dK/dV) as two 16-row
// groups, and stream the other operand through LDS in tiles of 64 rows; each group's two waves
// split every tile, one taking its 16-row blocks 0-1 and the other 2-3, and their partial sums
// are added in a fixed order at the end (or, for dQ's row constants, between its sweeps).
// Against one wave per 16 rows over whole tiles this halves the longest causal block's
// sequential work and doubles the workgroups: at this path's sizes (a few (b, h) slices) the
// grid fills the GPU about once, so the longest block sets the kernel's time.  Row constants, tile mask, tau
// partials and workspace are those of the bf16 kernels' interface (BwdParams), with fp32 rows of
// eight constants.
#include "flash.h"

namespace pnfx {
namespace {

constexpr int TB = 64;  // rows per LDS tile
constexpr int RB = 32;  // rows (forward, dQ) or keys (dK/dV) per workgroup
// Key tiles of one sequence with a tile mask (N <= 65536, the masks's own limit)
constexpr int kMaxTiles = 1024;

__device__ __forceinline__ float pow10f_(float u) {
  const float u2 = u * u;
  const float u4 = u2 * u2;
  return u4 * u4 * u2;
}

typedef double f64x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Row r of a 4x4-transposed 16-row block: the fp32 MFMA's register i of lane group g then
// holds row g + 4 i, as the fp64 MFMA's does.
__device__ __forceinline__ int perm4(int r) { return 4 * (r & 3) + (r >> 2); }

// The 32-row (or 32-key) block and the (b, h) slice of this workgroup in a 1-D grid of nb * BH
// workgroups.  Every slice's blocks go in the same order, one block of each slice at a time;
// heavy_last_index: the order runs from the last block down (the query-parallel kernels under
// a causal mask, whose last rows see the most keys), else from block 0 up (the key-parallel
// kernel, whose first keys see the most queries).  The grid holds a few workgroups per CU at
// this path's sizes, and dispatching the longest blocks first keeps one from starting last.
__device__ __forceinline__ void block_of(int nb, int BH, bool heavy_last_index, int& blk,
                                         int& bh) {
  const int j = blockIdx.x / BH;
  bh = blockIdx.x % BH;
  blk = heavy_last_index ? nb - 1 - j : j;
}

// Rows row0 .. row0 + 63 of two [N, D] slices (row strides sa, sb) staged into LDS tiles of pitch
// LD, zero past N; 256 threads, coalesced along each row.  load() issues every global load of a
// tile into registers and returns at once, so the next tile's loads are in flight while the
// current tile is computed; store() writes them to LDS (after the barrier that frees it).
template <int D, int LD>
struct TilePair {
  static constexpr int PER = TB * D / 256;
  float va[PER], vb[PER];
  __device__ __forceinline__ void load(const float* sa_, int64_t sa, const float* sb_, int64_t sb,
                                       int row0, int N, int tid) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = tid + 256 * j, r = idx / D, c = idx % D;
      const bool ok = row0 + r < N;
      va[j] = ok ? sa_[(int64_t)(row0 + r) * sa + c] : 0.f;
      vb[j] = ok ? sb_[(int64_t)(row0 + r) * sb + c] : 0.f;
    }
  }
  __device__ __forceinline__ void store(float* da, float* db, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int idx = tid + 256 * j, r = idx / D, c = idx % D;
      da[r * LD + c] = va[j];
      db[r * LD + c] = vb[j];
    }
  }
};

// NB 16-row blocks of a 64-row tile at once, from block kb0 (independent MFMA chains, which keep
// the MFMA pipeline busy where one chain would wait on its own results): block kb's lane row is
// tile row 16 (kb0 + kb) + (PERM ? perm4(r) : r).  Each block runs exactly the MFMA sequence of
// one 16-row block (D/4 chained MFMAs in head-column order), so its values do not depend on
// the interleaving.
template <int D, int LD, bool PERM, int NB>
__device__ __forceinline__ void dot_tile(const float* tile, int r, int g, const float (&b)[D / 4],
                                         f32x4 (&out)[NB], int kb0) {
  constexpr int KS = D / 4;
  const int row = PERM ? perm4(r) : r;
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) out[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; s += 4) {
    f32x4 a[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb)
      a[kb] = *reinterpret_cast<const f32x4*>(tile + (16 * (kb0 + kb) + row) * LD + g * KS + s);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int kb = 0; kb < NB; ++kb) out[kb] = mfma4(a[kb][j], b[s + j], out[kb]);
  }
}
template <int D, int LD, int NB>
__device__ __forceinline__ void dot_tile64(const float* tile, int r, int g,
                                           const double (&b)[D / 4], f32x4 (&out)[NB], int kb0) {
  constexpr int KS = D / 4;
  f64x4 acc[NB];
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) acc[kb] = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int s = 0; s < KS; s += 4) {
    f32x4 a[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb)
      a[kb] = *reinterpret_cast<const f32x4*>(tile + (16 * (kb0 + kb) + r) * LD + g * KS + s);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int kb = 0; kb < NB; ++kb)
        acc[kb] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a[kb][j], b[s + j], acc[kb], 0, 0, 0);
  }
#pragma unroll
  for (int kb = 0; kb < NB; ++kb)
    out[kb] = f32x4{(float)acc[kb][0], (float)acc[kb][1], (float)acc[kb][2], (float)acc[kb][3]};
}

// The lane's D/4 head columns g D/4 .. of one row of global memory (zero if the row is absent).
template <int D, typename T>
__device__ __forceinline__ void load_row(T (&dst)[D / 4], const float* row, bool ok, int g) {
#pragma unroll
  for (int s = 0; s < D / 4; ++s) dst[s] = ok ? (T)row[g * (D / 4) + s] : (T)0;
}

template <int D, bool CAUSAL, bool HAS_GAMMA>
__global__ __launch_bounds__(256) void f32_fwd_kernel(FwdParams p) {
  constexpr int KS = D / 4, DB = D / 16, LD = D + 4;
  __shared__ __attribute__((aligned(16))) float Ks[TB * LD];
  __shared__ __attribute__((aligned(16))) float Vs[TB * LD];
  // each wave's activity bit per key tile (one 32-bit word per 32 tiles), for the tile mask
  __shared__ uint32_t act_s[4][(kMaxTiles + 31) / 32];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
  const int N = p.N;
  int blk, bh;
  block_of((N + RB - 1) / RB, p.B * p.H, CAUSAL, blk, bh);
  const int b = bh / p.H, h = bh % p.H;
  // the wave's 16-row group and the half (key blocks 2 kp, 2 kp + 1) of every key tile it takes
  const int rg = w >> 1, kp = w & 1;
  const int m0 = blk * RB, qw = m0 + 16 * rg, row = qw + r;
  if (lane < (kMaxTiles + 31) / 32) act_s[w][lane] = 0u;
  const bool has = row < N;
  const float* Q = static_cast<const float*>(p.q) + b * p.qsb + h * p.qsh;
  const float* K = static_cast<const float*>(p.k) + b * p.ksb + h * p.ksh;
  const float* V = static_cast<const float*>(p.v) + b * p.vsb + h * p.vsh;
  const float ntau = -p.tau[0], scale = p.scale;
  double qf[KS];
  load_row<D>(qf, Q + (int64_t)row * p.qsn, has, g);
  f32x4 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = 0.f, mass = 0.f;
  int cnt = 0;
  const int kv_end = CAUSAL ? min(m0 + RB, N) : N;
  const int ntiles = (kv_end + TB - 1) / TB;
  const int g0 = blk;  // the workgroup's 32-row group of the tile mask
  TilePair<D, LD> pre;
  if (ntiles > 0) pre.load(K, p.ksn, V, p.vsn, 0, N, tid);
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * TB;
    __syncthreads();
    pre.store(Ks, Vs, tid);
    __syncthreads();
    if (t + 1 < ntiles) pre.load(K, p.ksn, V, p.vsn, n0 + TB, N, tid);
    bool act = false;
    // some key of the wave's half of the tile is at or below the wave's diagonal
    if (!(CAUSAL && n0 + 32 * kp > qw + 15)) {
      f32x4 st[2];
      dot_tile64<D, LD, 2>(Ks, r, g, qf, st, 2 * kp);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kb = 2 * kp + j;
        if (CAUSAL && n0 + 16 * kb > qw + 15) break;  // the block is above the wave's diagonal
        float pw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = n0 + 16 * kb + g + 4 * i;
          const float sv = __builtin_fmaf(st[j][i], scale, ntau);
          const bool valid = has && key < N && !(CAUSAL && key > row);
          const float u = (valid && sv > 0.f) ? sv : 0.f;
          act |= u > 0.f;
          if (u > m) {
            m = u;
            cnt = 1;
          } else if (u == m) {
            ++cnt;
          }
          pw[i] = pow10f_(u);
          mass += pw[i];
        }
        // O^T[d][query] += V^T[d][key] P[key][query]: register i is k-slot g of MFMA i (key g + 4i)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int db = 0; db < DB; ++db)
            acc[db] = mfma4(Vs[(16 * kb + g + 4 * i) * LD + 16 * db + r], pw[i], acc[db]);
      }
    }
    const bool wave_act = __any(act);  // every lane of the wave takes part in the vote
    if (p.mask && wave_act && lane == 0) act_s[w][t >> 5] |= 1u << (t & 31);  // nk64 <= kMaxTiles
  }
  __syncthreads();  // every wave's tiles and activity bits are done
  if (p.mask) {  // the workgroup's 32-row group: all four waves
    for (int t = tid; t < p.nk64; t += 256) {
      const uint32_t bit = 1u << (t & 31);
      const int wd = t >> 5;
      const bool a0 = t < ntiles && ((act_s[0][wd] | act_s[1][wd] | act_s[2][wd] | act_s[3][wd]) & bit);
      if (g0 < p.nq32) p.mask[((int64_t)bh * p.nq32 + g0) * p.nk64 + t] = a0 ? 1 : 0;
    }
  }
  // The second half (kp = 1) of each row group hands its lane-wise sums to the first through
  // LDS (the K tile's, free now); the first adds them, half 0 then half 1.
  constexpr int NX = 4 * DB + 3;  // floats per lane: the P.V sums, peak, tie count, mass
  static_assert(2 * NX * 64 <= TB * LD, "the halves' sums fit the K tile");
  float* xs = Ks + rg * NX * 64 + lane;
  if (kp == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[(4 * db + i) * 64] = acc[db][i];
    xs[(4 * DB) * 64] = m;
    xs[(4 * DB + 1) * 64] = __int_as_float(cnt);
    xs[(4 * DB + 2) * 64] = mass;
  }
  __syncthreads();
  if (kp == 1) return;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[db][i] += xs[(4 * db + i) * 64];
  {
    const float m1 = xs[(4 * DB) * 64];
    const int c1 = __float_as_int(xs[(4 * DB + 1) * 64]);
    const float mm = fmaxf(m, m1);
    cnt = (m == mm ? cnt : 0) + (m1 == mm ? c1 : 0);
    m = mm;
    mass += xs[(4 * DB + 2) * 64];
  }
  // the four lane groups of a query row hold disjoint keys: combine their statistics
  float M = fmaxf(m, __shfl_xor(m, 16, 64));
  M = fmaxf(M, __shfl_xor(M, 32, 64));
  int c = (m == M) ? cnt : 0;
  c += __shfl_xor(c, 16, 64);
  c += __shfl_xor(c, 32, 64);
  float ms = mass + __shfl_xor(mass, 16, 64);
  ms += __shfl_xor(ms, 32, 64);
  if (!has) return;
  const float gate = M > 0.f ? (HAS_GAMMA ? M / (M + p.gamma) : 1.f) : 0.f;
  const float z = ms + 1e-12f;
  const float so = gate / z;
  float* O = static_cast<float*>(p.o) + b * p.osb + h * p.osh + (int64_t)row * p.osn;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) O[16 * db + 4 * g + i] = acc[db][i] * so;
  if (g == 0) {
    const int64_t si = (int64_t)bh * N + row;
    p.M[si] = M;
    p.Z[si] = z;
    if (p.Nmax) p.Nmax[si] = M > 0.f ? c : 0;
  }
}

// Row constants (eight floats per row): M, g/Z, 10 g/Z scale, D (written by the dQ kernel),
// the dS share of a peak tie (written by the dQ kernel), 10 g/Z.
template <int D, bool HAS_GAMMA>
__global__ __launch_bounds__(256) void f32_bwd_pre_kernel(BwdParams p) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= (int64_t)p.B * p.H * p.N) return;
  const float M = p.M[row], Z = p.Z[row];
  const float g = M > 0.f ? (HAS_GAMMA ? M / (M + p.gamma) : 1.f) : 0.f;
  float* rc = p.rc + 8 * row;
  rc[0] = M;
  rc[1] = g / Z;
  rc[2] = 10.f * g / Z * p.scale;  // dS = du scale, for the dK/dV kernel
  rc[5] = 10.f * g / Z;            // du, for the dQ kernel (its sum is the tau gradient)
}

// Whether 64-key tile t is silent for 32-row group grp by the forward's tile mask (if given).
__device__ __forceinline__ bool silent_tile(const BwdParams& p, int bh, int grp, int t) {
  return p.mask && p.mask[((int64_t)bh * p.nq32 + grp) * p.nk64 + t] == 0;
}

// dQ and the tau partials: query-parallel, the forward's tiling, in two sweeps over the keys.
// The first forms each row's D = sum_j (P_j / Z) dW_j (src/triton_pnfirtau.py:575-577 take it
// from the flash identity <dO, O>/g instead; in fp32 that difference of two separately rounded
// values loses the cancellation of dW - D on peaked rows, while this sum holds the very dW
// values the gradient subtracts it from, bitwise the same in every sweep and in the dK/dV
// kernel) and counts the peak ties; the second accumulates dQ, with G/Nmax for tied keys.
template <int D, bool CAUSAL, bool HAS_GAMMA>
__global__ __launch_bounds__(256) void f32_bwd_dq_kernel(BwdParams p) {
  constexpr int KS = D / 4, DB = D / 16, LD = D + 4;
  __shared__ __attribute__((aligned(16))) float Ks[TB * LD];
  __shared__ __attribute__((aligned(16))) float Vs[TB * LD];
  __shared__ double part_s[4];
  __shared__ float pdw_s[4][16];  // each wave's row sums of P dW and tie counts, between sweeps
  __shared__ int nt_s[4][16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
  const int N = p.N, nb = (N + RB - 1) / RB;
  int blk, bh;
  block_of(nb, p.B * p.H, CAUSAL, blk, bh);
  const int b = bh / p.H, h = bh % p.H;
  // the wave's 16-row group and the half (key blocks 2 kp, 2 kp + 1) of every key tile it takes
  const int rg = w >> 1, kp = w & 1;
  const int m0 = blk * RB, qw = m0 + 16 * rg, row = qw + r;
  const bool has = row < N;
  const float* Q = static_cast<const float*>(p.q) + b * p.qsb + h * p.qsh;
  const float* K = static_cast<const float*>(p.k) + b * p.ksb + h * p.ksh;
  const float* V = static_cast<const float*>(p.v) + b * p.vsb + h * p.vsh;
  const float* dO = static_cast<const float*>(p.dout) + b * p.dosb + h * p.dosh;
  const float ntau = -p.tau[0], scale = p.scale;
  double qf[KS];
  float df[KS];
  load_row<D>(qf, Q + (int64_t)row * p.qsn, has, g);
  load_row<D>(df, dO + (int64_t)row * p.dosn, has, g);
  float* rcp = p.rc + 8 * ((int64_t)bh * N + (has ? row : 0));
  const float rM = has ? rcp[0] : 0.f, rcoef = has ? rcp[5] : 0.f;
  const float Zr = has ? p.Z[(int64_t)bh * N + row] : 1.f;
  const int kv_end = CAUSAL ? min(m0 + RB, N) : N;
  const int ntiles = (kv_end + TB - 1) / TB;
  // score of register i of key block kb of the tile at n0, masked and rectified
  const auto score = [&](const f32x4& s, int n0, int kb, int i) {
    const int key = n0 + 16 * kb + g + 4 * i;
    const float sv = __builtin_fmaf(s[i], scale, ntau);
    const bool valid = has && key < N && !(CAUSAL && key > row);
    return (valid && sv > 0.f) ? sv : 0.f;
  };
  const int grp = blk;  // the workgroup's 32-row group of the tile mask
  // nothing of the wave's half of tile t is at or below its diagonal, or the tile is silent
  const auto skip = [&](int t) {
    return qw >= N || silent_tile(p, bh, grp, t) || (CAUSAL && t * TB + 32 * kp > qw + 15);
  };
  // First sweep: sum P dW and the peak-tie counts (the backward has no Nmax from the forward).
  float pdw = 0.f;
  int nt = 0;
  TilePair<D, LD> pre;
  if (ntiles > 0) pre.load(K, p.ksn, V, p.vsn, 0, N, tid);
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * TB;
    __syncthreads();
    pre.store(Ks, Vs, tid);
    __syncthreads();
    // the next tile of this sweep, or the first of the next sweep
    pre.load(K, p.ksn, V, p.vsn, t + 1 < ntiles ? n0 + TB : 0, N, tid);
    if (skip(t)) continue;
    f32x4 st[2], dwt[2];
    dot_tile64<D, LD, 2>(Ks, r, g, qf, st, 2 * kp);
    dot_tile<D, LD, true, 2>(Vs, r, g, df, dwt, 2 * kp);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = 2 * kp + j;
      if (CAUSAL && n0 + 16 * kb > qw + 15) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float u = score(st[j], n0, kb, i);
        pdw = __builtin_fmaf(pow10f_(u), dwt[j][i], pdw);
        nt += (u == rM && u > 0.f) ? 1 : 0;
      }
    }
  }
  pdw += __shfl_xor(pdw, 16, 64);
  pdw += __shfl_xor(pdw, 32, 64);
  nt += __shfl_xor(nt, 16, 64);
  nt += __shfl_xor(nt, 32, 64);
  // the row group's two halves: half 0's sums plus half 1's, the same in both waves
  if (g == 0) {
    pdw_s[w][r] = pdw;
    nt_s[w][r] = nt;
  }
  __syncthreads();
  pdw = pdw_s[2 * rg][r] + pdw_s[2 * rg + 1][r];
  nt = nt_s[2 * rg][r] + nt_s[2 * rg + 1][r];
  const float rD = rM > 0.f ? pdw / Zr : 0.f;
  float rGu = 0.f;  // the whole row's peak-tie du
  if (HAS_GAMMA && rM > 0.f) rGu = rD * (p.gamma / ((rM + p.gamma) * (rM + p.gamma)));
  const float rG = nt > 0 ? rGu / (float)nt : 0.f;  // du share of a tied key
  if (has && g == 0 && kp == 0) {
    rcp[3] = rD;          // read by the dK/dV kernel
    rcp[4] = rG * scale;  // its dS share of a tied key
  }
  f32x4 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  double dsum = 0.0;  // the lane's sum of du; per-tile fp32 sums are added in fp64
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * TB;
    __syncthreads();
    pre.store(Ks, Vs, tid);
    __syncthreads();
    if (t + 1 < ntiles) pre.load(K, p.ksn, V, p.vsn, n0 + TB, N, tid);
    if (skip(t)) continue;
    float tsum = 0.f;
    f32x4 st[2], dwt[2];
    dot_tile64<D, LD, 2>(Ks, r, g, qf, st, 2 * kp);
    dot_tile<D, LD, true, 2>(Vs, r, g, df, dwt, 2 * kp);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = 2 * kp + j;
      if (CAUSAL && n0 + 16 * kb > qw + 15) break;
      float ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float u = score(st[j], n0, kb, i);
        const float u2 = u * u, u4 = u2 * u2;
        const float u9 = u4 * u4 * u;
        float du = rcoef * u9 * (dwt[j][i] - rD);
        if (u == rM && u > 0.f) du += rG;
        tsum += du;
        ds[i] = du * scale;
      }
      // dQ^T[d][query] += K^T[d][key] dS^T[key][query]
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int db = 0; db < DB; ++db)
          acc[db] = mfma4(Ks[(16 * kb + g + 4 * i) * LD + 16 * db + r], ds[i], acc[db]);
    }
    dsum += (double)tsum;
  }
  dsum = wave_sum_d(dsum);
  if (lane == 0) part_s[w] = dsum;
  __syncthreads();  // also: every wave is done with the K tile, which takes half 1's dQ sums
  if (tid == 0)
    p.partials[(int64_t)bh * nb + blk] = (part_s[0] + part_s[1]) + (part_s[2] + part_s[3]);
  static_assert(2 * 4 * DB * 64 <= TB * LD, "the halves' dQ sums fit the K tile");
  float* xs = Ks + rg * 4 * DB * 64 + lane;
  if (kp == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[(4 * db + i) * 64] = acc[db][i];
  }
  __syncthreads();
  if (kp == 1 || !has) return;
  float* dQ = static_cast<float*>(p.dq) + b * p.dqsb + h * p.dqsh + (int64_t)row * p.dqsn;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) dQ[16 * db + 4 * g + i] = acc[db][i] + xs[(4 * db + i) * 64];
}

// dK and dV: key-parallel, 32 keys per workgroup (16 per wave pair, held as MFMA B operands);
// query tiles of 64 rows and their row constants stream through LDS, each wave of a pair taking
// half of every tile's 16-row query blocks.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256) void f32_bwd_dkdv_kernel(BwdParams p) {
  constexpr int KS = D / 4, DB = D / 16, LD = D + 4;
  __shared__ __attribute__((aligned(16))) float Qs[TB * LD];
  __shared__ __attribute__((aligned(16))) float dOs[TB * LD];
  __shared__ __attribute__((aligned(16))) float RC[TB * 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, g = lane >> 4;
  const int N = p.N;
  int blk, bh;
  block_of((N + RB - 1) / RB, p.B * p.H, false, blk, bh);
  const int b = bh / p.H, h = bh % p.H;
  // the wave's 16-key group and the half (query blocks 2 qp, 2 qp + 1) of every query tile
  const int kg = w >> 1, qp = w & 1;
  const int k0 = blk * RB, kw = k0 + 16 * kg, key = kw + r;
  const int kt = k0 / TB;  // the 64-key tile of the tile mask that holds these keys
  const bool has = key < N;
  const float* Q = static_cast<const float*>(p.q) + b * p.qsb + h * p.qsh;
  const float* K = static_cast<const float*>(p.k) + b * p.ksb + h * p.ksh;
  const float* V = static_cast<const float*>(p.v) + b * p.vsb + h * p.vsh;
  const float* dO = static_cast<const float*>(p.dout) + b * p.dosb + h * p.dosh;
  const float ntau = -p.tau[0], scale = p.scale;
  double kf[KS];
  float vf[KS];
  load_row<D>(kf, K + (int64_t)key * p.ksn, has, g);
  load_row<D>(vf, V + (int64_t)key * p.vsn, has, g);
  f32x4 adk[DB], adv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    adk[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    adv[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int nqt = (N + TB - 1) / TB;
  const int qt0 = CAUSAL ? kt : 0;
  const float* rcb = p.rc + 8 * (int64_t)bh * N;
  TilePair<D, LD> pre;
  float rcn[2];  // the row constants of the next tile (8 floats per row, two per thread)
  const auto load_rc = [&](int m) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int idx = tid + 256 * j;
      rcn[j] = (m + idx / 8 < N) ? rcb[8 * (int64_t)m + idx] : 0.f;
    }
  };
  if (qt0 < nqt) {
    pre.load(Q, p.qsn, dO, p.dosn, qt0 * TB, N, tid);
    load_rc(qt0 * TB);
  }
  for (int qt = qt0; qt < nqt; ++qt) {
    const int m0 = qt * TB;
    __syncthreads();
    pre.store(Qs, dOs, tid);
    RC[tid] = rcn[0];
    RC[tid + 256] = rcn[1];
    __syncthreads();
    if (qt + 1 < nqt) {
      pre.load(Q, p.qsn, dO, p.dosn, m0 + TB, N, tid);
      load_rc(m0 + TB);
    }
    if (p.mask) {
      const int r32 = m0 >> 5;
      const bool a0 = p.mask[((int64_t)bh * p.nq32 + r32) * p.nk64 + kt] != 0;
      const bool a1 = (r32 + 1 < p.nq32) &&
                      p.mask[((int64_t)bh * p.nq32 + r32 + 1) * p.nk64 + kt] != 0;
      if (!a0 && !a1) continue;
    }
    // every query of the wave's half of the tile precedes its keys
    if (kw >= N || (CAUSAL && m0 + 32 * qp + 31 < kw)) continue;
    // S[query][key] = Q K^T (Q as A, fp64): bitwise the forward's S^T, transposed
    f32x4 st[2], dwt[2];
    dot_tile64<D, LD, 2>(Qs, r, g, kf, st, 2 * qp);
    dot_tile<D, LD, true, 2>(dOs, r, g, vf, dwt, 2 * qp);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int qb = 2 * qp + j;
      if (CAUSAL && m0 + 16 * qb + 15 < kw) continue;  // every query of the block precedes the keys
      float wv[4], ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qi = 16 * qb + g + 4 * i, q = m0 + qi;
        const float* c = RC + 8 * qi;
        const float sv = __builtin_fmaf(st[j][i], scale, ntau);
        const bool valid = has && q < N && !(CAUSAL && key > q);
        const float u = (valid && sv > 0.f) ? sv : 0.f;
        const float u2 = u * u, u4 = u2 * u2, u8 = u4 * u4;
        wv[i] = u8 * u2 * c[1];
        float d = c[2] * (u8 * u) * (dwt[j][i] - c[3]);
        if (u == c[0] && u > 0.f) d += c[4];
        ds[i] = d;
      }
      // dV^T[d][key] += dO^T[d][query] W[query][key]; dK^T likewise with Q and dS
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int off = (16 * qb + g + 4 * i) * LD + 16 * db + r;
          adv[db] = mfma4(dOs[off], wv[i], adv[db]);
          adk[db] = mfma4(Qs[off], ds[i], adk[db]);
        }
    }
  }
  // half 1 of each key group hands its sums to half 0 through LDS (the query tiles', free
  // once every wave is past the loop); half 0 adds them, its own first
  __syncthreads();
  static_assert(2 * 4 * DB * 64 <= TB * LD, "the halves' sums fit a query tile");
  float* xk = Qs + kg * 4 * DB * 64 + lane;
  float* xv = dOs + kg * 4 * DB * 64 + lane;
  if (qp == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xk[(4 * db + i) * 64] = adk[db][i];
        xv[(4 * db + i) * 64] = adv[db][i];
      }
  }
  __syncthreads();
  if (qp == 1 || !has) return;
  float* dK = static_cast<float*>(p.dk) + b * p.dksb + h * p.dksh + (int64_t)key * p.dksn;
  float* dV = static_cast<float*>(p.dv) + b * p.dvsb + h * p.dvsh + (int64_t)key * p.dvsn;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dK[16 * db + 4 * g + i] = adk[db][i] + xk[(4 * db + i) * 64];
      dV[16 * db + 4 * g + i] = adv[db][i] + xv[(4 * db + i) * 64];
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
  const int64_t nwg = (int64_t)((fp.N + RB - 1) / RB) * fp.B * fp.H;
  if (nwg >= (1ll << 31)) {
    set_error("flash(f32): %lld workgroups exceed the grid", (long long)nwg);
    return PNFX_EINVAL;
  }
  const dim3 grid((unsigned)nwg), block(256);
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
  const int64_t nb = (bp.N + RB - 1) / RB;
  if (nb * bp.B * bp.H >= (1ll << 31)) {
    set_error("flash(f32): %lld workgroups exceed the grid", (long long)(nb * bp.B * bp.H));
    return PNFX_EINVAL;
  }
  const dim3 grid((unsigned)(nb * bp.B * bp.H)), block(256);
  if (stages & PNFX_BWD_PREPARE) {
    const int64_t rows = (int64_t)bp.B * bp.H * bp.N;
    const dim3 gpre((unsigned)((rows + 255) / 256));
    if (has_gamma) hipLaunchKernelGGL((f32_bwd_pre_kernel<D, true>), gpre, dim3(256), 0, st, bp);
    else hipLaunchKernelGGL((f32_bwd_pre_kernel<D, false>), gpre, dim3(256), 0, st, bp);
    const int rc = launch_status("pnfx_flash_bwd(f32 prepare)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DQ) {
    if (causal) {
      if (has_gamma) hipLaunchKernelGGL((f32_bwd_dq_kernel<D, true, true>), grid, block, 0, st, bp);
      else hipLaunchKernelGGL((f32_bwd_dq_kernel<D, true, false>), grid, block, 0, st, bp);
    } else {
      if (has_gamma) hipLaunchKernelGGL((f32_bwd_dq_kernel<D, false, true>), grid, block, 0, st, bp);
      else hipLaunchKernelGGL((f32_bwd_dq_kernel<D, false, false>), grid, block, 0, st, bp);
    }
    hipLaunchKernelGGL(f32_dtau_kernel, dim3(1), dim3(256), 0, st, bp.partials,
                       bp.B * bp.H * nb, bp.dtau);
    const int rc = launch_status("pnfx_flash_bwd(f32 dq)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DKDV) {  // reads the D and G/Nmax the dQ stage wrote
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
