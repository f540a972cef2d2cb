// Flash pn_fir_tau attention on bf16 MFMA (gfx950), forward and deterministic backward.
//
// Math (src/triton_pnfirtau.py:313-621): per query row i and key j <= i,
//   s = fma(q_i . k_j, scale, -tau), u = relu(s), P = u^10 (four multiplies, no exp),
//   mass += bf16(P), peak = max u, Nmax = #(u == peak);
//   O_i = (sum_j bf16(P_ij) v_j) * gate_i / (mass_i + 1e-12), gate = peak/(peak + gamma).
// There is no running rescale (unlike softmax), so mass and peak stay lane-local for the
// whole key loop and are reduced across lanes once, in the epilogue.
//
// MFMA mapping: v_mfma_f32_16x16x32_bf16.  The forward and the dQ kernel compute S^T =
// K Q^T, whose C layout gives each lane one query row (lane % 16) and four keys per 16-key
// block.  The key order of the K fragment is permuted (perm_row below) so that the 8 keys a
// lane group holds after two blocks are contiguous: the C registers then feed the next
// MFMA (P^T or dS^T as its B operand) directly, and the A operand (V^T or K^T) is one
// 16-byte LDS read from a transposed tile.  The dK/dV kernel computes S = Q K^T with the
// same trick on the query axis.  MFMA results are bitwise transpose-symmetric on gfx950,
// so every kernel recomputes exactly the forward's scores; the peak-tie test u == M of
// the backward therefore sees the forward's ties.
//
// Backward (deterministic, no atomics): a per-row preprocess kernel forms the row
// constants (D_i = <dO_i, O_i>/g_i and the gate/normaliser factors); a query-parallel
// kernel accumulates dQ; a key-parallel kernel accumulates dK, dV and the tau partials;
// a one-block kernel sums the partials in fp64.  Both backward kernels skip the 32x64
// sub-tiles that the forward recorded as silent.
#include "flash.h"

namespace pnfx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Row of a 16-row MFMA block (block index blk, row r) inside its 64-row/key tile.
// Blocks 2t and 2t+1 interleave in groups of four so that lane group a (= r / 4) ends up
// holding rows 32t + 8a .. 32t + 8a + 7 across the pair.
__device__ __forceinline__ int perm_row(int blk, int r) {
  return 32 * (blk >> 1) + 8 * (r >> 2) + 4 * (blk & 1) + (r & 3);
}

__device__ __forceinline__ bf16x8 ld16(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// Stage rows [row0, row0 + ROWS) of a [N, D] slice (row stride sn) into LDS, row-major with
// row stride STR and zero padding up to DK columns and beyond N.
template <int ROWS, int D, int DK, int STR>
__device__ __forceinline__ void stage_rows(bf16* dst, const bf16* src, int64_t sn, int row0, int N,
                                           int tid) {
#pragma unroll
  for (int c = tid; c < ROWS * (DK / 8); c += 256) {
    const int row = c / (DK / 8), col = (c % (DK / 8)) * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row0 + row < N && col < D)
      v = *reinterpret_cast<const u32x4*>(src + (int64_t)(row0 + row) * sn + col);
    *reinterpret_cast<u32x4*>(dst + row * STR + col) = v;
  }
}

// Stage rows [row0, row0 + ROWS) transposed: dst[d * STR + row] (D rows of ROWS columns).
template <int ROWS, int D, int STR>
__device__ __forceinline__ void stage_rows_t(bf16* dst, const bf16* src, int64_t sn, int row0,
                                             int N, int tid) {
#pragma unroll
  for (int c = tid; c < (ROWS / 2) * (D / 8); c += 256) {
    const int rp = c % (ROWS / 2), col = (c / (ROWS / 2)) * 8;
    const int row = 2 * rp;
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (row0 + row < N) a = *reinterpret_cast<const u32x4*>(src + (int64_t)(row0 + row) * sn + col);
    if (row0 + row + 1 < N)
      b = *reinterpret_cast<const u32x4*>(src + (int64_t)(row0 + row + 1) * sn + col);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t lo = (e & 1) ? (a[e >> 1] >> 16) : (a[e >> 1] & 0xffffu);
      const uint32_t hi = (e & 1) ? (b[e >> 1] & 0xffff0000u) : (b[e >> 1] << 16);
      *reinterpret_cast<uint32_t*>(dst + (col + e) * STR + row) = lo | hi;
    }
  }
}

__device__ __forceinline__ float pow10f_(float u) {
  const float u2 = u * u;
  const float u4 = u2 * u2;
  return u4 * u4 * u2;
}

// Map a linear block id to (bh, block index) so that each XCD (block id % 8 on the
// round-robin dispatcher) works through a contiguous range of (b, h) slices -- their K/V
// stay in that XCD's L2 -- and, within a slice, the heaviest causal blocks go first.
__device__ __forceinline__ void map_block(int nblk, int BH, bool heavy_last_index, int& bh,
                                          int& blk) {
  const int total = nblk * BH;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  bh = L / nblk;
  const int j = L % nblk;
  blk = heavy_last_index ? nblk - 1 - j : j;
}

// ------------------------------------------------------------------------------ forward
template <int D, bool CAUSAL, bool HAS_GAMMA>
__global__ __launch_bounds__(256, 2) void flash_fwd_kernel(FwdParams p) {
  constexpr int BM = 128, BN = 64;
  constexpr int DK = D < 32 ? 32 : D;
  constexpr int KS = DK / 32;
  constexpr int DB = D / 16;
  constexpr int KSTR = DK + 8;
  constexpr int VSTR = BN + 8;
  __shared__ __attribute__((aligned(16))) bf16 Ks[BN * KSTR];
  __shared__ __attribute__((aligned(16))) bf16 Vt[D * VSTR];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r16 = lane & 15;
  const int N = p.N;
  const int nqb = (N + BM - 1) / BM;
  int bh, qblk;
  map_block(nqb, p.B * p.H, CAUSAL, bh, qblk);
  const int b = bh / p.H, h = bh % p.H;
  const bf16* Q = static_cast<const bf16*>(p.q) + b * p.qsb + h * p.qsh;
  const bf16* K = static_cast<const bf16*>(p.k) + b * p.ksb + h * p.ksh;
  const bf16* V = static_cast<const bf16*>(p.v) + b * p.vsb + h * p.vsh;
  const int m0 = qblk * BM;
  const int qrow0 = m0 + 32 * w;
  const bool has_rows = qrow0 < N;
  const float ntau = -p.tau[0];
  const float scale = p.scale;

  bf16x8 qf[2][KS];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = qrow0 + 16 * qb + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int col = 32 * ks + 8 * g;
      qf[qb][ks] = (row < N && col < D) ? ld16(Q + (int64_t)row * p.qsn + col) : zero_bf16x8();
    }
  }

  f32x4 acc[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) acc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The power mass is accumulated by the MFMA as one extra "dimension" of V whose value is
  // 1: a constant A fragment with ones in row 0.  The mass is then the sum of exactly the
  // bf16-rounded P that weights V, so O = gate * sum(P v) / sum(P) is a true convex
  // combination and the flash identity D = <dO, O>/gate holds for the P actually used.
  f32x4 accm[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  bf16x8 ones = zero_bf16x8();
  if (r16 == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (bf16)1.0f;
  }
  float mrun[2] = {0.f, 0.f};
  int cnt[2] = {0, 0};

  const int kv_end = CAUSAL ? min(m0 + BM, N) : N;
  const int ntiles = (kv_end + BN - 1) / BN;
  uint8_t* mrow =
      (p.mask && has_rows) ? p.mask + ((int64_t)bh * p.nq32 + (qrow0 >> 5)) * p.nk64 : nullptr;

  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * BN;
    __syncthreads();
    stage_rows<BN, D, DK, KSTR>(Ks, K, p.ksn, n0, N, tid);
    stage_rows_t<BN, D, VSTR>(Vt, V, p.vsn, n0, N, tid);
    __syncthreads();

    bool active = false;
    if (has_rows && !(CAUSAL && n0 > qrow0 + 31)) {
      f32x4 s[4][2];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const bf16* kr = Ks + perm_row(kb, r16) * KSTR + 8 * g;
        bf16x8 kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kf[ks] = ld16(kr + 32 * ks);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) a = mfma16x16x32(kf[ks], qf[qb][ks], a);
          s[kb][qb] = a;
        }
      }
      const bool diag = CAUSAL && (n0 + BN - 1 > qrow0);
      const bool edge = n0 + BN > N;
      bool any = false;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float sv = __builtin_fmaf(s[kb][qb][i], scale, ntau);
            float u = sv > 0.f ? sv : 0.f;
            if (diag || edge) {
              const int key = n0 + perm_row(kb, 4 * g + i);
              const int qrow = qrow0 + 16 * qb + r16;
              if ((CAUSAL && key > qrow) || key >= N) u = 0.f;
            }
            s[kb][qb][i] = u;
            any |= u > 0.f;
          }
      active = __any(any);
      if (active) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          float tm = 0.f;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) tm = fmaxf(tm, s[kb][qb][i]);
          const float mnew = fmaxf(mrun[qb], tm);
          int c = (mnew == mrun[qb]) ? cnt[qb] : 0;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) c += (s[kb][qb][i] == mnew) ? 1 : 0;
          cnt[qb] = c;
          mrun[qb] = mnew;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[kb][qb][i] = pow10f_(s[kb][qb][i]);
        }
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
          bf16x8 pf[2];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            pf[qb] = pack8(s[2 * tp][qb][0], s[2 * tp][qb][1], s[2 * tp][qb][2], s[2 * tp][qb][3],
                           s[2 * tp + 1][qb][0], s[2 * tp + 1][qb][1], s[2 * tp + 1][qb][2],
                           s[2 * tp + 1][qb][3]);
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const bf16x8 vf = ld16(Vt + (16 * db + r16) * VSTR + 32 * tp + 8 * g);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) acc[db][qb] = mfma16x16x32(vf, pf[qb], acc[db][qb]);
          }
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) accm[qb] = mfma16x16x32(ones, pf[qb], accm[qb]);
        }
      }
    }
    if (mrow && lane == 0) mrow[t] = active ? 1 : 0;
  }
  if (mrow && lane == 0)
    for (int t = ntiles; t < p.nk64; ++t) mrow[t] = 0;

  // Epilogue: reduce the lane-local statistics over the four lane groups of a row.
  bf16* O = static_cast<bf16*>(p.o) + b * p.osb + h * p.osh;
  bf16* Olo = p.o_lo ? static_cast<bf16*>(p.o_lo) + b * p.osb + h * p.osh : nullptr;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float m = mrun[qb];
    float Mx = fmaxf(m, __shfl_xor(m, 16, 64));
    Mx = fmaxf(Mx, __shfl_xor(Mx, 32, 64));
    int c = (m == Mx) ? cnt[qb] : 0;
    c += __shfl_xor(c, 16, 64);
    c += __shfl_xor(c, 32, 64);
    // row 0 of the mass block lives in lane r16 (lane group 0), register 0
    const float ms = __shfl(accm[qb][0], r16, 64);
    const float gate = Mx > 0.f ? (HAS_GAMMA ? Mx / (Mx + p.gamma) : 1.f) : 0.f;
    const float z = ms + 1e-12f;
    const float so = gate / z;
    const int qrow = qrow0 + 16 * qb + r16;
    if (qrow < N) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        bf16x4 o4, r4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float of = acc[db][qb][i] * so;
          o4[i] = (bf16)of;
          r4[i] = (bf16)(of - (float)o4[i]);
        }
        const int64_t off = (int64_t)qrow * p.osn + 16 * db + 4 * g;
        *reinterpret_cast<bf16x4*>(O + off) = o4;
        if (Olo) *reinterpret_cast<bf16x4*>(Olo + off) = r4;
      }
      if (g == 0) {
        const int64_t si = (int64_t)bh * N + qrow;
        p.M[si] = Mx;
        p.Z[si] = z;
        p.Nmax[si] = Mx > 0.f ? c : 0;
      }
    }
  }
}

// ------------------------------------------------------------------------------ backward
// Row constants: D_i = <dO_i, O_i> / g_i (the flash identity of src/triton_pnfirtau.py:575-577),
// r = g/Z, c = 10 g/Z * scale, G = D gamma/(M+gamma)^2 / Nmax * scale (zero on silent rows).
template <int D, bool HAS_GAMMA>
__global__ __launch_bounds__(256) void flash_bwd_pre_kernel(BwdParams p) {
  constexpr int LPR = D / 8;  // lanes per row
  constexpr int RPB = 256 / LPR;
  const int tid = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * RPB + tid / LPR;
  const int part = tid % LPR;
  const int64_t total = (int64_t)p.B * p.H * p.N;
  float dot = 0.f;
  int64_t bh = 0, i = 0;
  if (row < total) {
    bh = row / p.N;
    i = row % p.N;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t ooff = b * p.osb + h * p.osh + i * p.osn + 8 * part;
    const u32x4 ov = *reinterpret_cast<const u32x4*>(static_cast<const bf16*>(p.o) + ooff);
    u32x4 lv = {0u, 0u, 0u, 0u};
    if (p.o_lo) lv = *reinterpret_cast<const u32x4*>(static_cast<const bf16*>(p.o_lo) + ooff);
    const u32x4 dv =
        *reinterpret_cast<const u32x4*>(static_cast<const bf16*>(p.dout) + b * p.dosb + h * p.dosh + i * p.dosn + 8 * part);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float o0 = __uint_as_float(ov[e] << 16) + __uint_as_float(lv[e] << 16);
      const float o1 = __uint_as_float(ov[e] & 0xffff0000u) + __uint_as_float(lv[e] & 0xffff0000u);
      dot = __builtin_fmaf(o0, __uint_as_float(dv[e] << 16), dot);
      dot = __builtin_fmaf(o1, __uint_as_float(dv[e] & 0xffff0000u), dot);
    }
  }
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
  if (row < total && part == 0) {
    const float M = p.M[row], Z = p.Z[row];
    const float g = M > 0.f ? (HAS_GAMMA ? M / (M + p.gamma) : 1.f) : 0.f;
    const float Dv = g > 0.f ? dot / g : 0.f;
    float G = 0.f;
    if (HAS_GAMMA && M > 0.f) {
      const float dgate = p.gamma / ((M + p.gamma) * (M + p.gamma));
      G = Dv * dgate / (float)p.Nmax[row] * p.scale;
    }
    f32x4 c0 = {M, g / Z, 10.f * g / Z * p.scale, Dv};
    f32x4 c1 = {G, 0.f, 0.f, 0.f};
    reinterpret_cast<f32x4*>(p.rc)[2 * row] = c0;
    reinterpret_cast<f32x4*>(p.rc)[2 * row + 1] = c1;
  }
}

// dQ: query-parallel, same tiling as the forward (4 waves x 32 rows, 64-key tiles).
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_bwd_dq_kernel(BwdParams p) {
  constexpr int BM = 128, BN = 64;
  constexpr int DK = D < 32 ? 32 : D;
  constexpr int KS = DK / 32;
  constexpr int DB = D / 16;
  constexpr int KSTR = DK + 8;
  constexpr int TSTR = BN + 8;
  __shared__ __attribute__((aligned(16))) bf16 Ks[BN * KSTR];
  __shared__ __attribute__((aligned(16))) bf16 Vs[BN * KSTR];
  __shared__ __attribute__((aligned(16))) bf16 Kt[D * TSTR];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r16 = lane & 15;
  const int N = p.N;
  const int nqb = (N + BM - 1) / BM;
  int bh, qblk;
  map_block(nqb, p.B * p.H, CAUSAL, bh, qblk);
  const int b = bh / p.H, h = bh % p.H;
  const bf16* Q = static_cast<const bf16*>(p.q) + b * p.qsb + h * p.qsh;
  const bf16* K = static_cast<const bf16*>(p.k) + b * p.ksb + h * p.ksh;
  const bf16* V = static_cast<const bf16*>(p.v) + b * p.vsb + h * p.vsh;
  const bf16* dO = static_cast<const bf16*>(p.dout) + b * p.dosb + h * p.dosh;
  const int m0 = qblk * BM;
  const int qrow0 = m0 + 32 * w;
  const bool has_rows = qrow0 < N;
  const float ntau = -p.tau[0];
  const float scale = p.scale;

  bf16x8 qf[2][KS], dof[2][KS];
  float rM[2], rc[2], rD[2], rG[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = qrow0 + 16 * qb + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int col = 32 * ks + 8 * g;
      const bool ok = row < N && col < D;
      qf[qb][ks] = ok ? ld16(Q + (int64_t)row * p.qsn + col) : zero_bf16x8();
      dof[qb][ks] = ok ? ld16(dO + (int64_t)row * p.dosn + col) : zero_bf16x8();
    }
    f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    if (row < N) {
      c0 = reinterpret_cast<const f32x4*>(p.rc)[2 * ((int64_t)bh * N + row)];
      c1 = reinterpret_cast<const f32x4*>(p.rc)[2 * ((int64_t)bh * N + row) + 1];
    }
    rM[qb] = c0[0];
    rc[qb] = c0[2];
    rD[qb] = c0[3];
    rG[qb] = c1[0];
  }

  f32x4 acc[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) acc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kv_end = CAUSAL ? min(m0 + BM, N) : N;
  const int ntiles = (kv_end + BN - 1) / BN;
  const uint8_t* mrow =
      (p.mask && has_rows) ? p.mask + ((int64_t)bh * p.nq32 + (qrow0 >> 5)) * p.nk64 : nullptr;

  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * BN;
    __syncthreads();
    stage_rows<BN, D, DK, KSTR>(Ks, K, p.ksn, n0, N, tid);
    stage_rows<BN, D, DK, KSTR>(Vs, V, p.vsn, n0, N, tid);
    stage_rows_t<BN, D, TSTR>(Kt, K, p.ksn, n0, N, tid);
    __syncthreads();
    if (!has_rows || (CAUSAL && n0 > qrow0 + 31)) continue;
    if (mrow && mrow[t] == 0) continue;

    f32x4 s[4][2], dw[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int kr = perm_row(kb, r16) * KSTR + 8 * g;
      bf16x8 kf[KS], vf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[ks] = ld16(Ks + kr + 32 * ks);
        vf[ks] = ld16(Vs + kr + 32 * ks);
      }
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f}, c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          a = mfma16x16x32(kf[ks], qf[qb][ks], a);
          c = mfma16x16x32(vf[ks], dof[qb][ks], c);
        }
        s[kb][qb] = a;
        dw[kb][qb] = c;
      }
    }
    const bool diag = CAUSAL && (n0 + BN - 1 > qrow0);
    const bool edge = n0 + BN > N;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sv = __builtin_fmaf(s[kb][qb][i], scale, ntau);
          float u = sv > 0.f ? sv : 0.f;
          if (diag || edge) {
            const int key = n0 + perm_row(kb, 4 * g + i);
            const int qrow = qrow0 + 16 * qb + r16;
            if ((CAUSAL && key > qrow) || key >= N) u = 0.f;
          }
          const float u2 = u * u;
          const float u4 = u2 * u2;
          const float u9 = u4 * u4 * u;
          float ds = rc[qb] * u9 * (dw[kb][qb][i] - rD[qb]);
          if (u == rM[qb] && u > 0.f) ds += rG[qb];
          s[kb][qb][i] = ds;
        }
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {
      bf16x8 pf[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        pf[qb] = pack8(s[2 * tp][qb][0], s[2 * tp][qb][1], s[2 * tp][qb][2], s[2 * tp][qb][3],
                       s[2 * tp + 1][qb][0], s[2 * tp + 1][qb][1], s[2 * tp + 1][qb][2],
                       s[2 * tp + 1][qb][3]);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x8 kt = ld16(Kt + (16 * db + r16) * TSTR + 32 * tp + 8 * g);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) acc[db][qb] = mfma16x16x32(kt, pf[qb], acc[db][qb]);
      }
    }
  }

  bf16* dQ = static_cast<bf16*>(p.dq) + b * p.dqsb + h * p.dqsh;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qrow = qrow0 + 16 * qb + r16;
    if (qrow < N) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = (bf16)acc[db][qb][i];
        *reinterpret_cast<bf16x4*>(dQ + (int64_t)qrow * p.dqsn + 16 * db + 4 * g) = o4;
      }
    }
  }
}

// dK, dV and tau partials: key-parallel.  Each wave owns KPW keys (32 for D <= 64, 16 for
// D = 128) held as MFMA B fragments; the workgroup streams 64-row query tiles (Q, dO and
// their transposes, plus the row constants) through LDS from the causal diagonal down.
template <int D>
struct DkdvCfg {
  static constexpr int KPW = D <= 64 ? 32 : 16;
  static constexpr int KB = KPW / 16;
  static constexpr int BNK = 4 * KPW;
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_bwd_dkdv_kernel(BwdParams p) {
  constexpr int KPW = DkdvCfg<D>::KPW, KB = DkdvCfg<D>::KB, BNK = DkdvCfg<D>::BNK;
  constexpr int BMQ = 64;
  constexpr int DK = D < 32 ? 32 : D;
  constexpr int KS = DK / 32;
  constexpr int DB = D / 16;
  constexpr int QSTR = DK + 8;
  constexpr int TSTR = BMQ + 8;
  __shared__ __attribute__((aligned(16))) bf16 Qs[BMQ * QSTR];
  __shared__ __attribute__((aligned(16))) bf16 dOs[BMQ * QSTR];
  __shared__ __attribute__((aligned(16))) bf16 Qt[D * TSTR];
  __shared__ __attribute__((aligned(16))) bf16 dOt[D * TSTR];
  __shared__ __attribute__((aligned(16))) f32x4 RC[BMQ * 2];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, r16 = lane & 15;
  const int N = p.N;
  int bh, kvb;
  map_block(p.nkvb, p.B * p.H, false, bh, kvb);
  const int b = bh / p.H, h = bh % p.H;
  const bf16* Q = static_cast<const bf16*>(p.q) + b * p.qsb + h * p.qsh;
  const bf16* K = static_cast<const bf16*>(p.k) + b * p.ksb + h * p.ksh;
  const bf16* V = static_cast<const bf16*>(p.v) + b * p.vsb + h * p.vsh;
  const bf16* dO = static_cast<const bf16*>(p.dout) + b * p.dosb + h * p.dosh;
  const int kv0 = kvb * BNK;
  const int kw0 = kv0 + KPW * w;
  const bool has_keys = kw0 < N;
  const float ntau = -p.tau[0];
  const float scale = p.scale;

  bf16x8 kf[KB][KS], vf[KB][KS];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = kw0 + 16 * kb + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int col = 32 * ks + 8 * g;
      const bool ok = key < N && col < D;
      kf[kb][ks] = ok ? ld16(K + (int64_t)key * p.ksn + col) : zero_bf16x8();
      vf[kb][ks] = ok ? ld16(V + (int64_t)key * p.vsn + col) : zero_bf16x8();
    }
  }
  f32x4 adk[DB][KB], adv[DB][KB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      adk[db][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      adv[db][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  double dsum = 0.0;  // sum of ds; per-tile fp32 partials are added in fp64

  const int nqt = (N + BMQ - 1) / BMQ;
  const int qt0 = CAUSAL ? kv0 / BMQ : 0;
  const int ktile = kw0 >> 6;  // 64-key tile of this wave's keys (forward mask column)
  const uint8_t* mcol = (p.mask && has_keys) ? p.mask + (int64_t)bh * p.nq32 * p.nk64 + ktile : nullptr;

  for (int qt = qt0; qt < nqt; ++qt) {
    const int m0 = qt * BMQ;
    __syncthreads();
    stage_rows<BMQ, D, DK, QSTR>(Qs, Q, p.qsn, m0, N, tid);
    stage_rows<BMQ, D, DK, QSTR>(dOs, dO, p.dosn, m0, N, tid);
    stage_rows_t<BMQ, D, TSTR>(Qt, Q, p.qsn, m0, N, tid);
    stage_rows_t<BMQ, D, TSTR>(dOt, dO, p.dosn, m0, N, tid);
    if (tid < 2 * BMQ) {
      const int row = m0 + (tid >> 1);
      RC[tid] = row < N ? reinterpret_cast<const f32x4*>(p.rc)[2 * ((int64_t)bh * N + row) + (tid & 1)]
                        : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    if (!has_keys || (CAUSAL && m0 + BMQ - 1 < kw0)) continue;
    if (mcol) {
      const int r32 = m0 >> 5;
      const bool a0 = mcol[(int64_t)r32 * p.nk64] != 0;
      const bool a1 = (r32 + 1 < p.nq32) && mcol[(int64_t)(r32 + 1) * p.nk64] != 0;
      if (!a0 && !a1) continue;
    }

    f32x4 s[4][KB], dw[4][KB];
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
      const int qr = perm_row(qb, r16) * QSTR + 8 * g;
      bf16x8 qa[KS], da[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qa[ks] = ld16(Qs + qr + 32 * ks);
        da[ks] = ld16(dOs + qr + 32 * ks);
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f}, c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          a = mfma16x16x32(qa[ks], kf[kb][ks], a);
          c = mfma16x16x32(da[ks], vf[kb][ks], c);
        }
        s[qb][kb] = a;
        dw[qb][kb] = c;
      }
    }
    const bool diag = CAUSAL && (m0 < kw0 + KPW - 1);
    const bool edge = m0 + BMQ > N || kw0 + KPW > N;
    float tsum = 0.f;
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int lr = perm_row(qb, 4 * g + i);
        const f32x4 c0 = RC[2 * lr];
        const float rM = c0[0], rr = c0[1], rcoef = c0[2], rD = c0[3];
        const float rG = RC[2 * lr + 1][0];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const float sv = __builtin_fmaf(s[qb][kb][i], scale, ntau);
          float u = sv > 0.f ? sv : 0.f;
          if (diag || edge) {
            const int qrow = m0 + lr;
            const int key = kw0 + 16 * kb + r16;
            if ((CAUSAL && key > qrow) || key >= N || qrow >= N) u = 0.f;
          }
          const float u2 = u * u;
          const float u4 = u2 * u2;
          const float u8 = u4 * u4;
          const float u9 = u8 * u;
          s[qb][kb][i] = u8 * u2 * rr;  // w = P g / Z
          float ds = rcoef * u9 * (dw[qb][kb][i] - rD);
          if (u == rM && u > 0.f) ds += rG;
          dw[qb][kb][i] = ds;
          tsum += ds;
        }
      }
    }
    dsum += (double)tsum;
#pragma unroll
    for (int tp = 0; tp < 2; ++tp) {
      bf16x8 wf[KB], sf[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        wf[kb] = pack8(s[2 * tp][kb][0], s[2 * tp][kb][1], s[2 * tp][kb][2], s[2 * tp][kb][3],
                       s[2 * tp + 1][kb][0], s[2 * tp + 1][kb][1], s[2 * tp + 1][kb][2],
                       s[2 * tp + 1][kb][3]);
        sf[kb] = pack8(dw[2 * tp][kb][0], dw[2 * tp][kb][1], dw[2 * tp][kb][2], dw[2 * tp][kb][3],
                       dw[2 * tp + 1][kb][0], dw[2 * tp + 1][kb][1], dw[2 * tp + 1][kb][2],
                       dw[2 * tp + 1][kb][3]);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x8 ot = ld16(dOt + (16 * db + r16) * TSTR + 32 * tp + 8 * g);
        const bf16x8 qt_ = ld16(Qt + (16 * db + r16) * TSTR + 32 * tp + 8 * g);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          adv[db][kb] = mfma16x16x32(ot, wf[kb], adv[db][kb]);
          adk[db][kb] = mfma16x16x32(qt_, sf[kb], adk[db][kb]);
        }
      }
    }
  }

  bf16* dK = static_cast<bf16*>(p.dk) + b * p.dksb + h * p.dksh;
  bf16* dV = static_cast<bf16*>(p.dv) + b * p.dvsb + h * p.dvsh;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = kw0 + 16 * kb + r16;
    if (key < N) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        bf16x4 k4, v4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          k4[i] = (bf16)adk[db][kb][i];
          v4[i] = (bf16)adv[db][kb][i];
        }
        *reinterpret_cast<bf16x4*>(dK + (int64_t)key * p.dksn + 16 * db + 4 * g) = k4;
        *reinterpret_cast<bf16x4*>(dV + (int64_t)key * p.dvsn + 16 * db + 4 * g) = v4;
      }
    }
  }
  dsum = wave_sum_d(dsum);
  if (lane == 0) p.partials[((int64_t)bh * p.nkvb + kvb) * 4 + w] = dsum;
}

// dtau = -(sum of all ds partials) / scale, summed in fp64 by one block in a fixed order.
__global__ __launch_bounds__(256) void flash_dtau_kernel(const double* partials, int64_t n,
                                                         float scale, float* dtau) {
  __shared__ double red[256];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 256) acc += partials[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) dtau[0] = (float)(-red[0] / (double)scale);
}

template <int D>
int launch_fwd_d(const FwdParams& fp, bool causal, bool has_gamma, hipStream_t st) {
  const int nqb = (fp.N + 127) / 128;
  const dim3 grid((unsigned)(nqb * fp.B * fp.H)), block(256);
  if (causal) {
    if (has_gamma) hipLaunchKernelGGL((flash_fwd_kernel<D, true, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((flash_fwd_kernel<D, true, false>), grid, block, 0, st, fp);
  } else {
    if (has_gamma) hipLaunchKernelGGL((flash_fwd_kernel<D, false, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((flash_fwd_kernel<D, false, false>), grid, block, 0, st, fp);
  }
  return launch_status("pnfx_flash_fwd");
}

template <int D>
int launch_bwd_d(const BwdParams& bp, bool causal, bool has_gamma, int stages, hipStream_t st) {
  const dim3 block(256);
  if (stages & PNFX_BWD_PREPARE) {
    const int64_t rows = (int64_t)bp.B * bp.H * bp.N;
    const int rpb = 256 / (D / 8);
    const dim3 gpre((unsigned)((rows + rpb - 1) / rpb));
    if (has_gamma) hipLaunchKernelGGL((flash_bwd_pre_kernel<D, true>), gpre, block, 0, st, bp);
    else hipLaunchKernelGGL((flash_bwd_pre_kernel<D, false>), gpre, block, 0, st, bp);
    const int rc = launch_status("pnfx_flash_bwd(prepare)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DKDV) {
    const dim3 gkv((unsigned)(bp.nkvb * bp.B * bp.H));
    if (causal) hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, true>), gkv, block, 0, st, bp);
    else hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, false>), gkv, block, 0, st, bp);
    hipLaunchKernelGGL(flash_dtau_kernel, dim3(1), block, 0, st, bp.partials,
                       (int64_t)bp.B * bp.H * bp.nkvb * 4, bp.scale, bp.dtau);
    const int rc = launch_status("pnfx_flash_bwd(dkdv)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DQ) {
    const int nqb = (bp.N + 127) / 128;
    const dim3 gdq((unsigned)(nqb * bp.B * bp.H));
    if (causal) hipLaunchKernelGGL((flash_bwd_dq_kernel<D, true>), gdq, block, 0, st, bp);
    else hipLaunchKernelGGL((flash_bwd_dq_kernel<D, false>), gdq, block, 0, st, bp);
    const int rc = launch_status("pnfx_flash_bwd(dq)");
    if (rc) return rc;
  }
  return PNFX_OK;
}

}  // namespace

int64_t bwd_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t D) {
  const int64_t rc = B * H * N * 8 * 4;
  const int64_t parts = B * H * bwd_nkvb(N, D) * 4 * 8;
  return ((rc + 255) / 256) * 256 + ((parts + 255) / 256) * 256;
}

int flash_fwd_bf16(const FwdParams& fp, int64_t D, bool causal, bool has_gamma, hipStream_t st) {
  switch (D) {
    case 16: return launch_fwd_d<16>(fp, causal, has_gamma, st);
    case 32: return launch_fwd_d<32>(fp, causal, has_gamma, st);
    case 64: return launch_fwd_d<64>(fp, causal, has_gamma, st);
    case 128: return launch_fwd_d<128>(fp, causal, has_gamma, st);
  }
  set_error("flash: head dim %lld not in {16, 32, 64, 128}", (long long)D);
  return PNFX_EUNSUPPORTED;
}

int flash_bwd_bf16(const BwdParams& bp, int64_t D, bool causal, bool has_gamma, int stages,
                   hipStream_t st) {
  switch (D) {
    case 16: return launch_bwd_d<16>(bp, causal, has_gamma, stages, st);
    case 32: return launch_bwd_d<32>(bp, causal, has_gamma, stages, st);
    case 64: return launch_bwd_d<64>(bp, causal, has_gamma, stages, st);
    case 128: return launch_bwd_d<128>(bp, causal, has_gamma, stages, st);
  }
  set_error("flash: head dim %lld not in {16, 32, 64, 128}", (long long)D);
  return PNFX_EUNSUPPORTED;
}

}  // namespace pnfx
