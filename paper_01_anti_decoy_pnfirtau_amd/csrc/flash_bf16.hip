// Flash pn_fir_tau attention on bf16 MFMA (gfx950), forward and deterministic backward.
//
// Math (src/triton_pnfirtau.py:313-621): per query row i and key j <= i,
//   s = fma(q_i . k_j, scale, -tau), u = relu(s), P = u^10 (four multiplies, no exp),
//   mass += bf16(P), Z = sum P + 1e-12 (unrounded), peak = max u, Nmax = #(u == peak);
//   O_i = (sum_j bf16(P_ij) v_j) * gate_i / (mass_i + 1e-12), gate = peak/(peak + gamma).
// O is normalised by the mass of the rounded weights that multiply V (a true convex
// combination, so the flash identity of the backward holds for the weights actually used);
// the stored Z is the reference's unrounded sum, which the backward's gate/Z uses.
// There is no running rescale (unlike softmax), so mass and peak stay lane-local for the
// whole key loop and are reduced across lanes once, in the epilogue.
//
// MFMA mapping: v_mfma_f32_16x16x32_bf16.  The forward and the dQ kernel compute S^T =
// K Q^T, whose C layout gives each lane one query row (lane % 16) and four keys per 16-key
// block.  The key order of the K fragment is permuted (perm_row below) so that the 8 keys a
// lane group holds after two blocks are contiguous: the C registers then feed the next
// MFMA (P^T or dS^T as its B operand) directly, and the A operand (V^T or K^T) comes from
// the row-major tile through two transposing LDS reads.  The dK/dV kernel computes S = Q K^T with the
// same trick on the query axis.  MFMA results are bitwise transpose-symmetric on gfx950,
// so every kernel recomputes exactly the forward's scores; the peak-tie test u == M of
// the backward therefore sees the forward's ties.
//
// Backward (deterministic, no atomics), in this order: a per-row preprocess kernel forms the
// row constants (D_i = <dO_i, O_i>/g_i and the gate/normaliser factors); a query-parallel
// kernel accumulates dQ and the tau partials and counts the peak ties; a key-parallel kernel
// accumulates dK and dV, and one of its workgroups sums the tau partials in fp64.  Both
// gradient kernels skip the 32x64 sub-tiles that the forward recorded as silent.
#include <cmath>

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

// LDS tiles are unpadded and XOR-swizzled on the 16-byte chunk index of each row, with
// swizzles linear over GF(2) in the row bits.  They were chosen by measuring the LDS
// bank-conflict counter for every access pattern of the kernels (a b128 read is conflict
// free when each 16-lane group reads 16 consecutive tile rows at chunks g ^ swz(row)):
//  * tiles are row-major [rows][DK] and store logical row R at slot slot_of(R), which places
//    the 16 rows of an MFMA fragment (rows perm_row(blk, 0..15)) in consecutive slots
//    16 blk .. 16 blk + 15;
//  * the transposed operands (V^T, K^T, Q^T, dO^T) are read from the same row-major tiles
//    with ds_read_tr16_b64, which transposes 16-bit elements across each 16-lane group.
// Linearity lets a fragment's swizzle split into a per-lane part and a compile-time part.
__device__ __forceinline__ constexpr int parity6(int x) { return __builtin_popcount(x & 63) & 1; }
__device__ __forceinline__ constexpr int swz_cols(int d) {
  return parity6(d & 18) | (parity6(d & 39) << 1) | (parity6(d & 12) << 2);
}
// Row-major tiles: 64-column rows use swz_cols; 128-column rows (16 chunks) a 4-bit swizzle.
template <int DK>
__device__ __forceinline__ constexpr int swz_rt(int slot) {
  return DK == 128 ? (parity6(slot & 46) | (parity6(slot & 10) << 1) | (parity6(slot & 28) << 2) |
                      (parity6(slot & 13) << 3))
                   : swz_cols(slot) & (DK / 8 - 1);
}
// Slot of logical row R: rows perm_row(blk, r) -> 16 blk + r.
__device__ __forceinline__ constexpr int slot_of(int R) {
  return 16 * (2 * (R >> 5) + ((R >> 2) & 1)) + 4 * ((R >> 3) & 3) + (R & 3);
}

// Element offset of 16-byte chunk `chunk` of logical row `row` in a row-major tile of DK
// columns.
template <int DK>
__device__ __forceinline__ int rt_off(int row, int chunk) {
  const int slot = slot_of(row);
  return slot * DK + ((chunk ^ swz_rt<DK>(slot)) << 3);
}
// Fragment addressing with the lane part hoisted.  A row-major fragment reads logical row
// perm_row(blk, r16), i.e. slot 16 blk + r16 (disjoint bits), at chunk g + 4*ks:
//   offset = 16 blk DK + r16 DK + (((g ^ swz(r16)) ^ (4 ks ^ swz(16 blk))) << 3).
struct FragLane {
  int rbase;  // lane part of the element offset
  int x;      // lane part of the chunk index (XOR-combined with the constant part)
};
template <int DK>
__device__ __forceinline__ FragLane rt_lane(int r16, int g) {
  return FragLane{r16 * DK, g ^ swz_rt<DK>(r16)};
}
template <int DK>
__device__ __forceinline__ int rt_frag(const FragLane& fl, int blk, int ks) {
  const int cc = (4 * ks) ^ swz_rt<DK>(16 * blk);
  return 16 * blk * DK + fl.rbase + ((fl.x ^ cc) << 3);
}

// Transposed fragment X^T[16 db + r16][rows 32 hf + 8 g + t], t = 0..7 (the A operand of the
// second GEMM: V^T, K^T, Q^T or dO^T) from a row-major tile, as two ds_read_tr16_b64.  In
// each 16-lane group, lane 4 e + q addresses row 32 hf + 8 g + 4 u + e at columns
// 16 db + 4 q .. + 3 (u = 0, 1 for the two reads), and lane r16 = 4 q' + r' receives
// column 16 db + r16 of the four rows addressed by lanes 4 e + q'.  Row 32 hf + 8 g + 4 u + e
// sits in slot 16 (2 hf + u) + 4 g + e.
template <int DK>
__device__ __forceinline__ FragLane tr_lane(int lane) {
  const int g = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
  const int sl = 4 * g + e;
  return FragLane{sl * DK + 4 * (q & 1), (q >> 1) ^ swz_rt<DK>(sl)};
}
__device__ __forceinline__ bf16x4 ld_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)(p));
}
template <int DK>
__device__ __forceinline__ bf16x8 tr_frag(const bf16* tile, const FragLane& fl, int hf, int db) {
  bf16x4 h[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int sc = 16 * (2 * hf + u);
    const int cc = (2 * db) ^ swz_rt<DK>(sc);
    h[u] = ld_tr(tile + sc * DK + fl.rbase + ((fl.x ^ cc) << 3));
  }
  return __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7);
}

// Direct global -> LDS staging of a 64-row tile (rows row0 .. row0 + 63 of an [N, D] bf16
// slice with row stride sn) into the swizzled row-major layout, with global_load_lds_dwordx4:
// no register staging and no LDS store instructions.  Each such load writes 16 bytes per
// lane to LDS at (wave-uniform base) + 16 * lane, so a wave fills 64 consecutive chunks; each
// lane loads the global chunk that belongs at its position (the layout is a permutation of
// the tile's chunks).  The per-lane row and column are fixed at construction.  Rows >= N
// re-load row N - 1 and the padding chunks of D < DK re-load a real chunk of the row: both
// only ever meet masked scores or zero MFMA operands, so any finite value serves.  The
// caller waits for the loads (vmcnt) before the barrier that publishes the tile.
// Direct global -> LDS copy of 16 bytes per lane (lane l lands at dst + 8 l).  (The builtin
// sits in a plain function: called directly from a class template's member, it kept the
// host pass from emitting some of the kernels' launch stubs.)
__device__ __forceinline__ void lds_dma16(const bf16* src, bf16* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}
__device__ __forceinline__ int row_of_slot(int s) {  // inverse of slot_of
  return (s & 32) | ((s & 12) << 1) | ((s >> 2) & 4) | (s & 3);
}
template <int D, int DK>
struct TileDma {
  static constexpr int CPR = DK / 8;      // 16-byte chunks per tile row
  static constexpr int NI = 64 * CPR / 256;  // loads per thread
  int row[NI], col[NI];
  unsigned off[NI];  // byte offset of the lane's chunks from the tile's first row
  __device__ __forceinline__ TileDma(int w, int lane, int64_t sn) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int L = (4 * j + w) * 64 + lane;  // chunk index in the tile
      const int slot = L / CPR, pos = L % CPR;
      const int ch = pos ^ swz_rt<DK>(slot);
      row[j] = row_of_slot(slot);
      col[j] = 8 * (ch % (D / 8));
      off[j] = (unsigned)(2 * (row[j] * sn + col[j]));
    }
  }
  // A whole tile (row0 + 64 <= N) is a wave-uniform base plus 32-bit lane offsets, which the
  // load takes as scalar base + vector offset: no per-load address arithmetic.
  __device__ __forceinline__ void load(const bf16* src, int64_t sn, int row0, int N, bf16* tile,
                                       int w) const {
    if (row0 + 64 <= N) {
      const char* base = reinterpret_cast<const char*>(src + (int64_t)row0 * sn);
#pragma unroll
      for (int j = 0; j < NI; ++j)
        lds_dma16(reinterpret_cast<const bf16*>(base + off[j]), tile + (4 * j + w) * 512);
    } else {
      load_clamped(src, sn, row0, N, tile, w);
    }
  }
  // Any tile, from the row and column alone (fewer registers held across the loop, more
  // address arithmetic per load).
  __device__ __forceinline__ void load_clamped(const bf16* src, int64_t sn, int row0, int N,
                                               bf16* tile, int w) const {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int r = min(row0 + row[j], N - 1);
      lds_dma16(src + (int64_t)r * sn + col[j], tile + (4 * j + w) * 512);
    }
  }
};
// Direct global -> LDS copy of 4 bytes per lane (lane l lands at dst + l).
__device__ __forceinline__ void lds_dma4(const float* src, float* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 4, 0, 0);
}
// One LDS buffer of the forward and dQ kernels: a key tile of K and V (and, for the forward
// with the FIR fused into its key-tile load, the tile's raw key rows).
struct KVBuf {
  bf16* k;
  bf16* v;
  bf16* kr = nullptr;
};

// One LDS buffer of the dK/dV kernel: a query tile of Q (for D <= 64 scaled by 2^-e per row)
// and dO, and its row-constant planes.
struct QBuf {
  bf16* q;
  bf16* o;
  float* rc;  // [planes][64 rows]
};

// Wait for this wave's outstanding global loads (including direct-to-LDS ones).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Multiply the 8 bf16 values of a fragment by an exact power of two (no rounding).
__device__ __forceinline__ bf16x8 scale_frag(bf16x8 v, float s) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (bf16)((float)v[e] * s);
  return v;
}

// max(x, 0) of an MFMA result in one VALU op.  fmaxf would first canonicalize the operand
// (an extra op per element: the compiler cannot prove an MFMA accumulator free of
// signalling NaNs).  On the bit pattern, every negative float (and -0) is a negative
// int32, so a signed integer max with 0 is relu.  (Not inline asm: the compiler does not
// insert the MFMA-result wait states in front of an asm statement.)
__device__ __forceinline__ float relu_mfma(float x) {
  return __builtin_bit_cast(float, max(__builtin_bit_cast(int, x), 0));
}

__device__ __forceinline__ float pow10f_(float u) {
  const float u2 = u * u;
  const float u4 = u2 * u2;
  return u4 * u4 * u2;
}

// Map a linear block id to (bh, block index).  Each XCD (block id % 8 on the round-robin
// dispatcher) works through a contiguous range of (b, h) slices, so their K/V (forward, dQ)
// or Q/dO (dK/dV) tiles stay in that XCD's L2.  Within the range, slices go in pairs, and a
// pair's blocks are dispatched heaviest first across both slices: causal blocks range from
// one tile of work to N/64, and ordering them one slice at a time leaves the last slice's
// heavy blocks to start late and run alone.  Measured at C4 against one slice at a time:
// forward -3 %, dQ -4 %, dK/dV -2 % (-9 % with silent key tiles), for 20-25 % more L2
// misses; groups of four gain another 1-3 % on the forward only, at 2-3x the misses.
__device__ __forceinline__ void map_block(int nblk, int BH, bool heavy_last_index, int& bh,
                                          int& blk) {
  constexpr int G = 2;
  const int total = nblk * BH;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int c = L / (G * nblk), r = L % (G * nblk);
  const int ge = min(G, BH - c * G);  // the last group may hold fewer slices
  bh = c * G + r % ge;
  const int j = r / ge;
  blk = heavy_last_index ? nblk - 1 - j : j;
}

// ------------------------------------------------------------------------------ forward
// s -> u = relu(fma(s, scale, -tau)) in place for the 16 scores a lane holds in one 32-key
// half tile (S^T layout: key blocks 2*hf, 2*hf+1 x 2 query blocks x 4), zeroing keys past
// the causal diagonal or N when MASK; returns the lane's per-query-row maximum in tm.
// PS: the score scale is a power of two folded into the register-resident operand and -tau
// into the MFMA accumulator, so s already holds q.k*scale - tau.
// Scores in the key-major layout S^T (register i of lane group g holds key
// perm_row(blk, 4g+i), lane r16 holds query 16qb+r16).  Without the scale fold, the scores
// are first mapped to s*scale - tau (PS: the MFMA already produced that).
template <bool PS, int QB>
__device__ __forceinline__ void affine_kq(f32x4 (&s)[2][QB], float scale, float ntau) {
  if (PS) return;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[kk][qb][i] = __builtin_fmaf(s[kk][qb][i], scale, ntau);
}

// affine_kq with a scale and -tau per query block (the lane's row): the dQ kernel's
// peak-normalised scores.
template <bool PS, int QB>
__device__ __forceinline__ void affine_kq_rows(f32x4 (&s)[2][QB], const float (&scale)[QB],
                                               const float (&ntau)[QB]) {
  if (PS) return;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[kk][qb][i] = __builtin_fmaf(s[kk][qb][i], scale[qb], ntau[qb]);
}

// Causal and sequence-end mask, in place: entries outside it become -1, which the rectifier
// maps to 0.  Only tiles that straddle the diagonal or the sequence end run it, so the
// common tile's score code has no mask operations and no second copy.
template <int QB>
__device__ __forceinline__ void mask_kq(f32x4 (&s)[2][QB], int n0, int hf, int qrow0, int N,
                                        bool causal, int g, int r16) {
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = n0 + perm_row(2 * hf + kk, 4 * g + i);
        const int qrow = qrow0 + 16 * qb + r16;
        if ((causal && key > qrow) || key >= N) s[kk][qb][i] = -1.f;
      }
}

// Rectify in place and take each query's lane-local maximum.
__device__ __forceinline__ void rectify_kq(f32x4 (&s)[2][2], float (&tm)[2]) {
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float mx = 0.f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float u = relu_mfma(s[kk][qb][i]);
        s[kk][qb][i] = u;
        mx = fmaxf(mx, u);
      }
    tm[qb] = mx;
  }
}

// Silent-tile bound.  Every score of a (query, key) pair is at most |q| |k| |scale| - tau
// (Cauchy-Schwarz), so a tile whose largest query norm times largest key norm times |scale|
// is <= tau has no positive rectified score.  The MFMA's own rounding and that of the norms
// are far below the 2^-8 margin, so the test never drops an active tile.  The key side is
// one norm per 64-key tile, from this pass; the query side is formed by each forward wave.
constexpr float kBoundMargin = 1.f + 1.f / 256.f;
constexpr int kMaxBoundTiles = 1024;  // N <= 65536

// Largest key norm of each 64-key tile (one wave per tile, one key per lane).  With tau <= 0
// no tile can be bounded silent (tau = 0 with an all-zero tile aside), and K is not read.
template <int D>
__global__ __launch_bounds__(256) void flash_key_norm_kernel(FwdParams p) {
  const int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (tile >= (int64_t)p.B * p.H * p.nk64) return;
  if (!(p.tau[0] > 0.f)) {
    if (lane == 0) p.knorm[tile] = __builtin_inff();
    return;
  }
  const int bh = (int)(tile / p.nk64), t = (int)(tile % p.nk64);
  const int key = t * 64 + lane;
  float ss = 0.f;
  if (key < p.N) {
    const bf16* row = static_cast<const bf16*>(p.k) + (int64_t)(bh / p.H) * p.ksb +
                      (int64_t)(bh % p.H) * p.ksh + (int64_t)key * p.ksn;
#pragma unroll
    for (int c = 0; c < D; c += 8) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(row + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(v[e] << 16), hi = __uint_as_float(v[e] & 0xffff0000u);
        ss = __builtin_fmaf(lo, lo, ss);
        ss = __builtin_fmaf(hi, hi, ss);
      }
    }
  }
  ss = wave_max(ss);
  if (lane == 0) p.knorm[tile] = sqrtf(ss);
}

// Each query row's maximum of u = relu(s) is max(0, max s): an integer max from 0 over the
// raw bit patterns (positive floats order as their bits; negative ones are negative
// integers), so the silent-half test needs no rectified copy of the scores.
// Bit patterns through by-value helpers: clang's __builtin_bit_cast applied directly to an
// ext_vector element (v[i]) reads element 0 whatever i is.
__device__ __forceinline__ int f2i(float x) { return __builtin_bit_cast(int, x); }
__device__ __forceinline__ float i2f(int x) { return __builtin_bit_cast(float, x); }

__device__ __forceinline__ void row_max_kq(const f32x4 (&s)[2][2], float (&tm)[2]) {
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int mx = 0;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = max(mx, f2i(s[kk][qb][i]));
    tm[qb] = i2f(mx);
  }
}
// max of two non-negative floats as an integer max (no canonicalising operand copies)
__device__ __forceinline__ float max_nonneg(float a, float b) {
  return __builtin_bit_cast(float, max(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b)));
}

// Longest compacted key-tile list of the forward kernel (N <= 65536).
constexpr int kMaxListTiles = 1024;

// COUNT: also count the peak ties (Nmax); the training path leaves that to the backward.
// FIRK (D <= 64): p.k holds the raw keys, and each key tile is filtered in LDS (the causal
// FIR of pnfx_fir_fwd, fused into the key-tile load) before its scores; see
// pnfx_flash_fwd_fir.
template <int D, bool CAUSAL, bool PS, bool COUNT, bool FIRK = false>
__global__ __launch_bounds__(256, D <= 64 && !FIRK ? 3 : 2) void flash_fwd_kernel(FwdParams p) {
  constexpr int BM = 128, BN = 64;
  constexpr bool BOUND = D <= 64 && !FIRK;  // the silent-tile bound (see flash_key_norm_kernel)
  constexpr int DK = D < 32 ? 32 : D;
  constexpr int KS = DK / 32;
  constexpr int DB = D / 16;
  static_assert(!FIRK || D <= 64, "the fused FIR is built for d <= 64");
  // Two K/V tile buffers as separate LDS objects (see the dK/dV kernel), filled straight
  // from global memory.
  __shared__ __attribute__((aligned(16))) bf16 Ks0[BN * DK];
  __shared__ __attribute__((aligned(16))) bf16 Vs0[BN * DK];
  __shared__ __attribute__((aligned(16))) bf16 Ks1[BN * DK];
  __shared__ __attribute__((aligned(16))) bf16 Vs1[BN * DK];
  // FIRK: the raw key rows n0 - 8 .. n0 + 63 of each tile, row-major [72][D]
  constexpr int KR_ROWS = 72;
  constexpr int KCPR = D / 8;  // 16-byte chunks per raw key row
  __shared__ __attribute__((aligned(16))) bf16 Kr0[FIRK ? KR_ROWS * D : 8];
  __shared__ __attribute__((aligned(16))) bf16 Kr1[FIRK ? KR_ROWS * D : 8];
  const KVBuf buf0{Ks0, Vs0, Kr0}, buf1{Ks1, Vs1, Kr1};

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, provably uniform
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
  const FragLane flr = rt_lane<DK>(r16, g), flt = tr_lane<DK>(lane);

  // The silent-tile bound applies (key norms given, tau > 0: at tau <= 0 no tile but an
  // all-zero one can be bounded silent, and the kernel then runs without it).
  const bool bound = BOUND && p.knorm && p.nk64 <= kMaxBoundTiles && ntau < 0.f;
  bf16x8 qf[2][KS];
  // Largest squared query norm of the wave's rows: the diagonal of the 16x16 Gram blocks
  // Q Q^T, formed by the MFMA from the bf16 rows (exact products, fp32 sums).
  float qss = 0.f;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = qrow0 + 16 * qb + r16;
    f32x4 gram = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int col = 32 * ks + 8 * g;
      qf[qb][ks] = (row < N && col < D) ? ld16(Q + (int64_t)row * p.qsn + col) : zero_bf16x8();
      if (bound) gram = mfma16x16x32(qf[qb][ks], qf[qb][ks], gram);
      if (PS) qf[qb][ks] = scale_frag(qf[qb][ks], scale);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * g + i == r16) qss = fmaxf(qss, gram[i]);  // element (r16, r16)
  }
  const f32x4 s_init = PS ? f32x4{ntau, ntau, ntau, ntau} : f32x4{0.f, 0.f, 0.f, 0.f};

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
  // The unrounded mass sum P in fp32, the reference's normaliser (src/triton_pnfirtau.py:405):
  // the stored Z, from which the backward forms x = gate/Z.  O itself is normalised by the
  // MFMA mass of the rounded P above.
  float zf[2] = {0.f, 0.f};

  const int kv_end = CAUSAL ? min(m0 + BM, N) : N;
  const int ntiles = (kv_end + BN - 1) / BN;
  uint8_t* mrow =
      (p.mask && has_rows) ? p.mask + ((int64_t)bh * p.nq32 + (qrow0 >> 5)) * p.nk64 : nullptr;

  // Silent-tile bound (with the key norms): the wave's and the workgroup's largest query
  // norm times scale, with the margin; tile t is silent for them when that times the tile's
  // key norm is <= tau.  A tile silent for the workgroup is not loaded either.
  // The tile norms are staged in LDS once (their global loads could not be scalar loads in
  // the loop, which stores the mask bytes); sequences with more than kMaxBoundTiles key
  // tiles do without the bound, and so does D = 128, whose registers are all taken (the
  // bound's few values made it spill inside the tile loop).
  const float tau = -ntau;
  float qb_w = 0.f, qb_wg = 0.f;
  __shared__ float qss_s[4];
  __shared__ float kn_s[BOUND ? kMaxBoundTiles : 1];
  const float* kn = kn_s;
  if (bound) {
    for (int i = tid; i < ntiles; i += 256) kn_s[i] = p.knorm[(int64_t)bh * p.nk64 + i];
    qss = wave_max(qss);
    // |scale|: with a negative scale the bound is |q| |k| |scale| - tau just the same
    qb_w = sqrtf(qss) * fabsf(scale) * kBoundMargin;
    if (lane == 0) qss_s[w] = qss;
    __syncthreads();
    qb_wg = sqrtf(fmaxf(fmaxf(qss_s[0], qss_s[1]), fmaxf(qss_s[2], qss_s[3]))) * fabsf(scale) *
            kBoundMargin;
    // wave-uniform: keep them in scalar registers
    qb_w = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, qb_w)));
    qb_wg = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, qb_wg)));
  }
  // With the bound, the key loop runs over the tiles the workgroup cannot bound silent only,
  // compacted into a list (no load, barrier or mask lookup for the others); the mask bytes of
  // the skipped tiles are written here, the loop writes the rest.
  __shared__ uint16_t tl_s[BOUND ? kMaxListTiles : 1];
  int nlist = ntiles;
  if (bound) {
    // every wave forms the ballots (and zeroes its own skipped mask bytes); wave 0 writes the
    // list
    int base = 0;
    for (int c = 0; c < p.nk64; c += 64) {
      const int t = c + lane;
      const bool f = t < ntiles && !(qb_wg * kn[t] <= tau);
      if (!f && mrow && t < p.nk64) mrow[t] = 0;
      const uint64_t bal = __ballot(f);
      if (w == 0 && f) tl_s[base + __popcll(bal & ((1ull << lane) - 1ull))] = (uint16_t)t;
      base += __popcll(bal);
    }
    nlist = base;
    __syncthreads();
  } else if (mrow) {
    for (int t = ntiles + lane; t < p.nk64; t += 64) mrow[t] = 0;
  }
  const bool ident = nlist == ntiles;  // nothing skipped: the list is 0, 1, 2, ...
  // Entry e of the list (read into a scalar register: tile addresses stay scalar bases for
  // the tile loads); the identity list is not read at all, so the loop without the bound runs
  // as if there were no list.
  const auto tile_at = [&](int e) {
    return ident ? e : __builtin_amdgcn_readfirstlane((int)tl_s[min(e, nlist - 1)]);
  };

  // Software pipeline: tile t+1 streams from HBM/L2 straight into one LDS buffer while tile
  // t is computed from the other; one barrier per tile.
  const TileDma<D, DK> kdma(w, lane, p.ksn), vdma(w, lane, p.vsn);
  auto load_tile = [&](int n, const KVBuf& bb) {
    if constexpr (FIRK) {
      // raw rows n - 8 .. n + 63, KCPR chunks each (72 KCPR chunks, 64 per wave and load);
      // rows outside [0, N) re-load a real row (the filter skips rows before 0, and keys past
      // N are masked)
#pragma unroll
      for (int j = 0; j < (KR_ROWS * KCPR + 255) / 256; ++j) {
        const int L0 = j * 256 + w * 64;  // wave-uniform
        if (L0 >= KR_ROWS * KCPR) break;
        // each active lane lands 16 bytes at (its wave's base) + 16 lane: lanes past the last
        // chunk stay inactive, so nothing lands beyond the buffer
        const int L = L0 + lane;
        if (L < KR_ROWS * KCPR) {
          const int r = min(max(n - 8 + L / KCPR, 0), N - 1);
          lds_dma16(K + (int64_t)r * p.ksn + 8 * (L % KCPR), bb.kr + L0 * 8);
        }
      }
    } else {
      kdma.load(K, p.ksn, n, N, bb.k, w);
    }
    vdma.load(V, p.vsn, n, N, bb.v, w);
  };
  // FIRK: the filter taps of this head, h[u] = taps[K - 1 - u] (scalar registers)
  float fh[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (FIRK) {
    const float* tp = p.fir_taps + (p.fir_taps_rows == 1 ? 0 : h) * p.fir_k;
#pragma unroll
    for (int u = 0; u < 7; ++u) fh[u] = u < p.fir_k ? tp[p.fir_k - 1 - u] : 0.f;
  }
  // FIRK: the filtered key tile n0 .. n0 + 63 formed in bc.k from the raw rows in bc.kr, with
  // pnfx_fir_fwd's arithmetic (an fp32 FMA chain in lag order, one bf16 rounding): thread tid
  // forms FRT consecutive rows from r0 = FRT (tid / KCPR) of chunk tid % KCPR (two rows at
  // D = 64, one at D = 32; at D = 16 the first 128 threads one row each).
  constexpr int FRT = KCPR >= 8 ? 2 : 1;
  constexpr int FTHREADS = 64 * KCPR / FRT;
  auto filter_tile = [&](int n0, const KVBuf& bc) {
    if (tid >= FTHREADS) return;
    const int c = tid % KCPR, r0 = FRT * (tid / KCPR);
    u32x4 x[FRT + 6];  // raw rows n0 + r0 - 6 .. n0 + r0 + FRT - 1
#pragma unroll
    for (int i = 0; i < FRT + 6; ++i)
      x[i] = *reinterpret_cast<const u32x4*>(bc.kr + (r0 + 2 + i) * D + 8 * c);
    const auto elem = [](const u32x4& v, int e) {
      const uint32_t d = v[e >> 1];
      return __uint_as_float((e & 1) ? (d & 0xffff0000u) : (d << 16));
    };
#pragma unroll
    for (int o = 0; o < FRT; ++o) {
      const int n = n0 + r0 + o;
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = elem(x[o + 6], e) * fh[0];
#pragma unroll
      for (int u = 1; u < 7; ++u)
        if (u < p.fir_k && n - u >= 0)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(elem(x[o + 6 - u], e), fh[u], acc[e]);
      bf16x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (bf16)acc[e];
      *reinterpret_cast<bf16x8*>(bc.k + rt_off<DK>(r0 + o, c)) = y;
    }
  };
  // FIRK, D < DK (D = 16): the K tiles' padding chunks meet only zero Q fragments but must hold
  // finite values; the filter never writes them, so they are zeroed once here (published by
  // the first tile's barrier).
  if constexpr (FIRK && D < DK) {
    for (int i = tid; i < 2 * 64 * (DK - D) / 8; i += 256) {
      const int bsel = i / (64 * (DK - D) / 8), j = i % (64 * (DK - D) / 8);
      const int row = j / ((DK - D) / 8), c = KCPR + j % ((DK - D) / 8);
      *reinterpret_cast<bf16x8*>((bsel ? buf1.k : buf0.k) + rt_off<DK>(row, c)) = zero_bf16x8();
    }
  }
  // Entry e of the list: tile t, computed from buffer bc while the next entry's tile tn
  // streams into buffer bn.
  auto step = [&](int e, const KVBuf& bc, const KVBuf& bn) {
    int t = e, tn = e + 1;
    if (!ident) {
      t = tile_at(e);
      tn = tile_at(e + 1);
    }
    const int n0 = t * BN;
    wait_vmem();  // this wave's part of tile t is in LDS
    __syncthreads();
    if (e + 1 < nlist) load_tile(tn * BN, bn);
    if constexpr (FIRK) {  // the filtered tile, published by a second barrier
      filter_tile(n0, bc);
      __syncthreads();
    }
    // the wave's own bound (the tile norm is wave-uniform: a scalar register)
    const bool bounded = bound && qb_w * i2f(__builtin_amdgcn_readfirstlane(f2i(kn[t]))) <= tau;
    bool active = false;
    if (has_rows && !bounded && !(CAUSAL && n0 > qrow0 + 31)) {
      const bf16* Kc = bc.k;
      const bf16* Vc = bc.v;
      const bool masked = (CAUSAL && n0 + BN - 1 > qrow0) || n0 + BN > N;
      // Two 32-key halves: each half's scores are exactly one k-step of the P.V MFMA.
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        if (CAUSAL && n0 + 32 * hf > qrow0 + 31) break;  // half entirely above the diagonal
        f32x4 s[2][2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          bf16x8 kf[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) kf[ks] = ld16(Kc + rt_frag<DK>(flr, 2 * hf + kk, ks));
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            f32x4 a4 = s_init;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) a4 = mfma16x16x32(kf[ks], qf[qb][ks], a4);
            s[kk][qb] = a4;
          }
        }
        float tm[2];
        affine_kq<PS>(s, scale, ntau);
        if (masked) mask_kq(s, n0, hf, qrow0, N, CAUSAL, g, r16);
        if constexpr (COUNT) rectify_kq(s, tm);
        else row_max_kq(s, tm);
        if (!__any(max_nonneg(tm[0], tm[1]) > 0.f)) continue;  // silent half: skip P and P.V
        active = true;
        bf16x8 pf[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float mnew = max_nonneg(mrun[qb], tm[qb]);
          if (COUNT) {
            int c = (mnew == mrun[qb]) ? cnt[qb] : 0;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
              for (int i = 0; i < 4; ++i) c += (s[kk][qb][i] == mnew) ? 1 : 0;
            cnt[qb] = c;
          }
          mrun[qb] = mnew;
          // P = u^10 (u = relu(s); COUNT has rectified s already), summed unrounded into zf
          float pw[2][4];
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float u = COUNT ? s[kk][qb][i] : relu_mfma(s[kk][qb][i]);
              pw[kk][i] = pow10f_(u);
              zf[qb] += pw[kk][i];
            }
          pf[qb] = pack8(pw[0][0], pw[0][1], pw[0][2], pw[0][3], pw[1][0], pw[1][1], pw[1][2],
                         pw[1][3]);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 vf = tr_frag<DK>(Vc, flt, hf, db);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) acc[db][qb] = mfma16x16x32(vf, pf[qb], acc[db][qb]);
        }
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) accm[qb] = mfma16x16x32(ones, pf[qb], accm[qb]);
      }
      active = __any(active);
    }
    if (mrow && lane == 0) mrow[t] = active ? 1 : 0;
  };
  if (nlist > 0) load_tile(tile_at(0) * BN, buf0);
  for (int e = 0; e < nlist; e += 2) {
    step(e, buf0, buf1);
    if (e + 1 < nlist) step(e + 1, buf1, buf0);
  }

  // Epilogue: reduce the lane-local statistics over the four lane groups of a row.
  bf16* O = static_cast<bf16*>(p.o) + b * p.osb + h * p.osh;
  bf16* Olo = p.o_lo ? static_cast<bf16*>(p.o_lo) + b * p.osb + h * p.osh : nullptr;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float m = mrun[qb];
    float Mx = fmaxf(m, __shfl_xor(m, 16, 64));
    Mx = fmaxf(Mx, __shfl_xor(Mx, 32, 64));
    int c = 0;
    if (COUNT) {
      c = (m == Mx) ? cnt[qb] : 0;
      c += __shfl_xor(c, 16, 64);
      c += __shfl_xor(c, 32, 64);
    }
    // row 0 of the mass block lives in lane r16 (lane group 0), register 0
    const float ms = __shfl(accm[qb][0], r16, 64);
    float zr = zf[qb] + __shfl_xor(zf[qb], 16, 64);
    zr += __shfl_xor(zr, 32, 64);
    const float gate = Mx > 0.f ? (p.has_gamma ? Mx / (Mx + p.gamma) : 1.f) : 0.f;
    const float so = gate / (ms + 1e-12f);
    const float z = zr + 1e-12f;
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
        if (COUNT) p.Nmax[si] = Mx > 0.f ? c : 0;
      }
    }
  }
}

// ------------------------------------------------------------------------------ backward
// Row constants.  With D_i = <dO_i, O_i>/g_i (the flash identity of
// src/triton_pnfirtau.py:575-577), x_i = g_i/Z_i and the score gradient of :580-586,
//   du_ij = 10 x_i u_ij^9 (dW_ij - D_i) + [u_ij == M_i] D_i gate'(M_i)/Nmax_i,
//   dS_ij = scale du_ij,  w_ij = x_i u_ij^10.
// The gradient kernels round w and dS to bf16 once, before their products, as the reference
// does (:566-571, :598-600), and form them from the scores peak-normalised per row: with
// M = m 2^e (m in [0.5, 1)) the scores are computed scaled by 2^-e (exactly: a power of two
// folded into the operands), so every scaled score is below 1 (see pow9_unit) and u9s =
// u^9 2^-9e.  The dQ kernel rounds f du = (10 f x 2^9e) u9s (dW - D) + tie f D gate'/Nmax (f =
// scale, or 1 when scale = 0 so that the tau partials keep du).  The dK/dV kernel rounds
// w = (x 2^10e u9s) s_scaled and dS 2^e / (10 scale) (its dK product takes Q 2^-e and the
// sums are multiplied by 10 scale before they are stored).
// The row constants are eight planes of N floats per (b, h): M, -D, D gate'(M) (the tie
// gradient of du for a single tie), x, M 2^-e, -tau 2^-e, x 2^10e, and plane 7, the dK/dV
// kernel's tie term of dS 2^e / (10 scale) per tied key, written by the dQ kernel, which counts the ties.
// Exponent e of a row peak, M = m 2^e with m in [0.5, 1) (0 for silent rows), kept within
// +-64: a peak below 2^-64 then scales to below 1 all the same, and one above 2^64 has already
// overflowed the forward's u^10.
__device__ __forceinline__ int peak_exponent(float M) {
  return M > 0.f ? min(max(__builtin_amdgcn_frexp_expf(M), -64), 64) : 0;
}

__device__ __forceinline__ float* rc_plane(const BwdParams& p, int64_t bh, int k) {
  return p.rc + (bh * 8 + k) * (int64_t)p.N;
}

template <int D, bool HAS_GAMMA>
__global__ __launch_bounds__(256) void flash_bwd_pre_kernel(BwdParams p) {
  constexpr int LPR = D / 8;  // lanes per row
  constexpr int RPB = 256 / LPR;
  const int tid = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * RPB + tid / LPR;
  const int part = tid % LPR;
  const int64_t total = (int64_t)p.B * p.H * p.N;
  if (p.ktact) {  // cleared here, set by the dQ kernel, read by the dK/dV kernel
    const int64_t nkt = (int64_t)p.B * p.H * p.nk64;
    for (int64_t i = (int64_t)blockIdx.x * 256 + tid; i < nkt; i += (int64_t)gridDim.x * 256)
      p.ktact[i] = 0;
  }
  float dot = 0.f;
  if (row < total) {
    const int64_t bh = row / p.N, i = row % p.N;
    const int64_t b = bh / p.H, h = bh % p.H;
    const int64_t ooff = b * p.osb + h * p.osh + i * p.osn + 8 * part;
    const u32x4 ov = *reinterpret_cast<const u32x4*>(static_cast<const bf16*>(p.o) + ooff);
    u32x4 lv = {0u, 0u, 0u, 0u};
    if (p.o_lo) lv = *reinterpret_cast<const u32x4*>(static_cast<const bf16*>(p.o_lo) + ooff);
    const u32x4 dv = *reinterpret_cast<const u32x4*>(static_cast<const bf16*>(p.dout) + b * p.dosb +
                                                     h * p.dosh + i * p.dosn + 8 * part);
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
    const float M = p.M[row];
    const float g = M > 0.f ? (HAS_GAMMA ? M / (M + p.gamma) : 1.f) : 0.f;
    const float x = g / p.Z[row];  // 0 on silent rows
    const float Dv = g > 0.f ? dot / g : 0.f;
    float dgate = 0.f;
    if (HAS_GAMMA && M > 0.f) dgate = p.gamma / ((M + p.gamma) * (M + p.gamma));
    const int64_t bh = row / p.N, i = row % p.N;
    rc_plane(p, bh, 0)[i] = M;
    rc_plane(p, bh, 1)[i] = -Dv;
    rc_plane(p, bh, 2)[i] = Dv * dgate;
    rc_plane(p, bh, 3)[i] = x;
    // the peak-normalised form of the dK/dV kernel
    const int e = peak_exponent(M);
    rc_plane(p, bh, 4)[i] = __builtin_amdgcn_ldexpf(M, -e);
    rc_plane(p, bh, 5)[i] = __builtin_amdgcn_ldexpf(-p.tau[0], -e);
    rc_plane(p, bh, 6)[i] = __builtin_amdgcn_ldexpf(x, 10 * e);
  }
}

// Rectified power chain on a peak-normalised score.  The dQ kernel forms each row's scores
// scaled by 2^-e, where M = m 2^e (m in [0.5, 1)) is the row's peak: the scaling is exact
// (a power of two folded into the Q fragment and the tau term), and every scaled score is
// < 1.  So min(max(s |s|, 0), 1) -- one multiply with the clamp modifier, no separate
// rectifier -- is exactly u^2, the chain u^4, u^8 follows, and u^9 = u^8 s (u^8 = 0 for
// s <= 0).  Values and roundings are those of the unscaled chain times 2^-9e.
__device__ __forceinline__ float pow9_unit(float s) {
  const float t = __builtin_amdgcn_fmed3f(s * __builtin_fabsf(s), 0.f, 1.f);
  const float t2 = t * t;
  return (t2 * t2) * s;
}

// f du (see the row constants) for the 8 scores a lane holds in query block qb of one 32-key
// half tile of the dQ kernel (S^T layout, one query row per lane, scores scaled by 2^-e),
// written over dw = dW - D: (u9s R) dw + [u == M] T with R = 10 f x 2^9e and T the tie term
// (u, M in the scaled units).  Also counts the row's peak ties.
template <int QB>
__device__ __forceinline__ void ds_kq(const f32x4 (&s)[2][QB], f32x4 (&dw)[2][QB], int (&cnt)[QB],
                                      const float (&rM)[QB], const float (&rR)[QB],
                                      const float (&rT)[QB], int qb) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = pow9_unit(s[kk][qb][i]) * rR[qb];
      const bool tie = s[kk][qb][i] == rM[qb];  // M > 0; T = 0 on silent rows
      dw[kk][qb][i] = __builtin_fmaf(a, dw[kk][qb][i], tie ? rT[qb] : 0.f);
      cnt[qb] += tie ? 1 : 0;
    }
}

// ds_kq without the peak-tie term, for a query block where no row of the wave has a key of
// the half tile at its peak: f du = (u9s R) (dW - D).
template <int QB>
__device__ __forceinline__ void ds_kq_notie(const f32x4 (&s)[2][QB], f32x4 (&dw)[2][QB],
                                            const float (&rR)[QB], int qb) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int i = 0; i < 4; ++i) dw[kk][qb][i] = (pow9_unit(s[kk][qb][i]) * rR[qb]) * dw[kk][qb][i];
}

// Whether some lane of the wave holds, in query block qb, a score tied at its row's peak M on
// a row whose tie term is non-zero.  Every score is <= M (M is the forward's maximum of the
// same MFMA values), so a tie is a lane maximum equal to M; the maximum is an integer max
// over the raw bit patterns (order-preserving for positive floats; negatives, and the mask's
// -1, stay below any M > 0).  Half a VALU op per score against three for the tie compare,
// select and count of ds_kq.  Taken per 16-row block, the tie path runs on about half as
// many blocks as it would per 32-row half tile.
template <int QB>
__device__ __forceinline__ bool peak_tie(const f32x4 (&s)[2][QB], const float (&rM)[QB],
                                         const float (&rT)[QB], int qb) {
  int mx = f2i(s[0][qb][0]);
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = max(mx, f2i(s[kk][qb][i]));
  return __any(mx >= f2i(rM[qb]) && rT[qb] != 0.f);
}

// dQ: query-parallel, same tiling as the forward (4 waves x 32 rows, 64-key tiles), K and V
// tiles software-pipelined through LDS (double-buffered when it fits).
//
// Peak ties.  A key tied at the row's peak gets the extra gradient D gate'/Nmax.  The forward
// does not count ties, so the first pass over the keys gives every tied key the whole-row
// term while it counts the ties (one compare serves both).  Afterwards the per-key share
// goes to the row constants (for the dK/dV kernel) and the tau partial is corrected to one
// whole-row term per row.  A row with two or more ties got too much tie gradient in dQ: if
// the workgroup has any such row (rare: duplicated keys), it runs the key loop a second time
// with the per-key share.
// At D = 128 the dQ accumulators and the Q/dO fragments of 32 rows need more than the 256
// registers a wave has at two workgroups per CU, so each wave takes 16 rows there (64-row
// workgroups, two per CU) instead of running one 128-row workgroup per CU.
template <int D, bool CAUSAL, bool PS>
__global__ __launch_bounds__(256, 2) void flash_bwd_dq_kernel(BwdParams p) {
  // Query rows per wave: 32 (two 16-row MFMA blocks) up to D = 64; 16 at D = 128, where the
  // dQ accumulators and the Q/dO fragments of 32 rows would not fit two workgroups per CU.
  constexpr int QB = dq_qblocks(D), RPW = 16 * QB;
  constexpr int BM = 4 * RPW, BN = 64;
  constexpr int DK = D < 32 ? 32 : D;
  constexpr int KS = DK / 32;
  constexpr int DB = D / 16;
  // Two K/V tile buffers as separate LDS objects (see the dK/dV kernel), filled straight
  // from global memory.
  __shared__ __attribute__((aligned(16))) bf16 Ks0[BN * DK];
  __shared__ __attribute__((aligned(16))) bf16 Vs0[BN * DK];
  __shared__ __attribute__((aligned(16))) bf16 Ks1[BN * DK];
  __shared__ __attribute__((aligned(16))) bf16 Vs1[BN * DK];
  const KVBuf buf0{Ks0, Vs0}, buf1{Ks1, Vs1};

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, provably uniform
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
  const int qrow0 = m0 + RPW * w;
  const bool has_rows = qrow0 < N;
  const float ntau = -p.tau[0];
  const float scale = p.scale;
  // The loops form f du, rounded to bf16 once: with f = scale that is dS, rounded where the
  // reference rounds it; at scale = 0 (dS = 0), f = 1 keeps du for the tau partials.
  const float fdu = scale != 0.f ? scale : 1.f;
  const FragLane flr = rt_lane<DK>(r16, g), flt = tr_lane<DK>(lane);

  bf16x8 qf[QB][KS], dof[QB][KS];
  // Row constants.  The scores of row i are formed scaled by 2^-e_i, e_i the exponent of its
  // peak M_i (see pow9_unit): rM is the scaled peak, rR = 10 f x_i 2^(9 e_i) turns u9s into
  // the factor of dW - D, rT is the tie term (f D gate'; divided by the tie count in a second
  // pass), rT0 the whole-row term and rDg = D gate' for the dK/dV kernel's plane.
  float rM[QB], rR[QB], rT[QB], rT0[QB], rDg[QB];
  int rE[QB];
  f32x4 dw_init[QB];  // -D: the dW accumulator starts there
  f32x4 s_init[QB];   // the score accumulator starts at -tau 2^-e (scale folded into Q)
  float sc_e[QB], nt_e[QB];  // scale 2^-e and -tau 2^-e, for scales that are not folded
  // For the dK/dV kernel (which runs next): the rows of Q scaled by 2^-e.
  bf16* Qs = static_cast<bf16*>(p.qs) + (int64_t)bh * N * D;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = qrow0 + 16 * qb + r16;
    const bool rok = row < N;
    const float M = rok ? rc_plane(p, bh, 0)[row] : 0.f;
    const float nxd = rok ? rc_plane(p, bh, 1)[row] : 0.f;
    rDg[qb] = rok ? rc_plane(p, bh, 2)[row] : 0.f;
    const float x = rok ? rc_plane(p, bh, 3)[row] : 0.f;
    rE[qb] = peak_exponent(M);
    rM[qb] = __builtin_amdgcn_ldexpf(M, -rE[qb]);
    rR[qb] = __builtin_amdgcn_ldexpf(10.f * fdu * x, 9 * rE[qb]);
    rT0[qb] = fdu * rDg[qb];
    rT[qb] = rT0[qb];
    sc_e[qb] = __builtin_amdgcn_ldexpf(scale, -rE[qb]);
    nt_e[qb] = __builtin_amdgcn_ldexpf(ntau, -rE[qb]);
    s_init[qb] = PS ? f32x4{nt_e[qb], nt_e[qb], nt_e[qb], nt_e[qb]} : f32x4{0.f, 0.f, 0.f, 0.f};
    dw_init[qb] = f32x4{nxd, nxd, nxd, nxd};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int col = 32 * ks + 8 * g;
      const bool ok = rok && col < D;
      qf[qb][ks] = ok ? ld16(Q + (int64_t)row * p.qsn + col) : zero_bf16x8();
      dof[qb][ks] = ok ? ld16(dO + (int64_t)row * p.dosn + col) : zero_bf16x8();
      if (ok)
        *reinterpret_cast<bf16x8*>(Qs + (int64_t)row * D + col) =
            scale_frag(qf[qb][ks], __builtin_amdgcn_ldexpf(1.f, -rE[qb]));
      if (PS) qf[qb][ks] = scale_frag(qf[qb][ks], sc_e[qb]);  // a power of two: exact
    }
  }

  int cnt[QB] = {};  // lane-local tie counts (first pass)
  // Sum of every ds the wave forms, accumulated by the MFMA: a constant A fragment whose
  // row 0 is all ones turns the ds^T operand into its column sums (lanes g == 0, slot 0).
  f32x4 adt[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) adt[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 ones = zero_bf16x8();
  if (r16 == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (bf16)1.0f;
  }
  f32x4 acc[DB][QB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) acc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kv_end = CAUSAL ? min(m0 + BM, N) : N;
  const int ntiles = (kv_end + BN - 1) / BN;
  const uint8_t* mrow =
      (p.mask && has_rows) ? p.mask + ((int64_t)bh * p.nq32 + (qrow0 >> 5)) * p.nk64 : nullptr;
  // Activity/tie byte of each (32-row group, 64-key tile) for the dK/dV kernel (one wave
  // per group: at 16 rows per wave the launcher passes no map).
  uint8_t* arow = (p.amap && has_rows && QB == 2)
                      ? p.amap + ((int64_t)bh * p.nq32 + (qrow0 >> 5)) * p.nk64
                      : nullptr;
  // The activity byte of the next tile is fetched one iteration ahead and kept as a raw
  // byte until it is tested, so that its wait does not also wait for the tile prefetch.
  int act_next;

  // With the tile mask and tau > 0, the key loop runs over a compacted list of the tiles where
  // some 32-row group of the workgroup has an active sub-tile (no load, barrier or mask lookup
  // for the others); every wave forms the same ballots over the workgroup's mask rows, writes
  // the activity/tie bytes of its own skipped tiles, and wave 0 writes the list.  At tau <= 0
  // a sub-tile is silent only if all its 2048 scores are <= 0, too rare to pay for the list's
  // prologue (measured: +3 % on the dense dQ); silent sub-tiles still skip their work.
  __shared__ uint16_t tl_s[kMaxListTiles];
  int nlist = ntiles;
  if (p.mask && ntiles <= kMaxListTiles && ntau < 0.f) {
    const int r0 = m0 >> 5, r1 = min((m0 + BM + 31) >> 5, p.nq32);  // the workgroup's mask rows
    const uint8_t* mbase = p.mask + (int64_t)bh * p.nq32 * p.nk64;
    int base = 0;
    for (int c = 0; c < ntiles; c += 64) {
      const int t = c + lane;
      int any = 0;  // (independent loads, not a short-circuit chain)
      if (t < ntiles)
        for (int r = r0; r < r1; ++r) any |= mbase[(int64_t)r * p.nk64 + t];
      const bool f = any != 0;
      if (!f && arow && t < ntiles) arow[t] = 0;
      const uint64_t bal = __ballot(f);
      if (w == 0 && f) tl_s[base + __popcll(bal & ((1ull << lane) - 1ull))] = (uint16_t)t;
      base += __popcll(bal);
    }
    nlist = base;
    __syncthreads();
  }
  const bool ident = nlist == ntiles;  // nothing skipped: the list is 0, 1, 2, ...
  // Entry e of the list (a scalar: tile addresses stay scalar bases); the identity list is
  // not read at all, so the dense loop runs as if there were no list.
  const auto tile_at = [&](int e) {
    return ident ? e : __builtin_amdgcn_readfirstlane((int)tl_s[min(e, nlist - 1)]);
  };

  const TileDma<D, DK> kdma(w, lane, p.ksn), vdma(w, lane, p.vsn);
  auto load_tile = [&](int n, const KVBuf& bb) {
    kdma.load(K, p.ksn, n, N, bb.k, w);
    vdma.load(V, p.vsn, n, N, bb.v, w);
  };
  // Entry e of the list: computed from buffer bc while the next tile streams into buffer bn.
  auto step = [&](int e, const KVBuf& bc, const KVBuf& bn) {
    int t = e, tn = e + 1;
    if (!ident) {
      t = tile_at(e);
      tn = tile_at(e + 1);
    }
    const int n0 = t * BN;
    wait_vmem();  // this wave's part of tile t is in LDS
    __syncthreads();
    const bool pre = e + 1 < nlist;
    if (pre) load_tile(tn * BN, bn);
    const int act = act_next;
    if (mrow && pre) act_next = mrow[tn];
    const bool work = has_rows && !(CAUSAL && n0 > qrow0 + RPW - 1) && act != 0;
    int code = 0;  // the activity/tie byte of this (32-row group, tile)
    if (work) {
      code = 1;
      // key tile t has an active entry: the dK/dV kernel schedules it among the active tiles
      if (mrow && lane == 0) p.ktact[(int64_t)bh * p.nk64 + t] = 1;
      const bf16* Kc = bc.k;
      const bf16* Vc = bc.v;
      const bool masked = (CAUSAL && n0 + BN - 1 > qrow0) || n0 + BN > N;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        if (CAUSAL && n0 + 32 * hf > qrow0 + RPW - 1) break;
        f32x4 s[2][QB], dw[2][QB];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          bf16x8 kf[KS], vf[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const int off = rt_frag<DK>(flr, 2 * hf + kk, ks);
            kf[ks] = ld16(Kc + off);
            vf[ks] = ld16(Vc + off);
          }
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            f32x4 a4 = s_init[qb], c4 = dw_init[qb];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              a4 = mfma16x16x32(kf[ks], qf[qb][ks], a4);
              c4 = mfma16x16x32(vf[ks], dof[qb][ks], c4);
            }
            s[kk][qb] = a4;
            dw[kk][qb] = c4;
          }
        }
        affine_kq_rows<PS>(s, sc_e, nt_e);
        if (masked) mask_kq(s, n0, hf, qrow0, N, CAUSAL, g, r16);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (peak_tie(s, rM, rT, qb)) {
            ds_kq(s, dw, cnt, rM, rR, rT, qb);
            code |= 2 << hf;
          } else {
            ds_kq_notie(s, dw, rR, qb);
          }
        }
        bf16x8 pf[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          pf[qb] = pack8(dw[0][qb][0], dw[0][qb][1], dw[0][qb][2], dw[0][qb][3], dw[1][qb][0],
                         dw[1][qb][1], dw[1][qb][2], dw[1][qb][3]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 ktf = tr_frag<DK>(Kc, flt, hf, db);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) acc[db][qb] = mfma16x16x32(ktf, pf[qb], acc[db][qb]);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) adt[qb] = mfma16x16x32(ones, pf[qb], adt[qb]);
      }
    }
    if (arow && lane == 0) arow[t] = (uint8_t)code;
  };
  for (int pass = 0;; ++pass) {
  const int t0 = nlist > 0 ? tile_at(0) : 0;
  act_next = mrow ? mrow[t0] : 1;
  if (nlist > 0) load_tile(t0 * BN, buf0);
  for (int e = 0; e < nlist; e += 2) {
    step(e, buf0, buf1);
    if (e + 1 < nlist) step(e + 1, buf1, buf0);
  }
  if (pass == 1) break;

  // Tie counts per row (the four lane groups of a row), the dK/dV kernel's tie term per tied
  // key, and the tau partial: the MFMA sum holds f du over the row with Nmax whole-row tie
  // terms where one belongs.
  double dsum = 0.0;
  bool multi = false;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    int c = cnt[qb];
    c += __shfl_xor(c, 16, 64);
    c += __shfl_xor(c, 32, 64);
    const int qrow = qrow0 + 16 * qb + r16;
    if (g == 0 && qrow < N) {
      // dS per tied key in the dK/dV kernel's units, dS 2^e / (10 scale)
      const float ts = __builtin_amdgcn_ldexpf(rDg[qb], rE[qb]) / 10.f;
      rc_plane(p, bh, 7)[qrow] = c > 0 ? ts / (float)c : 0.f;
      double rs = (double)adt[qb][0];
      if (c > 1) rs -= (double)rT0[qb] * (double)(c - 1);
      dsum += rs;
    }
    multi = multi || (c > 1 && rT0[qb] != 0.f);
    rT[qb] = c > 0 ? rT0[qb] / (float)c : 0.f;  // for a second pass
  }
  // sum of du (f du / f)
  dsum = wave_sum_d(dsum) / (double)fdu;
  if (lane == 0) p.partials[((int64_t)bh * nqb + qblk) * 4 + w] = dsum;
  // Second pass only if some row of the workgroup has several ties (also a barrier: the
  // last tile's LDS buffer is free before the first tile is staged again).
  if (!__syncthreads_or(multi ? 1 : 0)) break;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) acc[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  bf16* dQ = static_cast<bf16*>(p.dq) + b * p.dqsb + h * p.dqsh;
  const float rowf = scale != 0.f ? 1.f : 0.f;  // dS = scale du: the sums are dQ (or 0)
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qrow = qrow0 + 16 * qb + r16;
    if (qrow < N) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = (bf16)(acc[db][qb][i] * rowf);
        *reinterpret_cast<bf16x4*>(dQ + (int64_t)qrow * p.dqsn + 16 * db + 4 * g) = o4;
      }
    }
  }
}

// dK and dV: key-parallel.  Each wave owns KPW consecutive keys (32 for D <= 64, 16 for
// D = 128) held as MFMA B fragments; the workgroup streams 64-row query tiles (Q 2^-e and
// dO, plus the row constants) through LDS from the last query tile back to the causal
// diagonal; the transposed operands come from the same tiles through transposing reads.
template <int D>
struct DkdvCfg {
  static constexpr int KPW = D <= 64 ? 32 : 16;
  static constexpr int KB = KPW / 16;
  static constexpr int BNK = 4 * KPW;
};

// Query-major layout S (register i of lane group g holds query perm_row(blk, 4g+i) of the
// tile, lane r16 holds key 16kb+r16 of the wave's keys): the affine map and the mask, as
// affine_kq and mask_kq above.
// The affine map with a -tau per query row (register i of block qq): the peak-normalised
// scores, formed from Q 2^-e.
template <int KB, bool PS>
__device__ __forceinline__ void affine_qk_rows(f32x4 (&s)[2][KB], float scale,
                                               const f32x4 (&ntau)[2]) {
  if (PS) return;
#pragma unroll
  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[qq][kb][i] = __builtin_fmaf(s[qq][kb][i], scale, ntau[qq][i]);
}

template <int KB>
__device__ __forceinline__ void mask_qk(f32x4 (&s)[2][KB], int m0, int hf, int kw0, int N,
                                        bool causal, int g, int r16) {
#pragma unroll
  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qrow = m0 + perm_row(2 * hf + qq, 4 * g + i);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int key = kw0 + 16 * kb + r16;
        if ((causal && key > qrow) || key >= N || qrow >= N) s[qq][kb][i] = -1.f;
      }
    }
}

// The scores are peak-normalised (scaled by 2^-e per row, see pow9_unit).  With
// aw = u9s x 2^10e = x u^9 2^e (rc plane 4 holds x 2^10e), the dV weight w = aw s = x u^10 is
// written over s, and dS 2^e / c = aw dw + [u == M] T 2^e / c over dw = dW - D, c = 10 scale:
// the reference's w and its dS up to the constant factor c, each to be rounded to bf16 once
// (dS 2^e / c rounds as dS does, to the same relative precision; the dK product takes Q 2^-e
// and the kernel multiplies its dK sums by c before they are stored).  rc holds the planes
// (M 2^-e, -D, T 2^e / c per tied key, -tau 2^-e, x 2^10e).
template <int KB>
__device__ __forceinline__ void w_ds_qk_x(f32x4 (&s)[2][KB], f32x4 (&dw)[2][KB], const float* rc,
                                          int pitch, int r4) {
#pragma unroll
  for (int qq = 0; qq < 2; ++qq) {
    const f32x4 m4 = *reinterpret_cast<const f32x4*>(rc + r4 + 4 * qq);
    const f32x4 t4 = *reinterpret_cast<const f32x4*>(rc + 2 * pitch + r4 + 4 * qq);
    const f32x4 x4 = *reinterpret_cast<const f32x4*>(rc + 4 * pitch + r4 + 4 * qq);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const float sv = s[qq][kb][i];
        const float aw = pow9_unit(sv) * x4[i];
        s[qq][kb][i] = aw * sv;                           // 0 for sv <= 0 (u9s = 0)
        const float tie = (sv == m4[i]) ? t4[i] : 0.f;  // M > 0; T = 0 on silent rows
        dw[qq][kb][i] = __builtin_fmaf(aw, dw[qq][kb][i], tie);
      }
  }
}

// w_ds_qk_x without the peak-tie term (no row of the half has a key of this wave at its peak).
template <int KB>
__device__ __forceinline__ void w_ds_qk_x_notie(f32x4 (&s)[2][KB], f32x4 (&dw)[2][KB],
                                                const float* rc, int pitch, int r4) {
#pragma unroll
  for (int qq = 0; qq < 2; ++qq) {
    const f32x4 x4 = *reinterpret_cast<const f32x4*>(rc + 4 * pitch + r4 + 4 * qq);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const float sv = s[qq][kb][i];
        const float aw = pow9_unit(sv) * x4[i];
        s[qq][kb][i] = aw * sv;
        dw[qq][kb][i] = aw * dw[qq][kb][i];
      }
  }
}

// Position e of the key-tile order of one (b, h): the tiles with act[t] != 0 ascending, then
// the others ascending.  Returns the tile (or -1 past the end) and whether it is active.
// Wave-uniform; two sweeps of nk64 bytes with ballots.
__device__ __forceinline__ int ordered_ktile(const uint8_t* act, int nk64, int e, int lane,
                                             bool& active) {
  int na = 0;
  for (int c = 0; c < nk64; c += 64) {
    const bool f = c + lane < nk64 && act[c + lane] != 0;
    na += __popcll(__ballot(f));
  }
  active = e < na;
  int want = active ? e : e - na;
  for (int c = 0; c < nk64; c += 64) {
    const bool f = c + lane < nk64 && (act[c + lane] != 0) == active;
    const uint64_t bal = __ballot(f);
    const int cnt = __popcll(bal);
    if (want < cnt) {
      const int below = __popcll(bal & ((1ull << lane) - 1ull));
      return c + __ffsll((long long)__ballot(f && below == want)) - 1;
    }
    want -= cnt;
  }
  active = false;
  return -1;
}

// dtau = -(sum of all du partials), summed in fp64 by one 256-thread workgroup in a fixed
// order (deterministic); each thread keeps eight independent loads in flight.  Run by the
// first workgroup of the dK/dV kernel after its own keys: the dQ stage that wrote the
// partials has finished by then (stream order), no launch of its own is needed, and that
// workgroup (the heaviest causal key block, dispatched first) ends well before the kernel.
__device__ __forceinline__ void dtau_sum(const double* partials, int64_t n, float* dtau, int tid) {
  __shared__ double red[4];
  double a[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  int64_t i = tid;
  for (; i + 7 * 256 < n; i += 8 * 256) {
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] += partials[i + u * 256];
  }
  for (; i < n; i += 256) a[0] += partials[i];
  const double acc =
      wave_sum_d(((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7])));
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) dtau[0] = (float)(-((red[0] + red[1]) + (red[2] + red[3])));
}

template <int D, bool CAUSAL, bool PS>
__global__ __launch_bounds__(256, 2) void flash_bwd_dkdv_kernel(BwdParams p) {
  // The scores are peak-normalised per row (from the dQ kernel's copy Q 2^-e, which also
  // serves the dK product) and the weights formed from u9s; the tiles are Q 2^-e and dO.
  constexpr int KPW = DkdvCfg<D>::KPW, KB = DkdvCfg<D>::KB, BNK = DkdvCfg<D>::BNK;
  constexpr int BMQ = 64;
  constexpr int DK = D < 32 ? 32 : D;
  constexpr int KS = DK / 32;
  constexpr int DB = D / 16;
  // Two LDS buffers, as separate objects: the compiler then knows that the direct-to-LDS
  // loads filling one buffer do not write the other, and does not make the reads of the
  // current tile wait for the prefetch of the next one.  Row constants are five planes of the
  // tile's rows: a lane reads the four consecutive rows its registers cover as one f32x4 per
  // plane (broadcast within a 16-lane group; the four groups' rows are 8 apart, in different
  // banks): M 2^-e, -D, T 2^e / c_ds per tied key, -tau 2^-e, x 2^10e.
  constexpr int NPL = 5;
  __shared__ __attribute__((aligned(16))) bf16 Qs0[BMQ * DK];
  __shared__ __attribute__((aligned(16))) bf16 dOs0[BMQ * DK];
  __shared__ __attribute__((aligned(16))) float RC0[NPL * BMQ];
  __shared__ __attribute__((aligned(16))) bf16 Qs1[BMQ * DK];
  __shared__ __attribute__((aligned(16))) bf16 dOs1[BMQ * DK];
  __shared__ __attribute__((aligned(16))) float RC1[NPL * BMQ];
  const QBuf buf0{Qs0, dOs0, RC0}, buf1{Qs1, dOs1, RC1};

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, r16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, provably uniform
  const int N = p.N;
  int bh, kvb;
  map_block(p.nkvb, p.B * p.H, false, bh, kvb);
  const int b = bh / p.H, h = bh % p.H;
  const bf16* K = static_cast<const bf16*>(p.k) + b * p.ksb + h * p.ksh;
  const bf16* V = static_cast<const bf16*>(p.v) + b * p.vsb + h * p.vsh;
  const bf16* dO = static_cast<const bf16*>(p.dout) + b * p.dosb + h * p.dosh;
  // Staging of the row constants: wave w copies one plane of the tile's rows, wave 0 also the
  // fifth (workspace planes 4, 1, 7, 5, 6).
  const float* RCgw = rc_plane(p, bh, w == 0 ? 4 : w == 2 ? 7 : w == 3 ? 5 : 1);
  const float* RCg4 = rc_plane(p, bh, 6);
  // Q 2^-e, written by the dQ kernel
  const bf16* Qsc = static_cast<const bf16*>(p.qs) + (int64_t)bh * N * D;
  // The workgroup's 64-key tiles.  With the tile activity of the dQ stage, workgroup j of a
  // (b, h) takes positions TPW j .. TPW j + TPW - 1 of the order "active tiles ascending, then
  // silent tiles": active tiles share workgroups, so no wave idles beside an active one, and
  // a workgroup of silent tiles only writes zeros.  Without it, tiles in index order.
  constexpr int TPW = BNK / 64;
  int wtile, tile0;
  bool wact = true, wg_active = true;
  if (p.ktact) {
    const uint8_t* act = p.ktact + (int64_t)bh * p.nk64;
    wtile = ordered_ktile(act, p.nk64, TPW * kvb + (KPW * w) / 64, lane, wact);
    tile0 = ordered_ktile(act, p.nk64, TPW * kvb, lane, wg_active);
    // wave-uniform by construction; keep them in scalar registers
    wtile = __builtin_amdgcn_readfirstlane(wtile);
    tile0 = __builtin_amdgcn_readfirstlane(tile0);
    wact = __builtin_amdgcn_readfirstlane(wact ? 1 : 0) != 0;
    wg_active = __builtin_amdgcn_readfirstlane(wg_active ? 1 : 0) != 0;
  } else {
    wtile = (kvb * BNK + KPW * w) / 64;
    tile0 = kvb * TPW;
  }
  const int kw0 = wtile < 0 ? N : wtile * 64 + (KPW * w) % 64;
  const bool has_keys = kw0 < N;  // the wave writes dK, dV rows (zeros if silent)
  const bool live = has_keys && wact;
  const float scale = p.scale;
  const float c_ds = 10.f * scale;  // the dK sums take dS / c_ds
  const FragLane flr = rt_lane<DK>(r16, g), flt = tr_lane<DK>(lane);

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
      if (PS) kf[kb][ks] = scale_frag(kf[kb][ks], scale);
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

  const int nqt = (N + BMQ - 1) / BMQ;
  // Query tiles qt0 .. nqt - 1, visited from the last one down: qt0 is the causal diagonal
  // of the workgroup's lowest active tile (the first in the order), none if the workgroup
  // has only silent tiles.  Every workgroup of a (b, h) starts at the last tile and moves
  // down in step with the others, so each Q/dO tile is fetched from HBM about once while
  // the workgroups that need it read it from L2 (ascending from the diagonals, workgroups
  // with distant diagonals read the same tile far apart in time: 3.5x the HBM reads with
  // half the key tiles silent).
  const int qt0 = !wg_active ? nqt : (CAUSAL ? tile0 * 64 / BMQ : 0);
  // Per-sub-tile activity, from the dQ stage's activity/tie map (bit 0 active, bit 1 + h a
  // peak tie in 32-key half h) or else from the forward's tile mask (no tie information: the
  // tie test runs everywhere).
  const uint8_t* msrc = p.amap ? p.amap : p.mask;
  const uint8_t* mcol = (msrc && live) ? msrc + (int64_t)bh * p.nq32 * p.nk64 + wtile : nullptr;
  const int tie_bit = p.amap ? 2 << (((KPW * w) % 64) / 32) : 0xff;

  // Tiles go straight from global memory to LDS buffer bb; rows >= N repeat row N - 1 (their
  // scores are masked), including their row constants.  D <= 64: whole tiles take a scalar
  // base plus the lanes' fixed 32-bit offsets; D = 128, at the register limit, forms every
  // address from the row and column.
  const TileDma<D, DK> tq(w, lane, D), tdo(w, lane, p.dosn);
  auto load_tile = [&](int m, const QBuf& bb) {
    if (D <= 64) {
      tq.load(Qsc, D, m, N, bb.q, w);
      tdo.load(dO, p.dosn, m, N, bb.o, w);
    } else {
      tq.load_clamped(Qsc, D, m, N, bb.q, w);
      tq.load_clamped(dO, p.dosn, m, N, bb.o, w);
    }
    const int row = min(m + lane, N - 1);
    lds_dma4(RCgw + row, bb.rc + w * BMQ);
    if (w == 0) lds_dma4(RCg4 + row, bb.rc + (NPL - 1) * BMQ);
  };
  if (qt0 < nqt) load_tile((nqt - 1) * BMQ, buf0);

  // Activity of a 64-row query tile for this wave's keys: either of its two 32-row halves.
  // Fetched one iteration ahead and kept as raw bytes until tested, so that its wait does
  // not also wait for the tile prefetch.
  int act_next[2] = {0xff, 0xff};  // without a map: every half active, tie test everywhere
  auto fetch_active = [&](int m) {
    const int r32 = m >> 5;
    act_next[0] = mcol[(int64_t)r32 * p.nk64];
    act_next[1] = r32 + 1 < p.nq32 ? mcol[(int64_t)(r32 + 1) * p.nk64] : 0;
  };
  if (mcol && qt0 < nqt) fetch_active((nqt - 1) * BMQ);
  // One query tile: computed from buffer bc while the next tile streams into buffer bn.
  auto step = [&](int qt, const QBuf& bc, const QBuf& bn) {
    const int m0 = qt * BMQ;
    wait_vmem();  // this wave's part of tile qt is in LDS
    __syncthreads();
    const bool pre = qt > qt0;
    if (pre) load_tile(m0 - BMQ, bn);
    const int act0 = act_next[0], act1 = act_next[1];
    if (mcol && pre) fetch_active(m0 - BMQ);
    const bool work = live && !(CAUSAL && m0 + BMQ - 1 < kw0) && ((act0 | act1) & 1) != 0;
    if (work) {
      const bf16* Qc = bc.q;
      const bf16* dOc = bc.o;
      const bf16* Qt = Qc;    // operand of dK += dS^T Q (dS 2^e / c_ds and Q 2^-e)
      const bf16* dOt = dOc;  // operand of dV += w^T dO
      const bool masked = (CAUSAL && m0 < kw0 + KPW - 1) || m0 + BMQ > N || kw0 + KPW > N;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        if (CAUSAL && m0 + 32 * hf + 31 < kw0) continue;  // rows of this half precede the keys
        // wave-uniform (one byte, loaded by every lane): keep it in a scalar register
        const int code = __builtin_amdgcn_readfirstlane(hf ? act1 : act0);
        if (!(code & 1)) continue;          // a silent 32-row half
        const bool ties = (code & tie_bit) != 0;
        f32x4 s[2][KB], dw[2][KB];
        f32x4 ntr[2];  // -tau 2^-e of the lane's rows in each 16-row block
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          // The dW accumulator starts at -D of the four rows the lane's registers cover, the
          // score accumulator at their -tau 2^-e (scale folded into K) or 0 (affine below)
          const int r4 = 32 * hf + 8 * g + 4 * qq;
          const f32x4 dw0 = *reinterpret_cast<const f32x4*>(bc.rc + BMQ + r4);
          ntr[qq] = *reinterpret_cast<const f32x4*>(bc.rc + 3 * BMQ + r4);
          const f32x4 sa0 = PS ? ntr[qq] : f32x4{0.f, 0.f, 0.f, 0.f};
          bf16x8 qa[KS], da[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const int off = rt_frag<DK>(flr, 2 * hf + qq, ks);
            qa[ks] = ld16(Qc + off);
            da[ks] = ld16(dOc + off);
          }
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            f32x4 a4 = sa0, c4 = dw0;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              a4 = mfma16x16x32(qa[ks], kf[kb][ks], a4);
              c4 = mfma16x16x32(da[ks], vf[kb][ks], c4);
            }
            s[qq][kb] = a4;
            dw[qq][kb] = c4;
          }
        }
        affine_qk_rows<KB, PS>(s, scale, ntr);
        if (masked) mask_qk<KB>(s, m0, hf, kw0, N, CAUSAL, g, r16);
        // rows 32 hf + 8 g + 4 qq + (0..3) of the tile are perm_row(2 hf + qq, 4 g + i)
        if (ties) w_ds_qk_x<KB>(s, dw, bc.rc, BMQ, 32 * hf + 8 * g);
        else w_ds_qk_x_notie<KB>(s, dw, bc.rc, BMQ, 32 * hf + 8 * g);
        bf16x8 wf[KB], sf[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          wf[kb] = pack8(s[0][kb][0], s[0][kb][1], s[0][kb][2], s[0][kb][3], s[1][kb][0],
                         s[1][kb][1], s[1][kb][2], s[1][kb][3]);
          sf[kb] = pack8(dw[0][kb][0], dw[0][kb][1], dw[0][kb][2], dw[0][kb][3], dw[1][kb][0],
                         dw[1][kb][1], dw[1][kb][2], dw[1][kb][3]);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 ot = tr_frag<DK>(dOt, flt, hf, db);
          const bf16x8 qt_ = tr_frag<DK>(Qt, flt, hf, db);
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            adv[db][kb] = mfma16x16x32(ot, wf[kb], adv[db][kb]);
            adk[db][kb] = mfma16x16x32(qt_, sf[kb], adk[db][kb]);
          }
        }
      }
    }
  };
  for (int qt = nqt - 1; qt >= qt0; qt -= 2) {
    step(qt, buf0, buf1);
    if (qt > qt0) step(qt - 1, buf1, buf0);
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
          k4[i] = (bf16)(adk[db][kb][i] * c_ds);
          v4[i] = (bf16)adv[db][kb][i];
        }
        *reinterpret_cast<bf16x4*>(dK + (int64_t)key * p.dksn + 16 * db + 4 * g) = k4;
        *reinterpret_cast<bf16x4*>(dV + (int64_t)key * p.dvsn + 16 * db + 4 * g) = v4;
      }
    }
  }
  if (blockIdx.x == 0) {  // the dQ stage's tau partials (one per dQ wave)
    constexpr int64_t rw = 64 * dq_qblocks(D);
    dtau_sum(p.partials, (int64_t)p.B * p.H * ((p.N + rw - 1) / rw) * 4, p.dtau, tid);
  }
}

// The score scale folds into the operands exactly when it is a power of two (d = 16, 64).
// All three kernels must make the same choice: the backward's peak-tie test u == M
// compares its recomputed scores with the forward's M bit for bit.
bool pow2_scale(float s) {
  int e;
  return s > 0.f && std::frexp(s, &e) == 0.5f;
}

template <int D, bool PS>
void launch_fwd_dp(const FwdParams& fp, bool causal, hipStream_t st) {
  if (fp.knorm && D <= 64 && fp.nk64 <= kMaxBoundTiles) {
    const int64_t tiles = (int64_t)fp.B * fp.H * fp.nk64;
    hipLaunchKernelGGL((flash_key_norm_kernel<D>), dim3((unsigned)((tiles + 3) / 4)), dim3(256), 0,
                       st, fp);
  }
  const int nqb = (fp.N + 127) / 128;
  const dim3 grid((unsigned)(nqb * fp.B * fp.H)), block(256);
  const bool count = fp.Nmax != nullptr;
  if (causal) {
    if (count) hipLaunchKernelGGL((flash_fwd_kernel<D, true, PS, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((flash_fwd_kernel<D, true, PS, false>), grid, block, 0, st, fp);
  } else {
    if (count) hipLaunchKernelGGL((flash_fwd_kernel<D, false, PS, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((flash_fwd_kernel<D, false, PS, false>), grid, block, 0, st, fp);
  }
}

template <int D>
int flash_fwd_fir_launch(const FwdParams& fp, bool causal, hipStream_t st) {
  const int nqb = (fp.N + 127) / 128;
  const dim3 grid((unsigned)(nqb * fp.B * fp.H)), block(256);
  const bool ps = pow2_scale(fp.scale);
  if (causal) {
    if (ps) hipLaunchKernelGGL((flash_fwd_kernel<D, true, true, false, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((flash_fwd_kernel<D, true, false, false, true>), grid, block, 0, st, fp);
  } else {
    if (ps) hipLaunchKernelGGL((flash_fwd_kernel<D, false, true, false, true>), grid, block, 0, st, fp);
    else hipLaunchKernelGGL((flash_fwd_kernel<D, false, false, false, true>), grid, block, 0, st, fp);
  }
  return launch_status("pnfx_flash_fwd_fir");
}

template <int D>
int launch_fwd_d(const FwdParams& fp, bool causal, hipStream_t st) {
  if (pow2_scale(fp.scale)) launch_fwd_dp<D, true>(fp, causal, st);
  else launch_fwd_dp<D, false>(fp, causal, st);
  return launch_status("pnfx_flash_fwd");
}

template <int D, bool PS>
void launch_dq(const BwdParams& bp, bool causal, dim3 grid, hipStream_t st) {
  const dim3 block(256);
  if (causal) hipLaunchKernelGGL((flash_bwd_dq_kernel<D, true, PS>), grid, block, 0, st, bp);
  else hipLaunchKernelGGL((flash_bwd_dq_kernel<D, false, PS>), grid, block, 0, st, bp);
}

template <int D>
int launch_bwd_d(const BwdParams& bp_in, bool causal, bool has_gamma, int stages, hipStream_t st) {
  const dim3 block(256);
  // The activity/tie map needs one dQ wave per 32-row group: not at 16 rows per wave.
  BwdParams bp = bp_in;
  if (dq_qblocks(D) < 2) bp.amap = nullptr;
  if (stages & PNFX_BWD_PREPARE) {
    const int64_t rows = (int64_t)bp.B * bp.H * bp.N;
    const int rpb = 256 / (D / 8);
    const dim3 gpre((unsigned)((rows + rpb - 1) / rpb));
    if (has_gamma) hipLaunchKernelGGL((flash_bwd_pre_kernel<D, true>), gpre, block, 0, st, bp);
    else hipLaunchKernelGGL((flash_bwd_pre_kernel<D, false>), gpre, block, 0, st, bp);
    const int rc = launch_status("pnfx_flash_bwd(prepare)");
    if (rc) return rc;
  }
  const bool ps = pow2_scale(bp.scale);
  if (stages & PNFX_BWD_DQ) {
    const int rw = (int)dq_rows_per_wg(D);
    const int nqb = (bp.N + rw - 1) / rw;
    const dim3 gdq((unsigned)(nqb * bp.B * bp.H));
    if (ps) launch_dq<D, true>(bp, causal, gdq, st);
    else launch_dq<D, false>(bp, causal, gdq, st);
    const int rc = launch_status("pnfx_flash_bwd(dq)");
    if (rc) return rc;
  }
  if (stages & PNFX_BWD_DKDV) {  // reads the tie terms and tau partials the dQ stage wrote
    const dim3 gkv((unsigned)(bp.nkvb * bp.B * bp.H));
    if (causal) {
      if (ps) hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, true, true>), gkv, block, 0, st, bp);
      else hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, true, false>), gkv, block, 0, st, bp);
    } else {
      if (ps) hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, false, true>), gkv, block, 0, st, bp);
      else hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, false, false>), gkv, block, 0, st, bp);
    }
    const int rc = launch_status("pnfx_flash_bwd(dkdv)");
    if (rc) return rc;
  }
  return PNFX_OK;
}

}  // namespace



int flash_fwd_bf16(const FwdParams& fp, int64_t D, bool causal, hipStream_t st) {
  switch (D) {
    case 16: return launch_fwd_d<16>(fp, causal, st);
    case 32: return launch_fwd_d<32>(fp, causal, st);
    case 64: return launch_fwd_d<64>(fp, causal, st);
    case 128: return launch_fwd_d<128>(fp, causal, st);
  }
  set_error("flash: head dim %lld not in {16, 32, 64, 128}", (long long)D);
  return PNFX_EUNSUPPORTED;
}

int flash_fwd_fir_bf16(const FwdParams& fp, int64_t D, bool causal, hipStream_t st) {
  switch (D) {
    case 16: return flash_fwd_fir_launch<16>(fp, causal, st);
    case 32: return flash_fwd_fir_launch<32>(fp, causal, st);
    case 64: return flash_fwd_fir_launch<64>(fp, causal, st);
  }
  set_error("flash_fwd_fir: head dim %lld (the fused FIR is built for 16, 32, 64)", (long long)D);
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
