// Internal interface between the flash C-ABI entry points and the per-dtype kernels.
#pragma once

#include "pnfx_common.h"

namespace pnfx {

struct FwdParams {
  const void *q, *k, *v;
  void* o;
  void* o_lo;  // optional bf16 rounding residual of O (same strides as o)
  int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn;
  float* M;
  float* Z;
  int32_t* Nmax;  // optional: the peak-tie counts are only formed when requested
  uint8_t* mask;
  float* knorm;  // optional [B*H][nk64]: largest key norm per 64-key tile (silent-tile bound)
  int B, H, N, nq32, nk64;
  const float* tau;
  float scale, gamma;
  int has_gamma;
  // pnfx_flash_fwd_fir: k holds the raw keys and the kernel filters each key tile with these
  // causal FIR taps ([fir_taps_rows][fir_k] fp32, as pnfx_fir_fwd) before its scores
  const float* fir_taps = nullptr;
  int fir_taps_rows = 0, fir_k = 0;
};

struct BwdParams {
  const void *q, *k, *v, *o, *o_lo, *dout;
  void *dq, *dk, *dv;
  int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn, dosb, dosh, dosn;
  int64_t dqsb, dqsh, dqsn, dksb, dksh, dksn, dvsb, dvsh, dvsn;
  const float* M;
  const float* Z;
  const uint8_t* mask;
  float* rc;         // row constants [B*H*N][8], layout private to each dtype's kernels
  double* partials;  // tau partials, one per wave of the dq kernel (bf16: [B*H][N/BM][4])
  void* qs;          // bf16: Q rows scaled by 2^-e (exactly; 2^e the power of two of
                     // the row's peak), contiguous [B*H, N, D]: the dK/dV kernel's scores and
                     // its dK product
  uint8_t* ktact;    // [B*H][nk64]: 64-key tiles with any active tile-mask entry (mask given)
  uint8_t* amap;     // [B*H][nq32][nk64] (mask given, N <= kAmapMaxN): bit 0 the sub-tile's
                     // activity, bit 1 + h a peak tie in its 32-key half h (dQ -> dK/dV)
  float* dtau;
  int B, H, N, nq32, nk64, nkvb;
  const float* tau;
  float scale, gamma;
};

// 16-row MFMA query blocks per wave of the bf16 dQ kernel (workgroups of four waves cover
// 64 * dq_qblocks(D) query rows).
constexpr int dq_qblocks(int64_t D) { return D <= 64 ? 2 : 1; }
inline int64_t dq_rows_per_wg(int64_t D) { return 64 * dq_qblocks(D); }

// Key blocks of the key-parallel backward kernel.
inline int bwd_nkvb(int64_t N, int64_t D) {
  const int64_t bnk = D <= 64 ? 128 : 64;
  return (int)((N + bnk - 1) / bnk);
}
// Workspace of the backward: row constants, tau partials (fp64, one per wave of the bf16 dq
// kernel, four per workgroup; the fp32 kernels use one per 64 rows), the peak-normalised
// copy of Q that the bf16 dK/dV kernel reads, one activity byte per 64-key
// tile, and the activity/tie map of the 32-query x 64-key sub-tiles (written by a dQ wave of
// 32 rows, so only where the dQ kernel runs two 16-row blocks per wave: D <= 64).
// The activity/tie map of the backward (BwdParams::amap) is kept up to this sequence length:
// N^2/2048 bytes per (b, h), 2 MiB at N = 65536.
constexpr int64_t kAmapMaxN = 65536;
struct BwdWorkspace {
  int64_t rc_bytes, parts_bytes, xt_bytes, kt_bytes, amap_bytes;
  BwdWorkspace(int64_t B, int64_t H, int64_t N, int64_t D) {
    const int64_t rw = dq_rows_per_wg(D);
    const int64_t slots = B * H * ((N + rw - 1) / rw) * 4;
    rc_bytes = round256(B * H * N * 8 * 4);
    parts_bytes = round256(slots * 8);
    xt_bytes = round256(B * H * N * D * 2);  // Q 2^-e
    kt_bytes = round256(B * H * ((N + 63) / 64));
    amap_bytes = (N <= kAmapMaxN && dq_qblocks(D) == 2)
                     ? round256(B * H * ((N + 31) / 32) * ((N + 63) / 64))
                     : 0;
  }
  int64_t total() const { return rc_bytes + parts_bytes + xt_bytes + kt_bytes + amap_bytes; }
  static int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }
};

int flash_fwd_bf16(const FwdParams& fp, int64_t D, bool causal, hipStream_t st);
int flash_fwd_fir_bf16(const FwdParams& fp, int64_t D, bool causal, hipStream_t st);
int flash_bwd_bf16(const BwdParams& bp, int64_t D, bool causal, bool has_gamma, int stages,
                   hipStream_t st);
int flash_fwd_f32(const FwdParams& fp, int64_t D, bool causal, bool has_gamma, hipStream_t st);
int flash_bwd_f32(const BwdParams& bp, int64_t D, bool causal, bool has_gamma, int stages,
                  hipStream_t st);

}  // namespace pnfx
