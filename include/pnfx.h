/*
 * pnfx.h -- C ABI of the MI355X (gfx950) pn_fir_tau hot-path library, libpnfx.so.
 *
 * Every entry point takes device pointers, element strides and sizes, and a
 * hipStream_t passed as `void*` (NULL = the legacy default stream).  Kernels are
 * enqueued on that stream; nothing blocks the host and nothing is allocated:
 * callers own every buffer, including the workspace of pnfx_flash_bwd (the one
 * exception, pnfx_flash_bwd_noalloc, uses a scratch array the library holds).
 *
 * Return value: PNFX_OK (0) or a negative PNFX_E* code; pnfx_last_error()
 * returns a thread-local message for the last failing call on that thread.
 *
 * Strides are in elements.  The innermost (channel / head-dim) stride of every
 * tensor argument is 1.  dtype is one of PNFX_F32, PNFX_BF16.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   pnfx_fir_fwd / pnfx_fir_bwd        src/triton_pnfirtau.py:629-691
 *                                      (_TritonCausalFir7Fn, triton_causal_fir)
 *   pnfx_pn_rows_fwd / pnfx_pn_rows_bwd src/triton_pnfirtau.py:694-811
 *                                      (_TritonPnFirTauScoresFn, triton_pn_fir_tau_scores)
 *   pnfx_flash_fwd / pnfx_flash_bwd    src/triton_pnfirtau.py:814-983
 *                                      (_FlashPnFirTauFn, flash_pn_fir_tau_attention)
 */
#ifndef PNFX_H_
#define PNFX_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PNFX_ABI_VERSION 3

#define PNFX_OK 0
#define PNFX_EINVAL (-1)       /* bad shape / stride / alignment / argument */
#define PNFX_EUNSUPPORTED (-2) /* valid request this build does not implement */
#define PNFX_ELAUNCH (-3)      /* the HIP runtime refused a launch */

#define PNFX_F32 0
#define PNFX_BF16 1

int pnfx_abi_version(void);
const char* pnfx_last_error(void);

/*
 * Causal depthwise FIR along the sequence axis.
 *   x    : [B, H, N, C] with strides (sb, sh, sn, 1)
 *   y    : contiguous [B, H, N, C], same dtype as x
 *   taps : fp32 [taps_rows, K], oldest lag first (taps[.., K-1] is lag 0);
 *          taps_rows == 1 (shared) or taps_rows == H (per head)
 * forward: y[n] = x[n]*h0 + sum_{u=1..K-1, n-u>=0} h_u x[n-u] as an fp32 fused
 * multiply-add chain in lag order, rounded once to the storage type.
 * 1 <= K <= 16.  Replaces _causal_fir7_fwd_kernel (src/triton_pnfirtau.py:40-87)
 * through _TritonCausalFir7Fn.forward (:631-658); the reference's [B,N,C] call
 * is H == 1.
 */
int pnfx_fir_fwd(const void* x, int64_t sb, int64_t sh, int64_t sn, void* y, int64_t B,
                 int64_t H, int64_t N, int64_t C, const float* taps, int64_t taps_rows, int K,
                 int dtype, void* stream);

/*
 * Adjoint of pnfx_fir_fwd: gx[n] = gy[n]*h0 + sum_{u, n+u<N} h_u gy[n+u].
 * Replaces _causal_fir7_bwd_kernel (src/triton_pnfirtau.py:89-135) through
 * _TritonCausalFir7Fn.backward (:660-682).
 */
int pnfx_fir_bwd(const void* gy, int64_t sb, int64_t sh, int64_t sn, void* gx, int64_t B,
                 int64_t H, int64_t N, int64_t C, const float* taps, int64_t taps_rows, int K,
                 int dtype, void* stream);

/*
 * Row-fused rectified power-norm score -> weight, rows of a square [.., N, N]
 * score tensor.  raw / w: R rows of N entries, row strides raw_rs / w_rs.
 * Row r is query position t = r % N (causal mask col <= t when causal != 0).
 * s = raw*scale - tau[0]; u = relu(s) on valid entries; pw = u^p (p == 10 and
 * p == 2 by repeated multiplication, otherwise exp(p log u)); Z = sum pw + 1e-12;
 * gate = M/(M+gamma) (has_gamma) or 1; w = pw * (gate/Z); stats M = max u,
 * Z, Nmax = #(u == M).  Silent rows (M <= 0): w = 0, M = 0, Z = 1e-12, Nmax = 0.
 * Replaces _pn_fir_tau_row_fwd_kernel (src/triton_pnfirtau.py:141-212) through
 * _TritonPnFirTauScoresFn.forward (:694-752).  Any N >= 1.
 */
int pnfx_pn_rows_fwd(const void* raw, int64_t raw_rs, void* w, int64_t w_rs, float* M, float* Z,
                     int32_t* Nmax, int64_t R, int64_t N, const float* tau, float scale, float p,
                     float gamma, int has_gamma, int causal, int dtype, void* stream);

/*
 * Backward of pnfx_pn_rows_fwd: d_raw (row stride draw_rs, dtype of raw) and
 * one fp32 partial per row, dtau_rows[r] = -sum_j du[r, j].  Replaces
 * _pn_fir_tau_row_bwd_kernel (src/triton_pnfirtau.py:214-303) through
 * _TritonPnFirTauScoresFn.backward (:754-785).
 */
int pnfx_pn_rows_bwd(const void* dw, int64_t dw_rs, const void* raw, int64_t raw_rs,
                     const float* M, const float* Z, const int32_t* Nmax, void* draw,
                     int64_t draw_rs, float* dtau_rows, int64_t R, int64_t N, const float* tau,
                     float scale, float p, float gamma, int has_gamma, int causal, int dtype,
                     void* stream);

/*
 * Flash pn_fir_tau attention forward (p = 10, peak gate), O(N) memory.
 *   q, k, v, o : [B, H, N, D] with strides (s?b, s?h, s?n, 1), same dtype; bf16:
 *                16-byte aligned, strides multiples of 8, row strides s?n < 2^25
 *   o_lo       : optional (may be NULL; bf16 only), o's strides: the bf16 rounding
 *                residual of O (fp32 O = o + o_lo to ~16 mantissa bits), which
 *                pnfx_flash_bwd uses to form D = <dO, O>/gate accurately
 *   M, Z       : fp32 [B, H, N] contiguous
 *   Nmax       : optional (may be NULL) int32 [B, H, N]: the number of keys tied
 *                at the peak (0 on silent rows).  Counting costs two VALU ops per
 *                score, so pass NULL unless the counts themselves are wanted: the
 *                backward does not need them (it counts ties in its dQ stage).
 *   tile_mask  : optional (may be NULL) uint8 [B*H, ceil(N/32), ceil(N/64)]:
 *                1 where the 32-query x 64-key sub-tile has a positive
 *                rectified score (the skip rule of src/triton_pnfirtau.py:395-400
 *                at 32-row granularity; OR adjacent row pairs for the 64x64 view).
 *   workspace  : optional (may be NULL), pnfx_flash_fwd_workspace_size(B, H, N, D)
 *                bytes, 256-byte aligned.  With it (bf16, tau > 0) the forward first
 *                takes the largest key norm of every 64-key tile and skips, without
 *                forming their scores or loading their K/V, the tiles where
 *                max|q| max|k| scale <= tau (Cauchy-Schwarz: every score is then
 *                <= 0).  Results are identical with and without it.
 * D in {16, 32, 64, 128}.  Replaces _flash_pn_fir_tau_fwd_kernel
 * (src/triton_pnfirtau.py:313-443) through _FlashPnFirTauFn.forward (:816-898).
 */
int pnfx_flash_fwd(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k,
                   int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                   int64_t vsh, int64_t vsn, void* o, int64_t osb, int64_t osh, int64_t osn,
                   void* o_lo, float* M, float* Z, int32_t* Nmax, uint8_t* tile_mask,
                   void* workspace, int64_t workspace_bytes, int64_t B, int64_t H,
                   int64_t N, int64_t D, const float* tau, float scale, float gamma,
                   int has_gamma, int causal, int dtype, void* stream);

/*
 * pnfx_flash_fwd with the causal FIR of the keys fused into the kernel's key-tile load:
 * k_raw holds the raw (pre-FIR) keys, taps / taps_rows / K are those of pnfx_fir_fwd
 * (K <= 7), and every key tile is filtered in LDS from its raw rows and 6-row halo with
 * pnfx_fir_fwd's arithmetic, so O, o_lo, M, Z and the tile mask are bitwise those of
 * pnfx_fir_fwd followed by pnfx_flash_fwd.  bf16, D in {16, 32, 64}, no tie counts, no
 * silent-tile bound.  Replaces src/pnfirtau_attention.py:299-315's separate causal_fir +
 * flash_pn_fir_tau_attention launches for a forward that needs no filtered keys afterwards
 * (inference).  It filters every key tile once per 128-query block that reads it: faster than
 * the two launches for short sequences (0.80x the GPU time at B=64 H=4 N=256 d=16), slower
 * for long ones (1.64x at N=8192); PnFirTauFlashMHA uses it for inference up to N = 512.
 */
int pnfx_flash_fwd_fir(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k_raw,
                       int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                       int64_t vsh, int64_t vsn, void* o, int64_t osb, int64_t osh, int64_t osn,
                       void* o_lo, float* M, float* Z, uint8_t* tile_mask, int64_t B,
                       int64_t H, int64_t N, int64_t D, const float* tau, float scale,
                       float gamma, int has_gamma, int causal, const float* taps,
                       int64_t taps_rows, int K, int dtype, void* stream);

/* Bytes of the optional pnfx_flash_fwd workspace for this shape (the per-tile key
 * norms of its silent-tile bound).  No counterpart in the reference. */
int64_t pnfx_flash_fwd_workspace_size(int64_t B, int64_t H, int64_t N, int64_t D);

/* Bytes of device workspace pnfx_flash_bwd needs for this shape. */
int64_t pnfx_flash_bwd_workspace_size(int64_t B, int64_t H, int64_t N, int64_t D);

/*
 * Flash backward.  Inputs as saved by the forward (q, k, v, o, o_lo, M, Z,
 * tile_mask -- o_lo and tile_mask may be NULL; without tile_mask every causal
 * tile is recomputed),
 * dO with its own strides.  Outputs dq, dk, dv ([B,H,N,D] with their own
 * strides, dtype of q) and dtau (one fp32: the fp64 sum of all per-tile
 * partials rounded once, as src/triton_pnfirtau.py:959).  Deterministic: no
 * atomics; the same inputs give bitwise the same outputs.  workspace must hold
 * pnfx_flash_bwd_workspace_size(B, H, N, D) bytes, 256-byte aligned.
 * Replaces _flash_pn_fir_tau_bwd_kernel (src/triton_pnfirtau.py:445-621)
 * through _FlashPnFirTauFn.backward (:900-968).
 */
int pnfx_flash_bwd(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k,
                   int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                   int64_t vsh, int64_t vsn, const void* o, int64_t osb, int64_t osh,
                   int64_t osn, const void* o_lo, const void* dout, int64_t dosb, int64_t dosh, int64_t dosn,
                   const float* M, const float* Z,
                   const uint8_t* tile_mask, void* dq, int64_t dqsb, int64_t dqsh,
                   int64_t dqsn, void* dk, int64_t dksb, int64_t dksh, int64_t dksn, void* dv,
                   int64_t dvsb, int64_t dvsh, int64_t dvsn, float* dtau, void* workspace,
                   int64_t workspace_bytes, int64_t B, int64_t H, int64_t N, int64_t D,
                   const float* tau, float scale, float gamma, int has_gamma, int causal,
                   int dtype, void* stream);

/*
 * The three stages of pnfx_flash_bwd, callable separately (same arguments,
 * plus a stage mask), and run in this order on one workspace: PNFX_BWD_PREPARE
 * forms the per-row constants (and clears the key-tile activity bytes);
 * PNFX_BWD_DQ writes dq and the tau partials, stores each row's peak-tie share
 * and marks the 64-key tiles with an active tile_mask entry; PNFX_BWD_DKDV (which
 * reads all of these) writes dk, dv and (bf16) dtau.  For fp32 the DQ stage writes
 * dtau.  pnfx_flash_bwd is the mask PNFX_BWD_ALL.
 */
#define PNFX_BWD_PREPARE 1
#define PNFX_BWD_DKDV 2
#define PNFX_BWD_DQ 4
#define PNFX_BWD_ALL 7
int pnfx_flash_bwd_stages(int stages, const void* q, int64_t qsb, int64_t qsh, int64_t qsn,
                          const void* k, int64_t ksb, int64_t ksh, int64_t ksn, const void* v,
                          int64_t vsb, int64_t vsh, int64_t vsn, const void* o, int64_t osb,
                          int64_t osh, int64_t osn, const void* o_lo, const void* dout,
                          int64_t dosb, int64_t dosh, int64_t dosn, const float* M,
                          const float* Z, const uint8_t* tile_mask,
                          void* dq, int64_t dqsb, int64_t dqsh, int64_t dqsn, void* dk,
                          int64_t dksb, int64_t dksh, int64_t dksn, void* dv, int64_t dvsb,
                          int64_t dvsh, int64_t dvsn, float* dtau, void* workspace,
                          int64_t workspace_bytes, int64_t B, int64_t H, int64_t N, int64_t D,
                          const float* tau, float scale, float gamma, int has_gamma, int causal,
                          int dtype, void* stream);

/*
 * pnfx_flash_bwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments and results as
 * pnfx_flash_bwd (bitwise the same outputs); the workspace is a scratch array of
 * PNFX_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on until the
 * process ends (it is part of the library's code object: every process that loads
 * libpnfx.so holds it on each GPU the library initialises, whether or not this entry point
 * is called).  Shapes whose pnfx_flash_bwd_workspace_size exceeds that return PNFX_EINVAL
 * (C4, B=4 H=16 N=8192 D=64, needs 86 MB and fits).  Allocates nothing: the first call on
 * a device looks up the array's address there (the current device must be the stream's).
 * Every call on one GPU uses the same array: calls that overlap on one GPU (different
 * streams or threads, or a captured HIP graph replayed while another call or replay of one
 * runs) race on it and give wrong results; serialise them.
 */
#define PNFX_NOALLOC_SCRATCH_BYTES (128ll << 20)
int pnfx_flash_bwd_noalloc(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k,
                           int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                           int64_t vsh, int64_t vsn, const void* o, int64_t osb, int64_t osh,
                           int64_t osn, const void* o_lo, const void* dout, int64_t dosb,
                           int64_t dosh, int64_t dosn, const float* M, const float* Z,
                           const uint8_t* tile_mask, void* dq, int64_t dqsb, int64_t dqsh,
                           int64_t dqsn, void* dk, int64_t dksb, int64_t dksh, int64_t dksn,
                           void* dv, int64_t dvsb, int64_t dvsh, int64_t dvsn, float* dtau,
                           int64_t B, int64_t H, int64_t N, int64_t D, const float* tau,
                           float scale, float gamma, int has_gamma, int causal, int dtype,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PNFX_H_ */
