// C-ABI entry points of the flash path: argument checks, workspace carving, dtype dispatch.
#include <mutex>

#include "flash.h"

// Scratch memory of pnfx_flash_bwd_noalloc: the backward's workspace for callers that cannot
// allocate.  Each GPU the library runs on holds its own copy until the process ends.  In
// host code `scratch` names a host-side stand-in, not device memory: its device address is
// taken once per device with hipGetSymbolAddress (scratch_address below) and only that
// address is handed to kernels.
static __device__ __align__(256) uint8_t scratch[PNFX_NOALLOC_SCRATCH_BYTES];

namespace pnfx {
namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Each [B, H, N, D] operand must have unit inner stride; the bf16 MFMA kernels read and
// write whole 16-byte (8-element) chunks of a row, and their tile loads address the rows of a
// 64-row tile by 32-bit byte offsets from the tile's first row (2 * 63 * sn < 2^32).
int check_operand(const char* name, const void* p, int64_t sb, int64_t sh, int64_t sn, int dtype) {
  PNFX_REQUIRE(p != nullptr, "flash: %s is null", name);
  if (dtype == PNFX_BF16) {
    PNFX_REQUIRE(aligned16(p) && sb % 8 == 0 && sh % 8 == 0 && sn % 8 == 0,
                 "flash: %s must be 16-byte aligned with strides that are multiples of 8 "
                 "elements (got %lld, %lld, %lld)",
                 name, (long long)sb, (long long)sh, (long long)sn);
    PNFX_REQUIRE(sn >= 0 && sn < (1ll << 25), "flash: %s row stride %lld outside [0, 2^25)",
                 name, (long long)sn);
  }
  return PNFX_OK;
}

int check_shape(int64_t B, int64_t H, int64_t N, int64_t D) {
  PNFX_REQUIRE(B >= 1 && H >= 1 && N >= 1, "flash: bad shape B=%lld H=%lld N=%lld", (long long)B,
               (long long)H, (long long)N);
  PNFX_REQUIRE(D == 16 || D == 32 || D == 64 || D == 128, "flash: head dim %lld not in {16,32,64,128}",
               (long long)D);
  PNFX_REQUIRE(B * H <= (1ll << 30) && N <= (1ll << 28) && B * H * ((N + 127) / 128) < (1ll << 31),
               "flash: shape too large for the launch grid");
  return PNFX_OK;
}

// Device address of `scratch` on the current device, taken on the first call on that device
// (with it current) and kept per device.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("flash_bwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return PNFX_ELAUNCH;
  }
  PNFX_REQUIRE(dev >= 0 && dev < kMaxDevices, "flash_bwd_noalloc: device %d out of range", dev);
  if (stream) {
    int sdev = -1;
    e = hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) {
      set_error("flash_bwd_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
      return PNFX_ELAUNCH;
    }
    PNFX_REQUIRE(sdev == dev, "flash_bwd_noalloc: the stream is on device %d, device %d is current",
                 sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("flash_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(e));
      return PNFX_ELAUNCH;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return PNFX_OK;
}

}  // namespace
}  // namespace pnfx

using namespace pnfx;

extern "C" int64_t pnfx_flash_fwd_workspace_size(int64_t B, int64_t H, int64_t N, int64_t D) {
  (void)D;
  return BwdWorkspace::round256(B * H * ((N + 63) / 64) * 4);
}

extern "C" int pnfx_flash_fwd(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k,
                              int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                              int64_t vsh, int64_t vsn, void* o, int64_t osb, int64_t osh,
                              int64_t osn, void* o_lo, float* M, float* Z, int32_t* Nmax,
                              uint8_t* tile_mask, void* workspace, int64_t workspace_bytes,
                              int64_t B, int64_t H, int64_t N, int64_t D, const float* tau,
                              float scale, float gamma, int has_gamma, int causal, int dtype,
                              void* stream) {
  int rc;
  if ((rc = check_shape(B, H, N, D))) return rc;
  PNFX_REQUIRE(dtype == PNFX_BF16 || dtype == PNFX_F32, "flash: unsupported dtype %d", dtype);
  if ((rc = check_operand("q", q, qsb, qsh, qsn, dtype))) return rc;
  if ((rc = check_operand("k", k, ksb, ksh, ksn, dtype))) return rc;
  if ((rc = check_operand("v", v, vsb, vsh, vsn, dtype))) return rc;
  if ((rc = check_operand("o", o, osb, osh, osn, dtype))) return rc;
  PNFX_REQUIRE(M && Z && tau, "flash_fwd: null statistics / tau pointer");
  PNFX_REQUIRE(!o_lo || (dtype == PNFX_BF16 && aligned16(o_lo)),
               "flash_fwd: o_lo is a 16-byte aligned bf16 buffer with o's strides");
  const int64_t fws = pnfx_flash_fwd_workspace_size(B, H, N, D);
  PNFX_REQUIRE(!workspace || (workspace_bytes >= fws &&
                              (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0),
               "flash_fwd: workspace needs %lld bytes, 256-byte aligned (got %lld)",
               (long long)fws, (long long)workspace_bytes);
  FwdParams fp{q, k, v, o, o_lo, qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn,
               M, Z, Nmax, tile_mask, static_cast<float*>(workspace), (int)B, (int)H, (int)N,
               (int)((N + 31) / 32), (int)((N + 63) / 64), tau, scale, gamma, has_gamma != 0};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return dtype == PNFX_BF16 ? flash_fwd_bf16(fp, D, causal != 0, st)
                            : flash_fwd_f32(fp, D, causal != 0, has_gamma != 0, st);
}

extern "C" int pnfx_flash_fwd_fir(const void* q, int64_t qsb, int64_t qsh, int64_t qsn,
                                  const void* k_raw, int64_t ksb, int64_t ksh, int64_t ksn,
                                  const void* v, int64_t vsb, int64_t vsh, int64_t vsn, void* o,
                                  int64_t osb, int64_t osh, int64_t osn, void* o_lo, float* M,
                                  float* Z, uint8_t* tile_mask, int64_t B, int64_t H, int64_t N,
                                  int64_t D, const float* tau, float scale, float gamma,
                                  int has_gamma, int causal, const float* taps, int64_t taps_rows,
                                  int K, int dtype, void* stream) {
  int rc;
  if ((rc = check_shape(B, H, N, D))) return rc;
  PNFX_REQUIRE(dtype == PNFX_BF16, "flash_fwd_fir: bf16 only (dtype %d)", dtype);
  if ((rc = check_operand("q", q, qsb, qsh, qsn, dtype))) return rc;
  if ((rc = check_operand("k_raw", k_raw, ksb, ksh, ksn, dtype))) return rc;
  if ((rc = check_operand("v", v, vsb, vsh, vsn, dtype))) return rc;
  if ((rc = check_operand("o", o, osb, osh, osn, dtype))) return rc;
  PNFX_REQUIRE(M && Z && tau && taps, "flash_fwd_fir: null statistics / tau / taps pointer");
  PNFX_REQUIRE(!o_lo || aligned16(o_lo), "flash_fwd_fir: o_lo is a 16-byte aligned bf16 buffer");
  PNFX_REQUIRE(K >= 1 && K <= 7, "flash_fwd_fir: FIR length K=%d outside [1, 7]", K);
  PNFX_REQUIRE(taps_rows == 1 || taps_rows == H, "flash_fwd_fir: taps_rows=%lld must be 1 or H=%lld",
               (long long)taps_rows, (long long)H);
  FwdParams fp{q, k_raw, v, o, o_lo, qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn,
               M, Z, nullptr, tile_mask, nullptr, (int)B, (int)H, (int)N,
               (int)((N + 31) / 32), (int)((N + 63) / 64), tau, scale, gamma, has_gamma != 0,
               taps, (int)taps_rows, K};
  return flash_fwd_fir_bf16(fp, D, causal != 0, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int64_t pnfx_flash_bwd_workspace_size(int64_t B, int64_t H, int64_t N, int64_t D) {
  return BwdWorkspace(B, H, N, D).total();
}

extern "C" int pnfx_flash_bwd_stages(int stages, const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k,
                              int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                              int64_t vsh, int64_t vsn, const void* o, int64_t osb, int64_t osh,
                              int64_t osn, const void* o_lo, const void* dout, int64_t dosb,
                              int64_t dosh,
                              int64_t dosn, const float* M, const float* Z,
                              const uint8_t* tile_mask, void* dq, int64_t dqsb, int64_t dqsh,
                              int64_t dqsn, void* dk, int64_t dksb, int64_t dksh, int64_t dksn,
                              void* dv, int64_t dvsb, int64_t dvsh, int64_t dvsn, float* dtau,
                              void* workspace, int64_t workspace_bytes, int64_t B, int64_t H,
                              int64_t N, int64_t D, const float* tau, float scale, float gamma,
                              int has_gamma, int causal, int dtype, void* stream) {
  int rc;
  PNFX_REQUIRE(stages > 0 && (stages & ~PNFX_BWD_ALL) == 0, "flash_bwd: bad stage mask %d", stages);
  if ((rc = check_shape(B, H, N, D))) return rc;
  PNFX_REQUIRE(dtype == PNFX_BF16 || dtype == PNFX_F32, "flash: unsupported dtype %d", dtype);
  if ((rc = check_operand("q", q, qsb, qsh, qsn, dtype))) return rc;
  if ((rc = check_operand("k", k, ksb, ksh, ksn, dtype))) return rc;
  if ((rc = check_operand("v", v, vsb, vsh, vsn, dtype))) return rc;
  if ((rc = check_operand("o", o, osb, osh, osn, dtype))) return rc;
  if ((rc = check_operand("dout", dout, dosb, dosh, dosn, dtype))) return rc;
  if ((rc = check_operand("dq", dq, dqsb, dqsh, dqsn, dtype))) return rc;
  if ((rc = check_operand("dk", dk, dksb, dksh, dksn, dtype))) return rc;
  if ((rc = check_operand("dv", dv, dvsb, dvsh, dvsn, dtype))) return rc;
  PNFX_REQUIRE(M && Z && tau && dtau, "flash_bwd: null statistics / tau pointer");
  PNFX_REQUIRE(!o_lo || (dtype == PNFX_BF16 && aligned16(o_lo)),
               "flash_bwd: o_lo is a 16-byte aligned bf16 buffer with o's strides");
  const BwdWorkspace wl(B, H, N, D);
  PNFX_REQUIRE(workspace && workspace_bytes >= wl.total() &&
                   (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
               "flash_bwd: workspace needs %lld bytes, 256-byte aligned (got %lld)",
               (long long)wl.total(), (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  float* rcbuf = reinterpret_cast<float*>(ws);
  double* parts = reinterpret_cast<double*>(ws + wl.rc_bytes);
  void* qs = wl.xt_bytes ? ws + wl.rc_bytes + wl.parts_bytes : nullptr;
  uint8_t* ktact = tile_mask ? reinterpret_cast<uint8_t*>(ws + wl.rc_bytes + wl.parts_bytes +
                                                          wl.xt_bytes)
                             : nullptr;
  uint8_t* amap = (tile_mask && wl.amap_bytes)
                      ? reinterpret_cast<uint8_t*>(ws + wl.rc_bytes + wl.parts_bytes +
                                                   wl.xt_bytes + wl.kt_bytes)
                      : nullptr;
  BwdParams bp{q, k, v, o, o_lo, dout, dq, dk, dv,
               qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn, osb, osh, osn, dosb, dosh, dosn,
               dqsb, dqsh, dqsn, dksb, dksh, dksn, dvsb, dvsh, dvsn,
               M, Z, tile_mask, rcbuf, parts, qs, ktact, amap, dtau,
               (int)B, (int)H, (int)N, (int)((N + 31) / 32), (int)((N + 63) / 64),
               bwd_nkvb(N, D), tau, scale, gamma};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return dtype == PNFX_BF16 ? flash_bwd_bf16(bp, D, causal != 0, has_gamma != 0, stages, st)
                            : flash_bwd_f32(bp, D, causal != 0, has_gamma != 0, stages, st);
}

extern "C" int pnfx_flash_bwd(const void* q, int64_t qsb, int64_t qsh, int64_t qsn, const void* k,
                              int64_t ksb, int64_t ksh, int64_t ksn, const void* v, int64_t vsb,
                              int64_t vsh, int64_t vsn, const void* o, int64_t osb, int64_t osh,
                              int64_t osn, const void* o_lo, const void* dout, int64_t dosb,
                              int64_t dosh, int64_t dosn, const float* M, const float* Z,
                              const uint8_t* tile_mask, void* dq,
                              int64_t dqsb, int64_t dqsh, int64_t dqsn, void* dk, int64_t dksb,
                              int64_t dksh, int64_t dksn, void* dv, int64_t dvsb, int64_t dvsh,
                              int64_t dvsn, float* dtau, void* workspace, int64_t workspace_bytes,
                              int64_t B, int64_t H, int64_t N, int64_t D, const float* tau,
                              float scale, float gamma, int has_gamma, int causal, int dtype,
                              void* stream) {
  return pnfx_flash_bwd_stages(PNFX_BWD_ALL, q, qsb, qsh, qsn, k, ksb, ksh, ksn, v, vsb, vsh, vsn,
                               o, osb, osh, osn, o_lo, dout, dosb, dosh, dosn, M, Z,
                               tile_mask, dq, dqsb, dqsh, dqsn, dk, dksb, dksh, dksn, dv, dvsb,
                               dvsh, dvsn, dtau, workspace, workspace_bytes, B, H, N, D, tau,
                               scale, gamma, has_gamma, causal, dtype, stream);
}

extern "C" int pnfx_flash_bwd_noalloc(const void* q, int64_t qsb, int64_t qsh, int64_t qsn,
                                      const void* k, int64_t ksb, int64_t ksh, int64_t ksn,
                                      const void* v, int64_t vsb, int64_t vsh, int64_t vsn,
                                      const void* o, int64_t osb, int64_t osh, int64_t osn,
                                      const void* o_lo, const void* dout, int64_t dosb,
                                      int64_t dosh, int64_t dosn, const float* M, const float* Z,
                                      const uint8_t* tile_mask, void* dq, int64_t dqsb,
                                      int64_t dqsh, int64_t dqsn, void* dk, int64_t dksb,
                                      int64_t dksh, int64_t dksn, void* dv, int64_t dvsb,
                                      int64_t dvsh, int64_t dvsn, float* dtau, int64_t B,
                                      int64_t H, int64_t N, int64_t D, const float* tau,
                                      float scale, float gamma, int has_gamma, int causal,
                                      int dtype, void* stream) {
  int rc;
  if ((rc = check_shape(B, H, N, D))) return rc;
  const int64_t need = pnfx_flash_bwd_workspace_size(B, H, N, D);
  PNFX_REQUIRE(need <= (int64_t)PNFX_NOALLOC_SCRATCH_BYTES,
               "flash_bwd_noalloc: B=%lld H=%lld N=%lld D=%lld needs %lld bytes of scratch, "
               "more than the %lld the library holds (use pnfx_flash_bwd with a workspace)",
               (long long)B, (long long)H, (long long)N, (long long)D, (long long)need,
               (long long)PNFX_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_address(stream, &ws))) return rc;
  // Nothing in the scratch needs clearing: every byte the kernels read is written earlier in
  // the same call (the key-tile activity bytes are zeroed by the prepare kernel).
  return pnfx_flash_bwd_stages(PNFX_BWD_ALL, q, qsb, qsh, qsn, k, ksb, ksh, ksn, v, vsb, vsh, vsn,
                               o, osb, osh, osn, o_lo, dout, dosb, dosh, dosn, M, Z, tile_mask,
                               dq, dqsb, dqsh, dqsn, dk, dksb, dksh, dksn, dv, dvsb, dvsh, dvsn,
                               dtau, ws, (int64_t)PNFX_NOALLOC_SCRATCH_BYTES, B, H, N, D, tau,
                               scale, gamma, has_gamma, causal, dtype, stream);
}
