// torch.library registration of the pnfx ops (namespace pnfx) over the C ABI of libpnfx.so.
//
// Host-only C++: every op checks and lays out its operands, allocates its outputs with torch's
// caching allocator on the input's device, and enqueues the HIP kernels on the current stream
// through include/pnfx.h; nothing blocks the host.  Kernels are registered for the CUDA (= HIP)
// dispatch key only, so CPU tensors are refused by the dispatcher; autograd is registered here
// too (Autograd key), so a forward + backward never leaves C++.  Fake (meta) kernels for
// torch.compile live in ops.py.
//
// op                        reference counterpart (src/triton_pnfirtau.py)
// pnfx::fir_fwd / fir_bwd   _TritonCausalFir7Fn         :629-682
// pnfx::pn_rows_fwd / _bwd  _TritonPnFirTauScoresFn     :694-785
// pnfx::flash_fwd / _bwd    _FlashPnFirTauFn            :814-968
// pnfx::flash_fwd_fir       (none: the FIR fused into the forward's key-tile load)
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include "../../include/pnfx.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == PNFX_OK, what, " failed (", rc, "): ", pnfx_last_error());
}

int dtype_code(const Tensor& t, const char* what) {
  if (t.scalar_type() == at::kFloat) return PNFX_F32;
  if (t.scalar_type() == at::kBFloat16) return PNFX_BF16;
  TORCH_CHECK_TYPE(false, what, ": dtype ", t.scalar_type(),
                   " is not supported (float32, bfloat16)");
  return -1;
}

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// tau as one fp32 value on the operands' device (the kernels read tau[0] there)
Tensor tau32(const Tensor& tau, const Tensor& like) {
  TORCH_CHECK_VALUE(tau.numel() == 1, "tau must hold one value, got shape ", tau.sizes());
  if (tau.scalar_type() == at::kFloat && tau.device() == like.device()) return tau;
  return tau.reshape({1}).to(like.device(), at::kFloat);
}

// A tensor the forward produced and a backward op is handed back (row statistics, tile
// mask): the kernels index it by row with no size of their own, so it must have the
// forward's layout: n contiguous elements of type st on the operands' device.
void check_saved(const Tensor& t, const char* op_name, const char* name, int64_t n,
                 at::ScalarType st, const Tensor& like) {
  TORCH_CHECK_TYPE(t.scalar_type() == st, op_name, ": ", name, " is ", t.scalar_type(),
                   ", the forward's is ", st);
  TORCH_CHECK_VALUE(t.numel() == n && t.is_contiguous(), op_name, ": ", name,
                    " must be the forward's contiguous ", n, " elements, got shape ", t.sizes(),
                    " with strides ", t.strides());
  TORCH_CHECK_VALUE(t.device() == like.device(), op_name, ": ", name, " is on ", t.device(),
                    ", the operands on ", like.device());
}

// -------------------------------------------------------------------------------- FIR
// x [B,N,C] or [B,H,N,C] with unit channel stride, seen as 4-D.
Tensor fir_call(const Tensor& x_in, const Tensor& taps, bool adjoint) {
  const char* what = adjoint ? "pnfx_fir_bwd" : "pnfx_fir_fwd";
  Tensor x = x_in.stride(-1) == 1 ? x_in : x_in.contiguous();
  TORCH_CHECK_VALUE(x.dim() == 3 || x.dim() == 4, "FIR input must be [B,N,C] or [B,H,N,C], got ",
                    x.sizes());
  const Tensor x4 = x.dim() == 3 ? x.unsqueeze(1) : x;
  Tensor taps2 = taps.reshape({-1, taps.size(-1)});
  if (taps2.scalar_type() != at::kFloat || !taps2.is_contiguous() ||
      taps2.device() != x.device())
    taps2 = taps2.to(x.device(), at::kFloat).contiguous();
  Tensor y = at::empty(x.sizes(), x.options());
  if (y.numel() == 0) return y;  // nothing to filter (the reference launches an empty grid)
  const c10::DeviceGuard guard(x.device());
  auto fn = adjoint ? pnfx_fir_bwd : pnfx_fir_fwd;
  check_rc(fn(x4.data_ptr(), x4.stride(0), x4.stride(1), x4.stride(2), y.data_ptr(), x4.size(0),
              x4.size(1), x4.size(2), x4.size(3), taps2.data_ptr<float>(), taps2.size(0),
              (int)taps2.size(1), dtype_code(x, "fir"), stream_of(x)),
           what);
  return y;
}

Tensor fir_fwd_cuda(const Tensor& x, const Tensor& taps) { return fir_call(x, taps, false); }
Tensor fir_bwd_cuda(const Tensor& gy, const Tensor& taps) { return fir_call(gy, taps, true); }

// ------------------------------------------------------------------------- row scores
// Rows of a [..., N, N] score tensor: the product of every extent but the last.
int64_t n_rows(const Tensor& raw) {
  int64_t R = 1;
  for (int64_t i = 0; i + 1 < raw.dim(); ++i) R *= raw.size(i);
  return R;
}

std::tuple<Tensor, Tensor, Tensor, Tensor> pn_rows_fwd_cuda(const Tensor& raw, const Tensor& tau,
                                                            double scale, double p, double gamma,
                                                            bool has_gamma, bool causal) {
  const int64_t N = raw.size(-1);
  const int64_t R = n_rows(raw);
  const Tensor r2 = raw.contiguous().view({R, N});
  Tensor w = at::empty_like(r2);
  const auto f32 = raw.options().dtype(at::kFloat);
  Tensor M = at::empty({R}, f32), Z = at::empty({R}, f32);
  Tensor Nm = at::empty({R}, raw.options().dtype(at::kInt));
  if (r2.numel() == 0) {  // no rows, or rows of length 0 (peak 0, mass 0 + 1e-12, no ties)
    M.zero_();
    Z.fill_(1e-12);
    Nm.zero_();
    return {w.view(raw.sizes()), M, Z, Nm};
  }
  const c10::DeviceGuard guard(raw.device());
  const Tensor t32 = tau32(tau, raw);
  check_rc(pnfx_pn_rows_fwd(r2.data_ptr(), N, w.data_ptr(), N, M.data_ptr<float>(),
                            Z.data_ptr<float>(), Nm.data_ptr<int32_t>(), R, N,
                            t32.data_ptr<float>(), (float)scale, (float)p, (float)gamma,
                            has_gamma, causal, dtype_code(raw, "pn_rows"), stream_of(raw)),
           "pnfx_pn_rows_fwd");
  return {w.view(raw.sizes()), M, Z, Nm};
}

std::tuple<Tensor, Tensor> pn_rows_bwd_cuda(const Tensor& dw, const Tensor& raw, const Tensor& tau,
                                            const Tensor& M, const Tensor& Z, const Tensor& Nmax,
                                            double scale, double p, double gamma, bool has_gamma,
                                            bool causal) {
  TORCH_CHECK_VALUE(dw.sizes() == raw.sizes(), "pn_rows_bwd: dw has shape ", dw.sizes(),
                    ", raw ", raw.sizes());
  const int64_t N = raw.size(-1);
  const int64_t R = n_rows(raw);
  check_saved(M, "pn_rows_bwd", "M", R, at::kFloat, raw);
  check_saved(Z, "pn_rows_bwd", "Z", R, at::kFloat, raw);
  check_saved(Nmax, "pn_rows_bwd", "Nmax", R, at::kInt, raw);
  const Tensor r2 = raw.contiguous().view({R, N});
  const Tensor g2 = dw.to(raw.scalar_type()).contiguous().view({R, N});
  Tensor d = at::empty_like(r2);
  Tensor dt = at::empty({R}, raw.options().dtype(at::kFloat));
  if (r2.numel() == 0) return {d.view(raw.sizes()), dt.zero_()};
  const c10::DeviceGuard guard(raw.device());
  const Tensor t32 = tau32(tau, raw);
  check_rc(pnfx_pn_rows_bwd(g2.data_ptr(), N, r2.data_ptr(), N, M.data_ptr<float>(),
                            Z.data_ptr<float>(), Nmax.data_ptr<int32_t>(), d.data_ptr(), N,
                            dt.data_ptr<float>(), R, N, t32.data_ptr<float>(), (float)scale,
                            (float)p, (float)gamma, has_gamma, causal, dtype_code(raw, "pn_rows"),
                            stream_of(raw)),
           "pnfx_pn_rows_bwd");
  return {d.view(raw.sizes()), dt};
}

// ------------------------------------------------------------------------------ flash
// Past this sequence length the forward records no silence map (N^2/2048 bytes per (b, h));
// the backward then recomputes every causal tile.  Kept equal to ops.MASK_MAX_N.
constexpr int64_t kMaskMaxN = 65536;

std::array<int64_t, 3> mask_shape(int64_t B, int64_t H, int64_t N) {
  if (N > kMaskMaxN) return {0, 0, 0};
  return {B * H, (N + 31) / 32, (N + 63) / 64};
}

// t with unit inner stride and (bf16) a 16-byte-aligned base and 8-element-multiple strides.
Tensor bhnd(const Tensor& t, const char* name, bool bf16) {
  TORCH_CHECK_VALUE(t.dim() == 4, name, " must be [B,H,N,D], got ", t.sizes());
  bool ok = t.stride(3) == 1;
  if (ok && bf16)
    ok = reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 && t.stride(0) % 8 == 0 &&
         t.stride(1) % 8 == 0 && t.stride(2) % 8 == 0;
  return ok ? t : t.contiguous();
}

// q, k and v must agree in shape, dtype and device: the kernels read all three with q's
// element size and extents.
void check_qkv(const Tensor& q, const Tensor& k, const Tensor& v) {
  for (const auto& [name, t] : {std::pair<const char*, const Tensor&>{"k", k}, {"v", v}}) {
    TORCH_CHECK_VALUE(t.sizes() == q.sizes(), "flash: ", name, " has shape ", t.sizes(),
                      ", q has ", q.sizes());
    TORCH_CHECK_TYPE(t.scalar_type() == q.scalar_type(), "flash: ", name, " is ",
                     t.scalar_type(), ", q is ", q.scalar_type());
    TORCH_CHECK_VALUE(t.device() == q.device(), "flash: ", name, " is on ", t.device(),
                      ", q on ", q.device());
  }
}

// O and its bf16 rounding residual (bf16 only), each [B,H,N,D] and each its own allocation
// (the schema declares no aliasing between outputs); with o_bnhd backed by [B,N,H,D] rows, so
// that the caller's transpose back to [B,N,H*D] is free.
std::pair<Tensor, Tensor> new_o_pair(const Tensor& q, bool o_bnhd, bool with_lo) {
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const auto one = [&]() {
    return o_bnhd ? at::empty({B, N, H, D}, q.options()).permute({0, 2, 1, 3})
                  : at::empty({B, H, N, D}, q.options());
  };
  return {one(), with_lo ? one() : q.new_empty({0})};
}

const void* ptr_or_null(const Tensor& t) { return t.numel() ? t.data_ptr() : nullptr; }

// Head sizes with a kernel of their own; any other size up to 128 is zero-padded to the next
// one (as the reference pads D to BLOCK_D = next_pow2(max(D, 16)) with masked loads,
// src/triton_pnfirtau.py:839-841): zero columns add exact zeros to every dot product, so the
// scores, O and the gradients' real columns are those of the unpadded problem.
bool kernel_head_dim(int64_t D) { return D == 16 || D == 32 || D == 64 || D == 128; }
int64_t padded_head_dim(int64_t D) { return D <= 16 ? 16 : D <= 32 ? 32 : D <= 64 ? 64 : 128; }
Tensor pad_d(const Tensor& t, int64_t Dp) {
  return t.numel() ? at::constant_pad_nd(t, {0, Dp - t.size(-1)}) : t;
}
void check_head_dim(int64_t D) {
  TORCH_CHECK_VALUE(D >= 1 && D <= 128, "flash: head dim ", D,
                    " has no flash kernel (1..128; flash_pn_fir_tau_attention and "
                    "PnFirTauFlashMHA take the materialised-score path above 128)");
}

// A problem this small spends less time in the forward than the key-norm pass of the
// silent-tile bound costs to launch: below it the forward runs without the bound (same results).
constexpr int64_t kBoundMinScores = int64_t(1) << 26;  // B*H*N^2, e.g. B*H = 64 at N = 1024

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> flash_fwd_cuda(
    const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, const Tensor& tau, double scale,
    double gamma, bool has_gamma, bool causal, bool o_bnhd, bool with_nmax) {
  check_qkv(q_in, k_in, v_in);
  const int code = dtype_code(q_in, "flash");
  const bool bf = code == PNFX_BF16;
  TORCH_CHECK_VALUE(q_in.dim() == 4, "q must be [B,H,N,D], got ", q_in.sizes());
  if (!kernel_head_dim(q_in.size(3))) {
    const int64_t D = q_in.size(3);
    check_head_dim(D);
    const int64_t Dp = padded_head_dim(D);
    auto [o, o_lo, M, Z, Nm, mask] = flash_fwd_cuda(pad_d(q_in, Dp), pad_d(k_in, Dp),
                                                    pad_d(v_in, Dp), tau, scale, gamma, has_gamma,
                                                    causal, false, with_nmax);
    auto [oo, oo_lo] = new_o_pair(q_in, o_bnhd, bf);
    oo.copy_(o.narrow(3, 0, D));
    if (bf) oo_lo.copy_(o_lo.narrow(3, 0, D));
    return {oo, oo_lo, M, Z, Nm, mask};
  }
  const Tensor q = bhnd(q_in, "q", bf), k = bhnd(k_in, "k", bf), v = bhnd(v_in, "v", bf);
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  auto [o, o_lo] = new_o_pair(q, o_bnhd, bf);
  // M, Z (fp32 [B,H,N]), Nmax (int32, only when asked for) and the tile mask (N^2/2048 bytes
  // per (b, h)), each its own allocation, and the silent-tile bound's workspace
  const int64_t rows = B * H * N;
  const auto ms = mask_shape(B, H, N);
  const int64_t mn = ms[0] * ms[1] * ms[2];
  const int64_t nws = (rows && B * H * N * N >= kBoundMinScores)
                          ? pnfx_flash_fwd_workspace_size(B, H, N, D) : 0;
  const auto f32 = q.options().dtype(at::kFloat);
  Tensor M = at::empty({B, H, N}, f32), Z = at::empty({B, H, N}, f32);
  Tensor Nm = at::empty(with_nmax ? at::IntArrayRef{B, H, N} : at::IntArrayRef{0},
                        q.options().dtype(at::kInt));
  Tensor mask = at::empty({ms[0], ms[1], ms[2]}, q.options().dtype(at::kByte));
  if (rows == 0) return {o, o_lo, M, Z, Nm, mask};  // empty input: empty outputs
  Tensor ws;
  if (nws) ws = at::empty({nws}, q.options().dtype(at::kByte));
  const c10::DeviceGuard guard(q.device());
  const Tensor t32 = tau32(tau, q);
  check_rc(pnfx_flash_fwd(q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(),
                          k.stride(0), k.stride(1), k.stride(2), v.data_ptr(), v.stride(0),
                          v.stride(1), v.stride(2), o.data_ptr(), o.stride(0), o.stride(1),
                          o.stride(2), bf ? o_lo.data_ptr() : nullptr, M.data_ptr<float>(),
                          Z.data_ptr<float>(), with_nmax ? Nm.data_ptr<int32_t>() : nullptr,
                          mn ? mask.data_ptr<uint8_t>() : nullptr,
                          nws ? ws.data_ptr() : nullptr, nws, B, H, N, D,
                          t32.data_ptr<float>(), (float)scale, (float)gamma, has_gamma, causal,
                          code, stream_of(q)),
           "pnfx_flash_fwd");
  return {o, o_lo, M, Z, Nm, mask};
}

// A [B,H,N,D] gradient laid out in its input's dimension order: for an input whose head
// stride is below its row stride (the heads of one [B,N,H*D] row, as the modules split a qkv
// projection) a [B,H,N,D] view of [B,N,H,D] memory, so that autograd's merge of the heads back
// into rows is a view and not a copy; [B,H,N,D] rows otherwise.  The fake kernel (ops.py)
// follows the same rule.
Tensor grad_like(const Tensor& t) {
  const int64_t B = t.size(0), H = t.size(1), N = t.size(2), D = t.size(3);
  if (H > 1 && N > 1 && t.stride(1) < t.stride(2))
    return at::empty({B, N, H, D}, t.options()).permute({0, 2, 1, 3});
  return at::empty({B, H, N, D}, t.options());
}

std::tuple<Tensor, Tensor, Tensor, Tensor> flash_bwd_cuda(
    const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, const Tensor& tau,
    const Tensor& o_in, const Tensor& o_lo, const Tensor& do_in, const Tensor& M, const Tensor& Z,
    const Tensor& mask, double scale, double gamma, bool has_gamma, bool causal) {
  check_qkv(q_in, k_in, v_in);
  TORCH_CHECK_VALUE(o_in.sizes() == q_in.sizes() && do_in.sizes() == q_in.sizes(),
                    "flash_bwd: o ", o_in.sizes(), " / dO ", do_in.sizes(), " must match q ",
                    q_in.sizes());
  const int code = dtype_code(q_in, "flash");
  const bool bf = code == PNFX_BF16;
  TORCH_CHECK_VALUE(q_in.dim() == 4, "q must be [B,H,N,D], got ", q_in.sizes());
  if (!kernel_head_dim(q_in.size(3))) {
    const int64_t D = q_in.size(3);
    check_head_dim(D);
    const int64_t Dp = padded_head_dim(D);
    auto [dq, dk, dv, dt] = flash_bwd_cuda(
        pad_d(q_in, Dp), pad_d(k_in, Dp), pad_d(v_in, Dp), tau, pad_d(o_in, Dp),
        o_lo.numel() == o_in.numel() ? pad_d(o_lo, Dp) : o_lo, pad_d(do_in, Dp), M, Z, mask,
        scale, gamma, has_gamma, causal);
    return {dq.narrow(3, 0, D).contiguous(), dk.narrow(3, 0, D).contiguous(),
            dv.narrow(3, 0, D).contiguous(), dt};
  }
  const Tensor q = bhnd(q_in, "q", bf), k = bhnd(k_in, "k", bf), v = bhnd(v_in, "v", bf);
  const Tensor o = bhnd(o_in, "o", bf);
  // the residual is used only with exactly O's layout (the C ABI takes one set of strides)
  const bool use_lo = bf && o_lo.numel() == o.numel() && o_lo.strides() == o.strides();
  const Tensor dout = bhnd(do_in.scalar_type() == q.scalar_type() ? do_in : do_in.to(q.scalar_type()),
                           "dO", bf);
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  check_saved(M, "flash_bwd", "M", B * H * N, at::kFloat, q);
  // Each gradient in its input's dimension order (see grad_like).
  check_saved(Z, "flash_bwd", "Z", B * H * N, at::kFloat, q);
  if (mask.numel()) {  // the forward's tile mask, or none (every causal tile recomputed)
    const auto ms = mask_shape(B, H, N);
    check_saved(mask, "flash_bwd", "mask", ms[0] * ms[1] * ms[2], at::kByte, q);
  }
  // dQ, dK, dV and dtau, each its own allocation (returned to autograd as the inputs' grads)
  Tensor dq = grad_like(q_in), dk = grad_like(k_in), dv = grad_like(v_in);
  Tensor dtau = at::empty({1}, q.options().dtype(at::kFloat));
  if (B * H * N == 0) return {dq, dk, dv, dtau.zero_()};  // -(sum over no scores) = 0
  const c10::DeviceGuard guard(q.device());
  const int64_t wsb = pnfx_flash_bwd_workspace_size(B, H, N, D);
  Tensor ws = at::empty({wsb}, q.options().dtype(at::kByte));
  const Tensor t32 = tau32(tau, q);
  check_rc(pnfx_flash_bwd(
               q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0),
               k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
               o.data_ptr(), o.stride(0), o.stride(1), o.stride(2),
               use_lo ? o_lo.data_ptr() : nullptr, dout.data_ptr(), dout.stride(0),
               dout.stride(1), dout.stride(2), M.data_ptr<float>(), Z.data_ptr<float>(),
               static_cast<const uint8_t*>(ptr_or_null(mask)), dq.data_ptr(), dq.stride(0),
               dq.stride(1), dq.stride(2), dk.data_ptr(), dk.stride(0), dk.stride(1),
               dk.stride(2), dv.data_ptr(), dv.stride(0), dv.stride(1), dv.stride(2),
               dtau.data_ptr<float>(), ws.data_ptr(), wsb, B, H, N, D, t32.data_ptr<float>(),
               (float)scale, (float)gamma, has_gamma, causal, code, stream_of(q)),
           "pnfx_flash_bwd");
  return {dq, dk, dv, dtau};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> flash_fwd_fir_cuda(
    const Tensor& q_in, const Tensor& kraw_in, const Tensor& v_in, const Tensor& tau,
    const Tensor& taps, double scale, double gamma, bool has_gamma, bool causal, bool o_bnhd) {
  check_qkv(q_in, kraw_in, v_in);
  const int code = dtype_code(q_in, "flash_fwd_fir");
  const Tensor q = bhnd(q_in, "q", true), kr = bhnd(kraw_in, "k_raw", true),
               v = bhnd(v_in, "v", true);
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const Tensor taps2 = taps.reshape({-1, taps.size(-1)}).to(q.device(), at::kFloat).contiguous();
  auto [o, o_lo] = new_o_pair(q, o_bnhd, true);
  const auto f32 = q.options().dtype(at::kFloat);
  Tensor M = at::empty({B, H, N}, f32), Z = at::empty({B, H, N}, f32);
  const auto ms = mask_shape(B, H, N);
  Tensor mask = at::empty({ms[0], ms[1], ms[2]}, q.options().dtype(at::kByte));
  if (B * H * N == 0) return {o, o_lo, M, Z, mask};
  const c10::DeviceGuard guard(q.device());
  const Tensor t32 = tau32(tau, q);
  check_rc(pnfx_flash_fwd_fir(q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), kr.data_ptr(),
                              kr.stride(0), kr.stride(1), kr.stride(2), v.data_ptr(), v.stride(0),
                              v.stride(1), v.stride(2), o.data_ptr(), o.stride(0), o.stride(1),
                              o.stride(2), o_lo.data_ptr(), M.data_ptr<float>(),
                              Z.data_ptr<float>(),
                              mask.numel() ? mask.data_ptr<uint8_t>() : nullptr, B, H, N, D,
                              t32.data_ptr<float>(), (float)scale, (float)gamma, has_gamma,
                              causal, taps2.data_ptr<float>(), taps2.size(0), (int)taps2.size(1),
                              code, stream_of(q)),
           "pnfx_flash_fwd_fir");
  return {o, o_lo, M, Z, mask};
}

// ---------------------------------------------------------------------------- autograd
// Each forward runs the op below autograd and saves what its backward kernel reads; only the
// differentiable outputs (the FIR output, W, O) carry gradients, and none is materialised for
// the statistics.

c10::OperatorHandle op(const char* name) {
  return c10::Dispatcher::singleton().findSchemaOrThrow(name, "");
}

// True when autograd has something to record: grad mode on and an input that requires a
// gradient (or carries a forward-mode tangent, which the Function then refuses as torch
// does for any custom Function without a jvp).  Otherwise the op runs straight below
// autograd, with no graph node built: the host time of an inference call.
bool records(std::initializer_list<const Tensor*> ts) {
  for (const Tensor* t : ts) {
    if (t->defined() && t->_fw_grad(/*level=*/0).defined()) return true;
  }
  if (!at::GradMode::is_enabled()) return false;
  for (const Tensor* t : ts) {
    if (t->defined() && t->requires_grad()) return true;
  }
  return false;
}

const auto& fir_fwd_op() {
  static auto h = op("pnfx::fir_fwd").typed<Tensor(const Tensor&, const Tensor&)>();
  return h;
}

class FirFn : public torch::autograd::Function<FirFn> {
 public:
  static Tensor forward(AutogradContext* ctx, const Tensor& x, const Tensor& taps) {
    at::AutoDispatchBelowADInplaceOrView guard;
    ctx->save_for_backward({taps});
    return fir_fwd_op().call(x, taps);
  }
  static variable_list backward(AutogradContext* ctx, variable_list gy) {
    static auto bwd = op("pnfx::fir_bwd").typed<Tensor(const Tensor&, const Tensor&)>();
    if (!gy[0].defined()) return {Tensor(), Tensor()};
    return {bwd.call(gy[0], ctx->get_saved_variables()[0]), Tensor()};
  }
};

Tensor fir_fwd_autograd(const Tensor& x, const Tensor& taps) {
  if (!records({&x, &taps})) {
    at::AutoDispatchBelowADInplaceOrView guard;
    return fir_fwd_op().call(x, taps);
  }
  return FirFn::apply(x, taps);
}

const auto& rows_fwd_op() {
  static auto h = op("pnfx::pn_rows_fwd")
                      .typed<std::tuple<Tensor, Tensor, Tensor, Tensor>(
                          const Tensor&, const Tensor&, double, double, double, bool, bool)>();
  return h;
}

class RowsFn : public torch::autograd::Function<RowsFn> {
 public:
  static variable_list forward(AutogradContext* ctx, const Tensor& raw, const Tensor& tau,
                               double scale, double p, double gamma, bool has_gamma, bool causal) {
    at::AutoDispatchBelowADInplaceOrView guard;
    auto [w, M, Z, Nm] = rows_fwd_op().call(raw, tau, scale, p, gamma, has_gamma, causal);
    ctx->mark_non_differentiable({M, Z, Nm});
    ctx->set_materialize_grads(false);
    ctx->save_for_backward({raw, tau, M, Z, Nm});
    ctx->saved_data["scale"] = scale;
    ctx->saved_data["p"] = p;
    ctx->saved_data["gamma"] = gamma;
    ctx->saved_data["has_gamma"] = has_gamma;
    ctx->saved_data["causal"] = causal;
    return {w, M, Z, Nm};
  }
  static variable_list backward(AutogradContext* ctx, variable_list g) {
    static auto bwd = op("pnfx::pn_rows_bwd")
                          .typed<std::tuple<Tensor, Tensor>(
                              const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                              const Tensor&, const Tensor&, double, double, double, bool, bool)>();
    variable_list none(7);
    if (!g[0].defined()) return none;  // W did not reach the loss
    const auto s = ctx->get_saved_variables();
    auto [d, dt] = bwd.call(g[0], s[0], s[1], s[2], s[3], s[4],
                            ctx->saved_data["scale"].toDouble(), ctx->saved_data["p"].toDouble(),
                            ctx->saved_data["gamma"].toDouble(),
                            ctx->saved_data["has_gamma"].toBool(),
                            ctx->saved_data["causal"].toBool());
    // fp64 sum of the row partials, as src/triton_pnfirtau.py:784
    none[0] = d;
    none[1] = dt.sum(at::kDouble).to(s[1].device(), s[1].scalar_type()).view_as(s[1]);
    return none;
  }
};

std::tuple<Tensor, Tensor, Tensor, Tensor> pn_rows_fwd_autograd(const Tensor& raw,
                                                                const Tensor& tau, double scale,
                                                                double p, double gamma,
                                                                bool has_gamma, bool causal) {
  if (!records({&raw, &tau})) {
    at::AutoDispatchBelowADInplaceOrView guard;
    return rows_fwd_op().call(raw, tau, scale, p, gamma, has_gamma, causal);
  }
  auto r = RowsFn::apply(raw, tau, scale, p, gamma, has_gamma, causal);
  return {r[0], r[1], r[2], r[3]};
}

const auto& flash_fwd_op() {
  static auto h = op("pnfx::flash_fwd")
                      .typed<std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>(
                          const Tensor&, const Tensor&, const Tensor&, const Tensor&, double,
                          double, bool, bool, bool, bool)>();
  return h;
}

class FlashFn : public torch::autograd::Function<FlashFn> {
 public:
  static variable_list forward(AutogradContext* ctx, const Tensor& q, const Tensor& k,
                               const Tensor& v, const Tensor& tau, double scale, double gamma,
                               bool has_gamma, bool causal, bool o_bnhd, bool with_nmax) {
    at::AutoDispatchBelowADInplaceOrView guard;
    auto [o, o_lo, M, Z, Nm, mask] = flash_fwd_op().call(q, k, v, tau, scale, gamma, has_gamma,
                                                         causal, o_bnhd, with_nmax);
    ctx->mark_non_differentiable({o_lo, M, Z, Nm, mask});
    ctx->set_materialize_grads(false);
    ctx->save_for_backward({q, k, v, tau, o, o_lo, M, Z, mask});
    ctx->saved_data["scale"] = scale;
    ctx->saved_data["gamma"] = gamma;
    ctx->saved_data["has_gamma"] = has_gamma;
    ctx->saved_data["causal"] = causal;
    return {o, o_lo, M, Z, Nm, mask};
  }
  static variable_list backward(AutogradContext* ctx, variable_list g) {
    static auto bwd = op("pnfx::flash_bwd")
                          .typed<std::tuple<Tensor, Tensor, Tensor, Tensor>(
                              const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                              const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                              const Tensor&, const Tensor&, double, double, bool, bool)>();
    variable_list grads(10);
    if (!g[0].defined()) return grads;  // O did not reach the loss
    const auto s = ctx->get_saved_variables();
    auto [dq, dk, dv, dt] =
        bwd.call(s[0], s[1], s[2], s[3], s[4], s[5], g[0], s[6], s[7], s[8],
                 ctx->saved_data["scale"].toDouble(), ctx->saved_data["gamma"].toDouble(),
                 ctx->saved_data["has_gamma"].toBool(), ctx->saved_data["causal"].toBool());
    grads[0] = dq;
    grads[1] = dk;
    grads[2] = dv;
    grads[3] = dt.to(s[3].device(), s[3].scalar_type()).view_as(s[3]);
    return grads;
  }
};

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> flash_fwd_autograd(
    const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& tau, double scale,
    double gamma, bool has_gamma, bool causal, bool o_bnhd, bool with_nmax) {
  if (!records({&q, &k, &v, &tau})) {
    at::AutoDispatchBelowADInplaceOrView guard;
    return flash_fwd_op().call(q, k, v, tau, scale, gamma, has_gamma, causal, o_bnhd, with_nmax);
  }
  auto r = FlashFn::apply(q, k, v, tau, scale, gamma, has_gamma, causal, o_bnhd, with_nmax);
  return {r[0], r[1], r[2], r[3], r[4], r[5]};
}

}  // namespace

TORCH_LIBRARY(pnfx, m) {
  m.def("fir_fwd(Tensor x, Tensor taps) -> Tensor");
  m.def("fir_bwd(Tensor gy, Tensor taps) -> Tensor");
  m.def("pn_rows_fwd(Tensor raw, Tensor tau, float scale, float p, float gamma, bool has_gamma, "
        "bool causal) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("pn_rows_bwd(Tensor dw, Tensor raw, Tensor tau, Tensor M, Tensor Z, Tensor Nmax, "
        "float scale, float p, float gamma, bool has_gamma, bool causal) -> (Tensor, Tensor)");
  m.def("flash_fwd(Tensor q, Tensor k, Tensor v, Tensor tau, float scale, float gamma, "
        "bool has_gamma, bool causal, bool o_bnhd, bool with_nmax) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("flash_bwd(Tensor q, Tensor k, Tensor v, Tensor tau, Tensor o, Tensor o_lo, Tensor do, "
        "Tensor M, Tensor Z, Tensor mask, float scale, float gamma, bool has_gamma, bool causal) "
        "-> (Tensor, Tensor, Tensor, Tensor)");
  m.def("flash_fwd_fir(Tensor q, Tensor k_raw, Tensor v, Tensor tau, Tensor taps, float scale, "
        "float gamma, bool has_gamma, bool causal, bool o_bnhd=False) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(pnfx, CUDA, m) {
  m.impl("fir_fwd", fir_fwd_cuda);
  m.impl("fir_bwd", fir_bwd_cuda);
  m.impl("pn_rows_fwd", pn_rows_fwd_cuda);
  m.impl("pn_rows_bwd", pn_rows_bwd_cuda);
  m.impl("flash_fwd", flash_fwd_cuda);
  m.impl("flash_bwd", flash_bwd_cuda);
  m.impl("flash_fwd_fir", flash_fwd_fir_cuda);
}

TORCH_LIBRARY_IMPL(pnfx, Autograd, m) {
  m.impl("fir_fwd", fir_fwd_autograd);
  m.impl("pn_rows_fwd", pn_rows_fwd_autograd);
  m.impl("flash_fwd", flash_fwd_autograd);
}
