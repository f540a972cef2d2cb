"""torch.library custom ops over libpnfx.so (namespace ``pnfx``), with autograd.

Each op allocates its outputs with the caching allocator on the input's device,
enqueues the HIP kernels on the current stream through the C ABI, and never
blocks the host.  Ops are registered for the CUDA (= HIP) device only: calling
them on CPU tensors raises, and a missing library raises ``PnfxError``.

Op                     reference counterpart (src/triton_pnfirtau.py)
pnfx::fir_fwd / _bwd   _TritonCausalFir7Fn              :629-682
pnfx::pn_rows_fwd/_bwd _TritonPnFirTauScoresFn          :694-785
pnfx::flash_fwd/_bwd   _FlashPnFirTauFn                 :814-968
"""
from __future__ import annotations

import functools
import math

import torch
from torch import Tensor

from . import _lib

_DT = {torch.float32: _lib.PNFX_F32, torch.bfloat16: _lib.PNFX_BF16}


def _code(t: Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: dtype {t.dtype} is not supported (float32, bfloat16)") from None


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _tau32(tau: Tensor) -> Tensor:
    t = tau.detach().reshape(1)
    return t if t.dtype == torch.float32 else t.to(torch.float32)


def _as_bhnc(x: Tensor) -> tuple[Tensor, int, int, int, int]:
    """View x ([B,N,C] or [B,H,N,C]) as 4-D with unit channel stride; returns (x4, B, H, N, C)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    x4 = x.unsqueeze(1) if x.dim() == 3 else x
    if x4.dim() != 4:
        raise ValueError(f"FIR input must be [B,N,C] or [B,H,N,C], got {tuple(x.shape)}")
    B, H, N, C = x4.shape
    return x4, B, H, N, C


# ---------------------------------------------------------------------------- FIR
def _fir_call(x: Tensor, taps: Tensor, adjoint: bool) -> Tensor:
    x4, B, H, N, C = _as_bhnc(x)
    taps2 = taps.reshape(-1, taps.shape[-1])
    if taps2.dtype != torch.float32 or not taps2.is_contiguous() or taps2.device != x.device:
        taps2 = taps2.to(device=x.device, dtype=torch.float32).contiguous()
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if y.numel() == 0:  # empty input: nothing to filter (the reference launches an empty grid)
        return y
    fn = _lib.lib().pnfx_fir_bwd if adjoint else _lib.lib().pnfx_fir_fwd
    rc = fn(x4.data_ptr(), x4.stride(0), x4.stride(1), x4.stride(2), y.data_ptr(), B, H, N, C,
            taps2.data_ptr(), taps2.shape[0], taps2.shape[1], _code(x, "fir"), _stream(x))
    _lib.check(rc, "pnfx_fir_bwd" if adjoint else "pnfx_fir_fwd")
    return y


@torch.library.custom_op("pnfx::fir_fwd", mutates_args=(), device_types="cuda")
def fir_fwd(x: Tensor, taps: Tensor) -> Tensor:
    """Causal FIR along N of x [B,N,C] or [B,H,N,C]; taps fp32 [K] or [H,K] (oldest lag first)."""
    return _fir_call(x, taps, False)


@torch.library.custom_op("pnfx::fir_bwd", mutates_args=(), device_types="cuda")
def fir_bwd(gy: Tensor, taps: Tensor) -> Tensor:
    """Adjoint of fir_fwd (anti-causal correlation with the same taps)."""
    return _fir_call(gy, taps, True)


@fir_fwd.register_fake
def _(x, taps):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


@fir_bwd.register_fake
def _(gy, taps):
    return torch.empty(gy.shape, dtype=gy.dtype, device=gy.device)


def _fir_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])


def _fir_backward(ctx, gy):
    (taps,) = ctx.saved_tensors
    return fir_bwd(gy, taps), None


torch.library.register_autograd("pnfx::fir_fwd", _fir_backward, setup_context=_fir_setup)


# ---------------------------------------------------------------------------- row scores
@torch.library.custom_op("pnfx::pn_rows_fwd", mutates_args=(), device_types="cuda")
def pn_rows_fwd(raw: Tensor, tau: Tensor, scale: float, p: float, gamma: float, has_gamma: bool,
                causal: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Row-fused score -> weight over raw [..., N, N]; returns (W, M, Z, Nmax), stats per row."""
    N = raw.shape[-1]
    R = math.prod(raw.shape[:-1])
    r2 = raw.contiguous().view(R, N)
    w = torch.empty_like(r2)
    M = torch.empty(R, device=raw.device, dtype=torch.float32)
    Z = torch.empty(R, device=raw.device, dtype=torch.float32)
    Nm = torch.empty(R, device=raw.device, dtype=torch.int32)
    if r2.numel() == 0:  # no rows, or rows of length 0 (peak 0, mass 0 + 1e-12, no ties)
        M.zero_()
        Z.fill_(1e-12)
        Nm.zero_()
        return w.view(raw.shape), M, Z, Nm
    t32 = _tau32(tau)
    rc = _lib.lib().pnfx_pn_rows_fwd(r2.data_ptr(), N, w.data_ptr(), N, M.data_ptr(), Z.data_ptr(),
                                     Nm.data_ptr(), R, N, t32.data_ptr(), scale, p, gamma,
                                     int(has_gamma), int(causal), _code(raw, "pn_rows"),
                                     _stream(raw))
    _lib.check(rc, "pnfx_pn_rows_fwd")
    return w.view(raw.shape), M, Z, Nm


@pn_rows_fwd.register_fake
def _(raw, tau, scale, p, gamma, has_gamma, causal):
    R = math.prod(raw.shape[:-1])
    f = lambda dt: torch.empty(R, device=raw.device, dtype=dt)  # noqa: E731
    # contiguous, as the real kernel returns it whatever raw's strides
    w = torch.empty(raw.shape, dtype=raw.dtype, device=raw.device)
    return w, f(torch.float32), f(torch.float32), f(torch.int32)


@torch.library.custom_op("pnfx::pn_rows_bwd", mutates_args=(), device_types="cuda")
def pn_rows_bwd(dw: Tensor, raw: Tensor, tau: Tensor, M: Tensor, Z: Tensor, Nmax: Tensor,
                scale: float, p: float, gamma: float, has_gamma: bool,
                causal: bool) -> tuple[Tensor, Tensor]:
    """Backward of pn_rows_fwd: (d_raw, dtau_rows) with dtau_rows[r] = -sum_j du[r, j]."""
    N = raw.shape[-1]
    R = math.prod(raw.shape[:-1])
    r2 = raw.contiguous().view(R, N)
    g2 = dw.to(raw.dtype).contiguous().view(R, N)
    d = torch.empty_like(r2)
    dt = torch.empty(R, device=raw.device, dtype=torch.float32)
    if r2.numel() == 0:
        return d.view(raw.shape), dt.zero_()
    t32 = _tau32(tau)
    rc = _lib.lib().pnfx_pn_rows_bwd(g2.data_ptr(), N, r2.data_ptr(), N, M.data_ptr(), Z.data_ptr(),
                                     Nmax.data_ptr(), d.data_ptr(), N, dt.data_ptr(), R, N,
                                     t32.data_ptr(), scale, p, gamma, int(has_gamma), int(causal),
                                     _code(raw, "pn_rows"), _stream(raw))
    _lib.check(rc, "pnfx_pn_rows_bwd")
    return d.view(raw.shape), dt


@pn_rows_bwd.register_fake
def _(dw, raw, tau, M, Z, Nmax, scale, p, gamma, has_gamma, causal):
    R = math.prod(raw.shape[:-1])
    return (torch.empty(raw.shape, dtype=raw.dtype, device=raw.device),
            torch.empty(R, device=raw.device, dtype=torch.float32))


def _rows_setup(ctx, inputs, output):
    raw, tau, scale, p, gamma, has_gamma, causal = inputs
    _, M, Z, Nm = output
    ctx.mark_non_differentiable(M, Z, Nm)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(raw, tau, M, Z, Nm)
    ctx.args = (scale, p, gamma, has_gamma, causal)


def _rows_backward(ctx, dw, dM, dZ, dN):
    if dw is None:  # W did not reach the loss
        return (None,) * 7
    raw, tau, M, Z, Nm = ctx.saved_tensors
    d, dt = pn_rows_bwd(dw, raw, tau, M, Z, Nm, *ctx.args)
    # fp64 sum of the row partials, as src/triton_pnfirtau.py:784
    dtau = dt.sum(dtype=torch.float64).to(tau.dtype).view_as(tau)
    return d, dtau, None, None, None, None, None


torch.library.register_autograd("pnfx::pn_rows_fwd", _rows_backward, setup_context=_rows_setup)


# ---------------------------------------------------------------------------- flash
def _bhnd(t: Tensor, name: str, bf16: bool) -> Tensor:
    """Return t with unit inner stride and (bf16) 16-byte-aligned, 8-element-multiple strides."""
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B,H,N,D], got {tuple(t.shape)}")
    ok = t.stride(-1) == 1
    if ok and bf16:
        ok = t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:3])
    return t if ok else t.contiguous()


def _check_qkv(q: Tensor, k: Tensor, v: Tensor) -> None:
    """q, k and v must agree in shape, dtype and device: the kernels read all three with
    q's element size.  (The Python entry points cast k and v to q's dtype first.)"""
    for name, t in (("k", k), ("v", v)):
        if t.shape != q.shape:
            raise ValueError(f"flash: {name} has shape {tuple(t.shape)}, q has {tuple(q.shape)}")
        if t.dtype != q.dtype:
            raise TypeError(f"flash: {name} is {t.dtype}, q is {q.dtype}")
        if t.device != q.device:
            raise ValueError(f"flash: {name} is on {t.device}, q on {q.device}")


# Above this sequence length the forward does not record the silence map (its
# B*H*ceil(N/32)*ceil(N/64) bytes grow as N^2/2048 per (b, h)); the backward then
# recomputes every causal tile.
MASK_MAX_N = 65536


def _mask_shape(B: int, H: int, N: int) -> tuple[int, int, int]:
    if N > MASK_MAX_N:
        return (0, 0, 0)
    return (B * H, (N + 31) // 32, (N + 63) // 64)


def _ptr4(t: Tensor) -> tuple[int, int, int, int]:
    """(data pointer, batch, head, row strides) of a [B,H,N,D] operand for the C ABI."""
    return t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)


def _new_o(q: Tensor, o_bnhd: bool) -> Tensor:
    B, H, N, D = q.shape
    if o_bnhd:
        return torch.empty((B, N, H, D), device=q.device, dtype=q.dtype).permute(0, 2, 1, 3)
    return torch.empty((B, H, N, D), device=q.device, dtype=q.dtype)


@functools.lru_cache(maxsize=None)
def _fwd_workspace_bytes(B: int, H: int, N: int, D: int) -> int:
    return int(_lib.lib().pnfx_flash_fwd_workspace_size(B, H, N, D))


@torch.library.custom_op("pnfx::flash_fwd", mutates_args=(), device_types="cuda")
def flash_fwd(q: Tensor, k: Tensor, v: Tensor, tau: Tensor, scale: float, gamma: float,
              has_gamma: bool, causal: bool, o_bnhd: bool,
              with_nmax: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Flash forward on [B,H,N,D]; returns (O, O_lo, M, Z, Nmax, tile_mask).

    O has shape [B,H,N,D]; with o_bnhd it is backed by a [B,N,H,D] buffer so that
    the caller's transpose back to [B,N,H*D] is free.  O_lo (bf16 only; empty for
    fp32) is O's bf16 rounding residual, saved for an accurate backward.
    Nmax (peak-tie counts) is formed only with_nmax, else returned empty: the
    backward does not need it.  tile_mask is uint8 [B*H, ceil(N/32), ceil(N/64)]
    (32-query x 64-key sub-tile activity): N^2/2048 bytes per (b, h), the one part of
    the saved state that is not O(N); past MASK_MAX_N it is not formed (shape (0, 0, 0))
    and the backward recomputes every causal tile.  k and v must have q's shape, dtype and
    device.
    """
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    code = _code(q, "flash")
    bf = code == _lib.PNFX_BF16
    q, k, v = _bhnd(q, "q", bf), _bhnd(k, "k", bf), _bhnd(v, "v", bf)
    o = _new_o(q, o_bnhd)
    o_lo = _new_o(q, o_bnhd) if bf else q.new_empty(0)
    M = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    Z = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    Nm = torch.empty((B, H, N) if with_nmax else (0,), device=q.device, dtype=torch.int32)
    # one allocation: the tile mask (N^2/2048 bytes per (b, h); none past MASK_MAX_N), then
    # (256-byte aligned) the workspace of the silent-tile bound (per-tile key norms, a few KiB)
    mshape = _mask_shape(B, H, N)
    mn = mshape[0] * mshape[1] * mshape[2]
    mbytes = (mn + 255) // 256 * 256
    nws = _fwd_workspace_bytes(B, H, N, D)
    buf = torch.empty(mbytes + nws, device=q.device, dtype=torch.uint8)
    mask = buf[:mn].view(mshape)
    ws = buf[mbytes:]
    if B * H * N == 0:  # empty input: empty outputs, as the reference's empty launch grid gives
        return o, o_lo, M, Z, Nm, mask
    t32 = _tau32(tau)
    rc = _lib.lib().pnfx_flash_fwd(
        *_ptr4(q), *_ptr4(k), *_ptr4(v), *_ptr4(o), o_lo.data_ptr() if bf else None,
        M.data_ptr(), Z.data_ptr(), Nm.data_ptr() if with_nmax else None,
        mask.data_ptr() if mn else None, ws.data_ptr() if nws else None, nws, B, H, N, D,
        t32.data_ptr(), scale, gamma, int(has_gamma), int(causal), code, _stream(q))
    _lib.check(rc, "pnfx_flash_fwd")
    return o, o_lo, M, Z, Nm, mask


def flash_fwd_fused_fir(q: Tensor, k_raw: Tensor, v: Tensor, tau: Tensor, taps: Tensor,
                        scale: float, gamma: float, has_gamma: bool,
                        causal: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Flash forward with the causal FIR of the keys fused into the key-tile load
    (pnfx_flash_fwd_fir): k_raw are the keys before the FIR, taps as fir_fwd (fp32 [K] or
    [H, K], K <= 7).  Returns (O, O_lo, M, Z, tile_mask), bitwise those of fir_fwd followed by
    flash_fwd.  bf16, d = 64, inference only (no autograd, no tie counts): the filtered keys
    are not materialised, so there is nothing for a backward to read."""
    _check_qkv(q, k_raw, v)
    B, H, N, D = q.shape
    code = _code(q, "flash_fwd_fir")
    q, k_raw, v = _bhnd(q, "q", True), _bhnd(k_raw, "k_raw", True), _bhnd(v, "v", True)
    taps2 = taps.reshape(-1, taps.shape[-1]).to(device=q.device, dtype=torch.float32).contiguous()
    o = _new_o(q, False)
    o_lo = _new_o(q, False)
    M = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    Z = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    mask = torch.empty(_mask_shape(B, H, N), device=q.device, dtype=torch.uint8)
    t32 = _tau32(tau)
    rc = _lib.lib().pnfx_flash_fwd_fir(
        *_ptr4(q), *_ptr4(k_raw), *_ptr4(v), *_ptr4(o), o_lo.data_ptr(), M.data_ptr(),
        Z.data_ptr(), mask.data_ptr() if mask.numel() else None, B, H, N, D, t32.data_ptr(),
        scale, gamma, int(has_gamma), int(causal), taps2.data_ptr(), taps2.shape[0],
        taps2.shape[1], code, _stream(q))
    _lib.check(rc, "pnfx_flash_fwd_fir")
    return o, o_lo, M, Z, mask


@flash_fwd.register_fake
def _(q, k, v, tau, scale, gamma, has_gamma, causal, o_bnhd, with_nmax):
    B, H, N, D = q.shape
    o = _new_o(q, o_bnhd)
    o_lo = _new_o(q, o_bnhd) if q.dtype == torch.bfloat16 else q.new_empty(0)
    f = lambda dt: q.new_empty((B, H, N), dtype=dt)  # noqa: E731
    nm = q.new_empty((B, H, N) if with_nmax else (0,), dtype=torch.int32)
    mask = q.new_empty(_mask_shape(B, H, N), dtype=torch.uint8)
    return o, o_lo, f(torch.float32), f(torch.float32), nm, mask


@torch.library.custom_op("pnfx::flash_bwd", mutates_args=(), device_types="cuda")
def flash_bwd(q: Tensor, k: Tensor, v: Tensor, tau: Tensor, o: Tensor, o_lo: Tensor, do: Tensor,
              M: Tensor, Z: Tensor, mask: Tensor, scale: float, gamma: float,
              has_gamma: bool, causal: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Deterministic flash backward; returns (dq, dk, dv, dtau) with dtau a 1-element fp32 tensor."""
    _check_qkv(q, k, v)
    if o.shape != q.shape or do.shape != q.shape:
        raise ValueError(f"flash_bwd: o {tuple(o.shape)} / dO {tuple(do.shape)} must match q "
                         f"{tuple(q.shape)}")
    B, H, N, D = q.shape
    code = _code(q, "flash")
    bf = code == _lib.PNFX_BF16
    q, k, v = _bhnd(q, "q", bf), _bhnd(k, "k", bf), _bhnd(v, "v", bf)
    use_lo = bf and o_lo.numel() == o.numel() and o_lo.stride() == o.stride()
    o = _bhnd(o, "o", bf)
    if use_lo and o_lo.stride() != o.stride():
        use_lo = False
    do = _bhnd(do.to(q.dtype), "dO", bf)
    dq = torch.empty((B, H, N, D), device=q.device, dtype=q.dtype)
    dk = torch.empty((B, H, N, D), device=q.device, dtype=q.dtype)
    dv = torch.empty((B, H, N, D), device=q.device, dtype=q.dtype)
    dtau = torch.empty(1, device=q.device, dtype=torch.float32)
    if B * H * N == 0:  # empty input: empty gradients, dtau = -(sum over no scores) = 0
        return dq, dk, dv, dtau.zero_()
    L = _lib.lib()
    ws_bytes = L.pnfx_flash_bwd_workspace_size(B, H, N, D)
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    t32 = _tau32(tau)
    rc = L.pnfx_flash_bwd(
        *_ptr4(q), *_ptr4(k), *_ptr4(v), *_ptr4(o), o_lo.data_ptr() if use_lo else None,
        *_ptr4(do), M.data_ptr(), Z.data_ptr(), mask.data_ptr() if mask.numel() else None,
        *_ptr4(dq), *_ptr4(dk), *_ptr4(dv), dtau.data_ptr(), ws.data_ptr(), ws_bytes, B, H, N, D,
        t32.data_ptr(), scale, gamma, int(has_gamma), int(causal), code, _stream(q))
    _lib.check(rc, "pnfx_flash_bwd")
    return dq, dk, dv, dtau


@flash_bwd.register_fake
def _(q, k, v, tau, o, o_lo, do, M, Z, mask, scale, gamma, has_gamma, causal):
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            torch.empty_like(k, memory_format=torch.contiguous_format),
            torch.empty_like(v, memory_format=torch.contiguous_format),
            q.new_empty(1, dtype=torch.float32))


def _flash_setup(ctx, inputs, output):
    q, k, v, tau, scale, gamma, has_gamma, causal, o_bnhd, with_nmax = inputs
    o, o_lo, M, Z, Nm, mask = output
    # Only O carries a gradient: no zero-filled gradients are materialised for the rest.
    ctx.mark_non_differentiable(o_lo, M, Z, Nm, mask)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, k, v, tau, o, o_lo, M, Z, mask)
    ctx.args = (scale, gamma, has_gamma, causal)


def _flash_backward(ctx, do, do_lo, dM, dZ, dN, dmask):
    if do is None:  # O did not reach the loss
        return (None,) * 10
    q, k, v, tau, o, o_lo, M, Z, mask = ctx.saved_tensors
    dq, dk, dv, dt = flash_bwd(q, k, v, tau, o, o_lo, do, M, Z, mask, *ctx.args)
    return dq, dk, dv, dt.to(tau.dtype).view_as(tau), None, None, None, None, None, None


torch.library.register_autograd("pnfx::flash_fwd", _flash_backward, setup_context=_flash_setup)
