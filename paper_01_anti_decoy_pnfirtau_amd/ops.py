"""The pnfx ops (namespace ``pnfx``) as torch.library operators, with autograd.

The operators, their HIP (CUDA-key) kernels and their autograd are registered in C++
(``csrc/torch_ops.cpp``, built into ``_pnfx_torch.so`` beside ``libpnfx.so``): each op
allocates its outputs with the caching allocator on the input's device, enqueues the HIP
kernels on the current stream through the C ABI, and never blocks the host.  Ops are
registered for the CUDA (= HIP) device only: calling them on CPU tensors raises, and a
missing library raises ``PnfxError``.  This module loads that library and adds the fake
(meta) kernels that torch.compile and FakeTensor tracing use.

Op                     reference counterpart (src/triton_pnfirtau.py)
pnfx::fir_fwd / _bwd   _TritonCausalFir7Fn              :629-682
pnfx::pn_rows_fwd/_bwd _TritonPnFirTauScoresFn          :694-785
pnfx::flash_fwd/_bwd   _FlashPnFirTauFn                 :814-968
pnfx::flash_fwd_fir    (none: the key FIR fused into the forward's key-tile load)
"""
from __future__ import annotations

import math
import os

import torch
from torch import Tensor

from . import _lib

TORCH_OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_pnfx_torch.so")


def _load() -> None:
    if not os.path.exists(TORCH_OPS_PATH):
        raise _lib.PnfxError(f"{TORCH_OPS_PATH} is not built; run "
                             "`python -m paper_01_anti_decoy_pnfirtau_amd.build`")
    _lib.lib()  # the C ABI library it links (and its ABI version check)
    torch.ops.load_library(TORCH_OPS_PATH)


_load()

fir_fwd = torch.ops.pnfx.fir_fwd
fir_bwd = torch.ops.pnfx.fir_bwd
pn_rows_fwd = torch.ops.pnfx.pn_rows_fwd
pn_rows_bwd = torch.ops.pnfx.pn_rows_bwd
flash_fwd = torch.ops.pnfx.flash_fwd
flash_bwd = torch.ops.pnfx.flash_bwd


def _check_qkv(q: Tensor, k: Tensor, v: Tensor) -> None:
    """q, k and v must agree in shape, dtype and device: the kernels read all three with
    q's element size.  (The C++ ops check the same; the Python entry points cast k and v to
    q's dtype first.)"""
    for name, t in (("k", k), ("v", v)):
        if t.shape != q.shape:
            raise ValueError(f"flash: {name} has shape {tuple(t.shape)}, q has {tuple(q.shape)}")
        if t.dtype != q.dtype:
            raise TypeError(f"flash: {name} is {t.dtype}, q is {q.dtype}")
        if t.device != q.device:
            raise ValueError(f"flash: {name} is on {t.device}, q on {q.device}")


# Above this sequence length the forward does not record the silence map (its
# B*H*ceil(N/32)*ceil(N/64) bytes grow as N^2/2048 per (b, h)); the backward then
# recomputes every causal tile.  The C++ ops use the same limit.
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


def flash_fwd_fused_fir(q: Tensor, k_raw: Tensor, v: Tensor, tau: Tensor, taps: Tensor,
                        scale: float, gamma: float, has_gamma: bool, causal: bool,
                        o_bnhd: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Flash forward with the causal FIR of the keys fused into the key-tile load
    (pnfx::flash_fwd_fir): k_raw are the keys before the FIR, taps as fir_fwd (fp32 [K] or
    [H, K], K <= 7).  Returns (O, O_lo, M, Z, tile_mask), bitwise those of fir_fwd followed by
    flash_fwd.  bf16, d in {16, 32, 64}, inference only (no autograd, no tie counts): the
    filtered keys are not materialised, so there is nothing for a backward to read."""
    return torch.ops.pnfx.flash_fwd_fir.default(q, k_raw, v, tau, taps, scale, gamma, has_gamma,
                                                causal, o_bnhd)


# ---------------------------------------------------------------------------- fake kernels
@torch.library.register_fake("pnfx::fir_fwd")
def _(x, taps):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


@torch.library.register_fake("pnfx::fir_bwd")
def _(gy, taps):
    return torch.empty(gy.shape, dtype=gy.dtype, device=gy.device)


@torch.library.register_fake("pnfx::pn_rows_fwd")
def _(raw, tau, scale, p, gamma, has_gamma, causal):
    R = math.prod(raw.shape[:-1])
    f = lambda dt: torch.empty(R, device=raw.device, dtype=dt)  # noqa: E731
    # contiguous, as the real kernel returns it whatever raw's strides
    w = torch.empty(raw.shape, dtype=raw.dtype, device=raw.device)
    return w, f(torch.float32), f(torch.float32), f(torch.int32)


@torch.library.register_fake("pnfx::pn_rows_bwd")
def _(dw, raw, tau, M, Z, Nmax, scale, p, gamma, has_gamma, causal):
    R = math.prod(raw.shape[:-1])
    return (torch.empty(raw.shape, dtype=raw.dtype, device=raw.device),
            torch.empty(R, device=raw.device, dtype=torch.float32))


@torch.library.register_fake("pnfx::flash_fwd")
def _(q, k, v, tau, scale, gamma, has_gamma, causal, o_bnhd, with_nmax):
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    o = _new_o(q, o_bnhd)
    o_lo = _new_o(q, o_bnhd) if q.dtype == torch.bfloat16 else q.new_empty(0)
    f = lambda dt: q.new_empty((B, H, N), dtype=dt)  # noqa: E731
    nm = q.new_empty((B, H, N) if with_nmax else (0,), dtype=torch.int32)
    mask = q.new_empty(_mask_shape(B, H, N), dtype=torch.uint8)
    return o, o_lo, f(torch.float32), f(torch.float32), nm, mask


def _grad_like(t: Tensor) -> Tensor:
    """The backward op's gradient layout (csrc/torch_ops.cpp, grad_like): a [B,H,N,D] view of
    [B,N,H,D] memory when the input's head stride is below its row stride, else [B,H,N,D]."""
    B, H, N, D = t.shape
    if H > 1 and N > 1 and t.stride(1) < t.stride(2):
        return t.new_empty((B, N, H, D)).permute(0, 2, 1, 3)
    return t.new_empty((B, H, N, D))


@torch.library.register_fake("pnfx::flash_bwd")
def _(q, k, v, tau, o, o_lo, do, M, Z, mask, scale, gamma, has_gamma, causal):
    if q.shape[-1] not in (16, 32, 64, 128):  # padded head sizes: contiguous slices
        return (q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape),
                q.new_empty(1, dtype=torch.float32))
    return _grad_like(q), _grad_like(k), _grad_like(v), q.new_empty(1, dtype=torch.float32)


@torch.library.register_fake("pnfx::flash_fwd_fir")
def _(q, k_raw, v, tau, taps, scale, gamma, has_gamma, causal, o_bnhd=False):
    _check_qkv(q, k_raw, v)
    B, H, N, D = q.shape
    f = lambda: q.new_empty((B, H, N), dtype=torch.float32)  # noqa: E731
    return (_new_o(q, o_bnhd), _new_o(q, o_bnhd), f(), f(),
            q.new_empty(_mask_shape(B, H, N), dtype=torch.uint8))
