"""HIP counterparts of the reference's accelerated entry points (src/triton_pnfirtau.py).

=============================  ==========================================  ==========
this module                    reference                                   lines
=============================  ==========================================  ==========
``hip_causal_fir``             ``triton_causal_fir``                       :685-691
``hip_pn_fir_tau_scores``      ``triton_pn_fir_tau_scores``                :788-811
``flash_pn_fir_tau_attention`` ``flash_pn_fir_tau_attention``              :971-983
=============================  ==========================================  ==========

The reference names ``triton_causal_fir`` / ``triton_pn_fir_tau_scores`` are
kept as aliases so call sites can switch imports without edits.

Dispatch follows the reference's rule, with the HIP kernels covering a wider
range: GPU tensors always run the HIP kernels (FIR: any channel count and
K <= 16 taps; row scores: any row length); CPU tensors take the eager
primitives, as the reference does for non-CUDA tensors (:687, :797).  Flash
attention has no CPU path in the reference and none here.
"""
from __future__ import annotations

import math

import torch

from . import ops  # noqa: F401  (registers the pnfx:: ops)
from .pnfirtau_attention import causal_fir, power_norm_peak_gate

FIR_MAX_TAPS = 16


def hip_causal_fir(x: torch.Tensor, taps: torch.Tensor) -> torch.Tensor:
    """Causal depthwise FIR along N for x [B, N, C] (any strides), taps [K] oldest lag first.

    GPU: HIP streaming kernel, fp32 taps and fp32 fused multiply-add chain in lag
    order, one rounding to x's dtype (src/triton_pnfirtau.py:40-135).  Returns a
    contiguous [B, N, C] tensor; backward is the adjoint FIR (taps get no grad).
    """
    if not x.is_cuda:
        return causal_fir(x, taps)
    K = taps.numel()
    if K > FIR_MAX_TAPS:
        raise NotImplementedError(f"hip_causal_fir: {K} taps > {FIR_MAX_TAPS}")
    if K <= 1:
        return x  # as the eager primitive (src/pnfirtau_attention.py:69-70)
    return torch.ops.pnfx.fir_fwd(x, taps.reshape(-1))


def hip_causal_fir_heads(k: torch.Tensor, taps: torch.Tensor) -> torch.Tensor:
    """Causal FIR along N of keys in [B, H, N, d] layout with per-head taps [H, K] (or shared [K])."""
    if not k.is_cuda:
        raise RuntimeError("hip_causal_fir_heads runs on the GPU only")
    return torch.ops.pnfx.fir_fwd(k, taps)


def hip_pn_fir_tau_scores(
    raw_scores: torch.Tensor,
    score_tau: torch.Tensor,
    scale: float = 1.0,
    p: float = 10.0,
    gamma: float | None = 0.5,
    causal_mask: bool = True,
) -> torch.Tensor:
    """Row-fused s = raw*scale - tau -> relu -> ^p -> normalise -> peak gate, raw [..., N, N].

    GPU: one HIP kernel forward and one backward (peak mode; src/triton_pnfirtau.py:141-303).
    CPU: the eager composition of src/triton_pnfirtau.py:802-811.
    """
    if not raw_scores.is_cuda:
        scores = raw_scores * scale - score_tau
        if causal_mask:
            n = scores.shape[-1]
            upper = torch.ones(n, n, device=scores.device, dtype=torch.bool).triu_(1)
            scores = scores.masked_fill(upper, -1e4)
        return power_norm_peak_gate(scores, p=p, gamma=gamma, silence_mode="peak")
    N = raw_scores.shape[-1]
    assert raw_scores.shape[-2] == N, "Expected [..., N, N] scores tensor"
    has_gamma = gamma is not None and gamma > 0.0
    w, _, _, _ = torch.ops.pnfx.pn_rows_fwd(raw_scores, score_tau, float(scale), float(p),
                                            float(gamma) if has_gamma else 0.0, has_gamma,
                                            bool(causal_mask))
    return w


def _flash_attention(q, k, v, score_tau, scale, gamma, causal_mask, o_bnhd=False):
    if not q.is_cuda:
        raise RuntimeError("flash_pn_fir_tau_attention runs on the GPU only (as in the reference)")
    has_gamma = gamma is not None and gamma > 0.0
    o = torch.ops.pnfx.flash_fwd(q, k, v, score_tau, float(scale),
                                 float(gamma) if has_gamma else 0.0, has_gamma,
                                 bool(causal_mask), bool(o_bnhd), False)[0]
    return o


def flash_pn_fir_tau_attention(
    q: torch.Tensor,
    k_tilde: torch.Tensor,
    v: torch.Tensor,
    score_tau: torch.Tensor,
    scale: float | None = None,
    gamma: float | None = 0.5,
    causal_mask: bool = True,
) -> torch.Tensor:
    """O(N)-memory flash pn_fir_tau attention (p = 10, peak gate) on [B, H, N, d] inputs.

    Returns O [B, H, N, d] (contiguous).  scale defaults to 1/sqrt(d).
    Backward is deterministic (no atomics) and returns grads for q, k_tilde, v and
    score_tau (src/triton_pnfirtau.py:814-983).
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return _flash_attention(q, k_tilde, v, score_tau, scale, gamma, causal_mask)


def flash_pn_fir_tau_attention_with_stats(q, k_tilde, v, score_tau, scale=None, gamma=0.5,
                                          causal_mask=True):
    """Forward only: (O, M, Z, Nmax, tile_mask) -- the saved statistics and the silence map."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    has_gamma = gamma is not None and gamma > 0.0
    o, _, M, Z, Nm, mask = torch.ops.pnfx.flash_fwd(q, k_tilde, v, score_tau, float(scale),
                                                   float(gamma) if has_gamma else 0.0, has_gamma,
                                                   bool(causal_mask), False, True)
    return o, M, Z, Nm, mask


def tile_mask_64(mask32: torch.Tensor) -> torch.Tensor:
    """64x64 view of the flash tile mask: OR of adjacent 32-row groups."""
    BH, n32, n64 = mask32.shape
    if n32 % 2:
        mask32 = torch.cat([mask32, mask32.new_zeros(BH, 1, n64)], dim=1)
    return mask32.view(BH, -1, 2, n64).amax(dim=2)


# reference names (src/triton_pnfirtau.py:685, :788)
triton_causal_fir = hip_causal_fir
triton_pn_fir_tau_scores = hip_pn_fir_tau_scores
