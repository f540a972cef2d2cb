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

Dispatch follows the reference's rules.  The FIR runs the HIP kernel exactly
where the reference runs its Triton kernel -- a GPU tensor, K == 7 taps and at
most 1024 channels (:687) -- and the eager ``causal_fir`` everywhere else, as
the reference does: that eager path casts the taps to x's dtype (bf16-rounded
taps for bf16 input), where the kernel keeps fp32 taps.  (Other tap counts up to
16 and any channel count are available from the kernel directly, as
``torch.ops.pnfx.fir_fwd``.)  Row scores run the HIP kernel for every GPU tensor
(the reference stops at N = 4096, :797; the kernel has no such limit) and the
eager composition for CPU tensors.  Flash attention has no CPU path in the
reference and none here.
"""
from __future__ import annotations

import math

import torch

from . import ops  # noqa: F401  (registers the pnfx:: ops)
from .pnfirtau_attention import causal_fir, power_norm_peak_gate

FIR_KERNEL_TAPS = 7  # the reference's kernel path (src/triton_pnfirtau.py:687)
FIR_KERNEL_MAX_C = 1024


def hip_causal_fir(x: torch.Tensor, taps: torch.Tensor) -> torch.Tensor:
    """Causal depthwise FIR along N for x [B, N, C] (any strides), taps [K] oldest lag first.

    GPU, K == 7, C <= 1024: the HIP streaming kernel -- fp32 taps and an fp32 fused
    multiply-add chain in lag order, one rounding to x's dtype
    (src/triton_pnfirtau.py:40-135); returns a contiguous [B, N, C] tensor, backward is
    the adjoint FIR (taps get no grad).  Otherwise the eager ``causal_fir``
    (src/triton_pnfirtau.py:685-691): CPU tensors, other tap counts, wider rows.
    """
    if x.is_cuda and taps.numel() == FIR_KERNEL_TAPS and x.shape[-1] <= FIR_KERNEL_MAX_C:
        return torch.ops.pnfx.fir_fwd.default(x, taps.reshape(-1))
    return causal_fir(x, taps)


def hip_causal_fir_heads(k: torch.Tensor, taps: torch.Tensor) -> torch.Tensor:
    """Causal FIR along N of keys in [B, H, N, d] layout with per-head taps [H, K] (or shared [K])."""
    if not k.is_cuda:
        raise RuntimeError("hip_causal_fir_heads runs on the GPU only")
    return torch.ops.pnfx.fir_fwd.default(k, taps)


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
    w, _, _, _ = torch.ops.pnfx.pn_rows_fwd.default(raw_scores, score_tau, float(scale), float(p),
                                            float(gamma) if has_gamma else 0.0, has_gamma,
                                            bool(causal_mask))
    return w


# Head sizes up to this have flash kernels (16, 32, 64, 128, the others zero-padded to the next
# one inside the ops); larger heads take _materialised_attention.
FLASH_MAX_HEAD_DIM = 128


def _materialised_attention(q, k, v, score_tau, scale, gamma, causal_mask):
    """pn_fir_tau attention for head sizes above FLASH_MAX_HEAD_DIM: the [B, H, N, N] scores in
    fp32 (the reference's kernels accumulate q k^T in fp32 too), the HIP row-fused score kernel
    in fp32 (pnfx::pn_rows_fwd, p = 10 and the peak gate) and W V in fp32, with autograd
    through all three.  The same values as the flash path (src/triton_pnfirtau.py:313-621) at
    O(N^2) memory -- the reference's flash kernel covers any head size by padding it to a power
    of two (:839-841), which this GPU's flash kernels stop at 128."""
    has_gamma = gamma is not None and gamma > 0.0
    raw = torch.matmul(q.float(), k.float().transpose(-2, -1))
    w = torch.ops.pnfx.pn_rows_fwd.default(raw, score_tau, float(scale), 10.0,
                                           float(gamma) if has_gamma else 0.0, has_gamma,
                                           bool(causal_mask))[0]
    return torch.matmul(w, v.float()).to(q.dtype)


def _flash_attention(q, k, v, score_tau, scale, gamma, causal_mask, o_bnhd=False):
    if not q.is_cuda:
        raise RuntimeError("flash_pn_fir_tau_attention runs on the GPU only (as in the reference)")
    # The reference's kernel types each operand separately; the HIP kernels take one dtype,
    # so k and v are brought to q's (autograd casts their gradients back).
    k = k if k.dtype == q.dtype else k.to(q.dtype)
    v = v if v.dtype == q.dtype else v.to(q.dtype)
    if q.shape[-1] > FLASH_MAX_HEAD_DIM:
        return _materialised_attention(q, k, v, score_tau, scale, gamma, causal_mask)
    has_gamma = gamma is not None and gamma > 0.0
    o = torch.ops.pnfx.flash_fwd.default(q, k, v, score_tau, float(scale),
                                 float(gamma) if has_gamma else 0.0, has_gamma,
                                 bool(causal_mask), bool(o_bnhd), False)[0]
    return o


# PnFirTauFlashMHA's inference forward (no autograd) runs the key FIR inside the flash
# forward's key-tile load when this is set and fused_fir_forward_applies(); False keeps the two
# launches (FIR, then flash) everywhere.
FUSED_FIR_INFERENCE = True
# The fused forward filters each key tile once per 128-query block that reads it, so its extra
# work grows with N while the launch it saves does not.  Measured on MI355X (GPU time per
# forward, from replayed HIP graphs): 0.80x the two launches at B=64 H=4 N=256 d=16, 0.95x at
# B=32 H=4 N=512 d=64, 1.04x at B=16 H=4 N=1024 d=16 and 1.64x at B=4 H=16 N=8192 d=64.
FUSED_FIR_MAX_N = 512


def fused_fir_forward_applies(q: torch.Tensor, k_raw: torch.Tensor, taps: torch.Tensor,
                              head_dim: int) -> bool:
    """Whether the module's forward may take the fused FIR + flash forward: inference (no
    tensor needs a gradient), bf16 GPU tensors, the reference's 7-tap kernel path of
    hip_causal_fir (src/triton_pnfirtau.py:687: K == 7, at most 1024 channels), a head size
    the fused kernel covers and a sequence where it measures faster (N <= FUSED_FIR_MAX_N).
    k_raw is [B, N, D]."""
    if not (FUSED_FIR_INFERENCE and q.is_cuda and q.dtype == torch.bfloat16
            and k_raw.dtype == torch.bfloat16 and head_dim in (16, 32, 64)
            and k_raw.shape[-2] <= FUSED_FIR_MAX_N
            and taps.numel() == FIR_KERNEL_TAPS and k_raw.shape[-1] <= FIR_KERNEL_MAX_C):
        return False
    return not (torch.is_grad_enabled() and (q.requires_grad or k_raw.requires_grad
                                              or taps.requires_grad))


def fused_fir_flash_forward(q, k_raw, v, taps, score_tau, scale, gamma, causal_mask):
    """O [B, H, N, d] (backed by [B, N, H, d] memory) of the flash forward with the causal FIR of
    the raw keys fused into its key-tile load: bitwise hip_causal_fir followed by
    flash_pn_fir_tau_attention (src/pnfirtau_attention.py:299-315) for the inputs
    fused_fir_forward_applies() accepts.  No autograd."""
    v = v if v.dtype == q.dtype else v.to(q.dtype)
    has_gamma = gamma is not None and gamma > 0.0
    return torch.ops.pnfx.flash_fwd_fir.default(q, k_raw, v, score_tau, taps.reshape(-1),
                                                float(scale), float(gamma) if has_gamma else 0.0,
                                                has_gamma, bool(causal_mask), True)[0]


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
    score_tau (src/triton_pnfirtau.py:814-983).  Any head size: 16, 32, 64 and 128 have
    kernels, other sizes up to 128 are zero-padded to the next of these, and larger heads
    take the materialised-score path (_materialised_attention).
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return _flash_attention(q, k_tilde, v, score_tau, scale, gamma, causal_mask)


def flash_pn_fir_tau_attention_with_stats(q, k_tilde, v, score_tau, scale=None, gamma=0.5,
                                          causal_mask=True):
    """Forward only: (O, M, Z, Nmax, tile_mask) -- the saved statistics and the silence map.

    M is the row peak of u = relu(q k^T scale - tau), Nmax its tie count, and Z the
    reference's normaliser: the sum of P = u^10 (unrounded fp32) plus 1e-12
    (src/triton_pnfirtau.py:405, :422).  For bf16 inputs P is rounded to bf16 before it
    weights V (as the reference's kernel does, :417-420), and O is divided by the sum of
    exactly those rounded values, so that it is a convex combination of the rows of V scaled
    by the gate (the reference divides by Z; the two normalisers differ by the rounding of
    the P terms, a relative 2^-8 at most).  For fp32 inputs both are the fp32 sum.
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if q.shape[-1] > FLASH_MAX_HEAD_DIM:
        raise ValueError(f"head dim {q.shape[-1]}: the flash statistics exist for head sizes up "
                         f"to {FLASH_MAX_HEAD_DIM} (larger heads run the materialised path)")
    has_gamma = gamma is not None and gamma > 0.0
    k_tilde = k_tilde if k_tilde.dtype == q.dtype else k_tilde.to(q.dtype)
    v = v if v.dtype == q.dtype else v.to(q.dtype)
    o, _, M, Z, Nm, mask = torch.ops.pnfx.flash_fwd.default(q, k_tilde, v, score_tau, float(scale),
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
