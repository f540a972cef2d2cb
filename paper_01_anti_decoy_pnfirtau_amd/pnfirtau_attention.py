"""pn_fir_tau attention: eager primitives and the three multi-head modules.

Drop-in for the reference module ``src/pnfirtau_attention.py`` (same names,
signatures, defaults, parameter/buffer names and ``state_dict`` keys):

* ``PnFirConfig``            src/pnfirtau_attention.py:35-47
* ``causal_gaussian_taps``   :50-62
* ``causal_fir``             :65-74   (eager, any device)
* ``power_norm_peak_gate``   :87-119  (eager, any device)
* ``PnFirTauMHA``            :195-247 (eager composition)
* ``PnFirTauTritonMHA``      :250-282 -> HIP FIR + HIP row-fused score kernel
* ``PnFirTauFlashMHA``       :285-316 -> HIP FIR + HIP flash attention

The eager primitives are the path for CPU callers; the two accelerated modules
run their attention core through libpnfx.so on the GPU (``hip_pnfirtau``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class PnFirConfig:
    """Hyper-parameters of one pn_fir_tau attention layer (src/pnfirtau_attention.py:35-47)."""

    d_model: int = 64
    n_heads: int = 4
    p: float = 10.0
    silence_gamma: float | None = 0.5
    silence_mode: str = "peak"
    tau_init: float = 0.0
    fir_k: int = 7
    fir_sigma_frac: float = 3.0
    dropout: float = 0.0
    causal_mask: bool = True
    bias: bool = False


def causal_gaussian_taps(
    k: int,
    device: torch.device | str = "cpu",
    dtype: torch.dtype = torch.float32,
    sigma_frac: float = 3.0,
) -> torch.Tensor:
    """Half-Gaussian causal taps [k]; index k-1 is lag 0 (present), index 0 the oldest lag.

    sigma = max((k-1)/sigma_frac, 0.5); tap(lag) = exp(-lag^2 / (2 sigma^2)), normalised
    to sum 1, evaluated in ``dtype`` (src/pnfirtau_attention.py:50-62).
    """
    assert k % 2 == 1 and k >= 1
    lag = (k - 1) - torch.arange(k, device=device, dtype=dtype)
    sigma = max((k - 1) / sigma_frac, 0.5)
    w = torch.exp(-0.5 * (lag / sigma) ** 2)
    return w / w.sum()


def causal_fir(x: torch.Tensor, taps: torch.Tensor) -> torch.Tensor:
    """Eager depthwise causal FIR along N for x [B, N, C] (src/pnfirtau_attention.py:65-74).

    The taps are cast to x's dtype first (so bf16 inputs use bf16-rounded taps),
    then one grouped convolution over a (K-1)-row causal zero pad.
    """
    K = taps.numel()
    if K <= 1:
        return x
    C = x.shape[-1]
    kernel = taps.to(dtype=x.dtype, device=x.device).reshape(1, 1, K).repeat(C, 1, 1)
    xc = F.pad(x.transpose(1, 2).contiguous(), (K - 1, 0))
    return F.conv1d(xc, kernel, groups=C).transpose(1, 2).contiguous()


def power_norm_peak_gate(
    scores: torch.Tensor,
    p: float = 10.0,
    gamma: float | None = 0.5,
    silence_mode: str = "peak",
) -> torch.Tensor:
    """W = relu(s)^p / (sum relu(s)^p + 1e-12) * gate (src/pnfirtau_attention.py:87-119).

    gate = strength/(strength + gamma) with strength the row peak of relu(s)
    ("peak"), its sum ("mass_relu") or the power mass ("mass_pow"); no gate when
    gamma is None or <= 0.  Row sums equal the gate.
    """
    pos = F.relu(scores)
    if p == 10.0:
        sq = pos * pos
        quad = sq * sq
        pw = quad * quad * sq
    elif p == 2.0:
        pw = pos * pos
    else:
        pw = torch.where(pos > 0, pos.pow(p), torch.zeros_like(pos))
    mass = pw.sum(dim=-1, keepdim=True)
    w = pw / (mass + 1e-12)
    if gamma is None or gamma <= 0:
        return w
    if silence_mode == "peak":
        strength = pos.amax(dim=-1, keepdim=True)
    elif silence_mode == "mass_relu":
        strength = pos.sum(dim=-1, keepdim=True)
    elif silence_mode == "mass_pow":
        strength = mass
    else:
        raise ValueError(f"unknown silence_mode={silence_mode}")
    return w * (strength / (strength + gamma))


def _causal_fill(scores: torch.Tensor) -> torch.Tensor:
    n = scores.shape[-1]
    upper = torch.ones(n, n, device=scores.device, dtype=torch.bool).triu_(1)
    return scores.masked_fill(upper, -1e4)


class PnFirTauMHA(nn.Module):
    """pn_fir_tau multi-head attention, eager composition (src/pnfirtau_attention.py:195-247).

    Parameters are created in the reference order ``qkv``, ``out``, ``score_tau``
    (so default init consumes the RNG identically) and ``fir_taps`` is a
    persistent buffer: checkpoints of the reference load unchanged.
    """

    def __init__(self, cfg: PnFirConfig):
        super().__init__()
        assert cfg.d_model % cfg.n_heads == 0
        assert cfg.fir_k % 2 == 1
        self.cfg = cfg
        self.n_heads = cfg.n_heads
        self.head_dim = cfg.d_model // cfg.n_heads
        self.qkv = nn.Linear(cfg.d_model, 3 * cfg.d_model, bias=cfg.bias)
        self.out = nn.Linear(cfg.d_model, cfg.d_model, bias=cfg.bias)
        self.drop = nn.Dropout(cfg.dropout)
        self.score_tau = nn.Parameter(torch.tensor(float(cfg.tau_init)))
        self.register_buffer(
            "fir_taps",
            causal_gaussian_taps(cfg.fir_k, torch.device("cpu"), torch.float32, cfg.fir_sigma_frac),
            persistent=True,
        )

    def _split_heads(self, t: torch.Tensor) -> torch.Tensor:
        B, N, _ = t.shape
        return t.reshape(B, N, self.n_heads, self.head_dim).transpose(1, 2)

    def forward(self, x: torch.Tensor, return_weights: bool = False):
        cfg = self.cfg
        B, N, D = x.shape
        q, k_raw, v = self.qkv(x).split(D, dim=-1)
        k = causal_fir(k_raw, self.fir_taps)
        q, k, v = self._split_heads(q), self._split_heads(k), self._split_heads(v)
        scores = torch.matmul(q, k.transpose(-2, -1)) * (1.0 / math.sqrt(self.head_dim))
        scores = scores - self.score_tau
        if cfg.causal_mask:
            scores = _causal_fill(scores)
        w = self.drop(power_norm_peak_gate(scores, cfg.p, cfg.silence_gamma, cfg.silence_mode))
        out = self.out(torch.matmul(w, v).transpose(1, 2).reshape(B, N, D))
        return (out, w) if return_weights else out


class PnFirTauTritonMHA(PnFirTauMHA):
    """Materialised-score variant: HIP FIR + HIP row-fused score kernel (src/pnfirtau_attention.py:250-282).

    The class keeps the reference's name so that existing model code and
    checkpoints switch over unchanged; nothing here uses Triton.
    """

    def forward(self, x: torch.Tensor, return_weights: bool = False):
        from .hip_pnfirtau import hip_causal_fir, hip_pn_fir_tau_scores

        cfg = self.cfg
        B, N, D = x.shape
        q, k_raw, v = self.qkv(x).split(D, dim=-1)
        k = self._split_heads(hip_causal_fir(k_raw, self.fir_taps))
        q, v = self._split_heads(q), self._split_heads(v)
        raw = torch.matmul(q, k.transpose(-2, -1))
        w = hip_pn_fir_tau_scores(raw, self.score_tau, scale=1.0 / math.sqrt(self.head_dim),
                                  p=cfg.p, gamma=cfg.silence_gamma, causal_mask=cfg.causal_mask)
        w = self.drop(w)
        out = self.out(torch.matmul(w, v).transpose(1, 2).reshape(B, N, D))
        return (out, w) if return_weights else out


class PnFirTauFlashMHA(PnFirTauMHA):
    """O(N)-memory flash variant: HIP FIR + HIP flash kernels with silent-tile skipping.

    Mirrors src/pnfirtau_attention.py:285-316, including its conventions: p = 10
    and the peak gate are fixed (cfg.p / cfg.silence_mode are not consulted), no
    attention dropout, and ``return_weights=True`` takes the row-fused path.
    The flash output is produced in [B, N, H, hd] memory order, so the merge of
    heads before the output projection is a view.
    """

    def forward(self, x: torch.Tensor, return_weights: bool = False):
        if return_weights:
            return PnFirTauTritonMHA.forward(self, x, return_weights=True)
        from . import hip_pnfirtau as hp

        cfg = self.cfg
        B, N, D = x.shape
        q, k_raw, v = self.qkv(x).split(D, dim=-1)
        if hp.fused_fir_forward_applies(q, k_raw, self.fir_taps, self.head_dim):
            # inference: the key FIR inside the forward's key-tile load (one launch, same bits)
            o = hp.fused_fir_flash_forward(self._split_heads(q), self._split_heads(k_raw),
                                           self._split_heads(v), self.fir_taps, self.score_tau,
                                           1.0 / math.sqrt(self.head_dim), cfg.silence_gamma,
                                           cfg.causal_mask)
            return self.out(o.transpose(1, 2).reshape(B, N, D))
        k = self._split_heads(hp.hip_causal_fir(k_raw, self.fir_taps))
        q, v = self._split_heads(q), self._split_heads(v)
        o = hp._flash_attention(q, k, v, self.score_tau, 1.0 / math.sqrt(self.head_dim),
                                cfg.silence_gamma, cfg.causal_mask, o_bnhd=True)
        return self.out(o.transpose(1, 2).reshape(B, N, D))
