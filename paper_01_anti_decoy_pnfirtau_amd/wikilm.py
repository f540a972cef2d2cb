"""The language model that consumes the pn_fir_tau attention path, and its training step.

Mirrors the reference's WikiText-2 model and step (``experiments/exp4_wikitext2_lm.py``):

* ``Block``   :183-201 -- pre-LN residual block: x + drop(attn(ln1 x)), then
  x + ffn(ln2 x) with ffn = Linear -> GELU -> Linear -> Dropout;
* ``WikiLM``  :203-247 -- token + learned position embeddings, ``n_layers`` blocks with the
  chosen attention module, final LayerNorm and a head tied to the token embedding;
* ``train_step`` :334-348 -- zero_grad, bf16 autocast forward, next-token cross-entropy,
  backward, AdamW (betas 0.9/0.95).

``GraphedStep`` captures that whole step (including the optimizer update) in one HIP graph,
as the reference's ``experiments/exp4c_cuda_graphs.py:81-108`` does for the attention stack:
the eager stack is launch-bound at these sizes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .pnfirtau_attention import PnFirConfig, PnFirTauFlashMHA, PnFirTauMHA, PnFirTauTritonMHA

ATTENTION = {
    "pn_fir_tau": PnFirTauMHA,
    "pn_fir_tau_triton": PnFirTauTritonMHA,
    "pn_fir_tau_flash": PnFirTauFlashMHA,
}


@dataclass
class WikiLMConfig:
    """Model shape and optimiser settings (defaults of experiments/exp4_wikitext2_lm.py:67-88)."""

    d_model: int = 64
    n_heads: int = 4
    n_layers: int = 6
    d_ff: int = 256
    max_seq: int = 256
    lr: float = 5e-4
    weight_decay: float = 0.1
    dropout: float = 0.1
    p: float = 10.0
    silence_gamma: float = 0.5
    tau_init: float = 0.0
    fir_k: int = 7


class Block(nn.Module):
    """Pre-LN residual block (experiments/exp4_wikitext2_lm.py:183-201)."""

    def __init__(self, d_model: int, attn: nn.Module, dropout: float, d_ff: int):
        super().__init__()
        self.ln1 = nn.LayerNorm(d_model)
        self.attn = attn
        self.ln2 = nn.LayerNorm(d_model)
        self.ffn = nn.Sequential(
            nn.Linear(d_model, d_ff), nn.GELU(), nn.Linear(d_ff, d_model), nn.Dropout(dropout)
        )
        self.drop = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.drop(self.attn(self.ln1(x)))
        return x + self.ffn(self.ln2(x))


class WikiLM(nn.Module):
    """Decoder-only LM with pn_fir_tau attention (experiments/exp4_wikitext2_lm.py:203-247).

    ``variant`` picks the attention module: ``pn_fir_tau`` (eager), ``pn_fir_tau_triton``
    (row-fused scores) or ``pn_fir_tau_flash`` (flash).  Parameters are created in the
    reference's order, so the same seed gives the same initial weights for every variant.
    """

    def __init__(self, vocab: int, cfg: WikiLMConfig, variant: str = "pn_fir_tau_flash"):
        super().__init__()
        if variant not in ATTENTION:
            raise ValueError(f"Unknown variant: {variant}")
        self.cfg = cfg
        self.variant = variant
        self.embed = nn.Embedding(vocab, cfg.d_model)
        self.pos = nn.Embedding(cfg.max_seq, cfg.d_model)
        self.drop = nn.Dropout(cfg.dropout)
        acfg = PnFirConfig(
            d_model=cfg.d_model, n_heads=cfg.n_heads, p=cfg.p, silence_gamma=cfg.silence_gamma,
            tau_init=cfg.tau_init, fir_k=cfg.fir_k, dropout=cfg.dropout, causal_mask=True,
            bias=False,
        )
        self.blocks = nn.ModuleList(
            Block(cfg.d_model, ATTENTION[variant](acfg), cfg.dropout, cfg.d_ff)
            for _ in range(cfg.n_layers)
        )
        self.ln_f = nn.LayerNorm(cfg.d_model)
        self.head = nn.Linear(cfg.d_model, vocab, bias=False)
        self.head.weight = self.embed.weight

    def forward(self, idx: torch.Tensor) -> torch.Tensor:
        _, n = idx.shape
        pos = torch.arange(n, device=idx.device).unsqueeze(0)
        h = self.drop(self.embed(idx) + self.pos(pos))
        for blk in self.blocks:
            h = blk(h)
        return self.head(self.ln_f(h))


def zipf_tokens(batch: int, seq: int, vocab: int, seed: int, s: float = 1.1) -> torch.Tensor:
    """Synthetic token ids [batch, seq] ~ Zipf(s) truncated to [0, vocab) by rejection,
    seeded on the CPU (the benchmark LM workload: no dataset is fetched)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    need, out = batch * seq, []
    while need > 0:
        z = rng.zipf(s, size=2 * need) - 1
        z = z[z < vocab][:need]
        out.append(z)
        need -= len(z)
    return torch.from_numpy(np.concatenate(out).reshape(batch, seq).astype(np.int64))


def make_optimizer(model: nn.Module, cfg: WikiLMConfig, capturable: bool = False,
                   fused: bool | None = None):
    """AdamW as the reference builds it (experiments/exp4_wikitext2_lm.py:326-328).

    ``fused=True`` selects torch's single-kernel AdamW (same update rule); with
    ``capturable=True`` it is the cheapest optimizer step to capture in a graph.
    """
    return torch.optim.AdamW(model.parameters(), lr=cfg.lr, betas=(0.9, 0.95),
                             weight_decay=cfg.weight_decay, capturable=capturable, fused=fused)


def lm_loss(model: nn.Module, x: torch.Tensor, amp: bool) -> torch.Tensor:
    """Next-token cross-entropy over the sequence, under bf16 autocast when ``amp``."""
    vocab = model.head.weight.shape[0]
    with torch.autocast(device_type=x.device.type, dtype=torch.bfloat16, enabled=amp):
        logits = model(x)
        return F.cross_entropy(logits[:, :-1].reshape(-1, vocab), x[:, 1:].reshape(-1))


def train_step(model: nn.Module, opt: torch.optim.Optimizer, x: torch.Tensor,
               amp: bool = True) -> torch.Tensor:
    """One step of experiments/exp4_wikitext2_lm.py:334-348; returns the loss (a tensor)."""
    opt.zero_grad(set_to_none=True)
    loss = lm_loss(model, x, amp)
    loss.backward()
    opt.step()
    return loss.detach()


class GraphedStep:
    """The training step of ``train_step`` captured once as a HIP graph and replayed.

    Gradients are cleared by a fill kernel inside the graph (``zero_grad`` with
    ``set_to_none=False``) rather than by dropping the tensors, so the captured addresses stay
    valid; the optimizer must be built with ``capturable=True`` and have no state yet.  ``x``
    is a static input: copy new tokens into it before ``replay``.  The loss of the last replay
    is ``self.loss``.

    Construction runs ``warmup`` real steps on ``x`` (the allocator and the optimizer's state
    must exist before capture), then puts every parameter and buffer back and zeroes the
    optimizer state in place (for Adam-type optimizers a zero state, step count included, is
    the fresh state): the first ``replay`` is the model's first training step.
    """

    def __init__(self, model: nn.Module, opt: torch.optim.Optimizer, x: torch.Tensor,
                 amp: bool = True, warmup: int = 3):
        self.model, self.opt, self.x, self.amp = model, opt, x, amp
        if any(len(st) for st in opt.state.values()):
            raise ValueError("GraphedStep: the optimizer already has state")
        saved = [t.detach().clone() for t in list(model.parameters()) + list(model.buffers())]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.loss = self._step()
        # capture records the step without running it: undo the warm-up steps in place, so
        # the captured addresses stay the live ones
        with torch.no_grad():
            for t, s in zip(list(model.parameters()) + list(model.buffers()), saved):
                t.copy_(s)
            for st in opt.state.values():
                for v in st.values():
                    if torch.is_tensor(v):
                        v.zero_()

    def _step(self) -> torch.Tensor:
        self.opt.zero_grad(set_to_none=False)
        loss = lm_loss(self.model, self.x, self.amp)
        loss.backward()
        self.opt.step()
        return loss.detach()

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.loss
