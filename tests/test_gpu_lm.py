"""GPU tests of the LM consumer of the path: training with the flash attention against the
eager module, and the HIP-graph-captured training step against the eager step.

The eager ``PnFirTauMHA`` is the reference module restated (pinned by the C1 golden
fixtures); here it runs on the GPU with torch ops and serves as the fp32 reference of a whole
training run (experiments/exp4_wikitext2_lm.py:385-455 compares the reference's variants the
same way, on matched seeds and data).
"""
import pytest
import torch

from paper_01_anti_decoy_pnfirtau_amd.wikilm import (GraphedStep, WikiLM, WikiLMConfig, lm_loss,
                                                      make_optimizer, train_step)

pytestmark = pytest.mark.gpu

VOCAB = 300
CFG = WikiLMConfig(d_model=64, n_heads=4, n_layers=2, d_ff=128, max_seq=128, dropout=0.0)


def _model(variant, dev, seed=0):
    torch.manual_seed(seed)
    return WikiLM(VOCAB, CFG, variant).to(dev)


def _batches(dev, n, batch=4, seq=128, seed=1):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, VOCAB, (batch, seq), generator=g).to(dev) for _ in range(n)]


def test_lm_flash_gradients_match_eager_fp32(dev):
    """Step-0 gradients of every parameter, flash (fp32 kernels) vs eager, fp32: 1e-4 of scale."""
    print("[lm grads fp32]", flush=True)
    x = _batches(dev, 1)[0]
    grads = {}
    for variant in ("pn_fir_tau", "pn_fir_tau_flash"):
        m = _model(variant, dev)
        lm_loss(m, x, amp=False).backward()
        grads[variant] = {n: p.grad.detach().clone() for n, p in m.named_parameters()}
    torch.cuda.synchronize()
    ref, got = grads["pn_fir_tau"], grads["pn_fir_tau_flash"]
    assert ref.keys() == got.keys()
    for n in ref:
        scale = ref[n].abs().max().item()
        err = (got[n] - ref[n]).abs().max().item()
        assert err <= 1e-4 * max(scale, 1e-12), f"{n}: max err {err:.3g} of scale {scale:.3g}"


def test_lm_flash_training_matches_eager_fp32(dev):
    """Eight AdamW steps on the same data: per-step loss of the flash model within 1e-4
    (relative) of the eager model's, all in fp32."""
    print("[lm train fp32]", flush=True)
    xs = _batches(dev, 8)
    losses = {}
    for variant in ("pn_fir_tau", "pn_fir_tau_flash"):
        m = _model(variant, dev)
        opt = make_optimizer(m, CFG)
        losses[variant] = [float(train_step(m, opt, x, amp=False)) for x in xs]
    for i, (a, b) in enumerate(zip(losses["pn_fir_tau"], losses["pn_fir_tau_flash"])):
        assert abs(a - b) <= 1e-4 * abs(a), f"step {i}: eager {a} flash {b}"
    assert losses["pn_fir_tau_flash"][-1] < losses["pn_fir_tau_flash"][0]


def test_lm_bf16_flash_training_tracks_fp32_eager(dev):
    """The bf16-autocast flash model trains like the fp32 eager model: per-step loss within
    1e-2 (relative) over eight steps."""
    print("[lm train bf16]", flush=True)
    xs = _batches(dev, 8, seed=2)
    m = _model("pn_fir_tau", dev)
    opt = make_optimizer(m, CFG)
    ref = [float(train_step(m, opt, x, amp=False)) for x in xs]
    m = _model("pn_fir_tau_flash", dev)
    opt = make_optimizer(m, CFG)
    got = [float(train_step(m, opt, x, amp=True)) for x in xs]
    for i, (a, b) in enumerate(zip(ref, got)):
        assert abs(a - b) <= 1e-2 * abs(a), f"step {i}: fp32 eager {a} bf16 flash {b}"


def test_graphed_lm_step_matches_eager_step(dev):
    """The captured training step (forward, backward, AdamW) replayed five times, with the
    eager model's own steps and host synchronisations between replays: every replay's loss
    matches the eager step on the same weights and data (bf16 autocast)."""
    print("[lm graph]", flush=True)
    xs = _batches(dev, 8, seed=3)
    eager = _model("pn_fir_tau_flash", dev)
    opt_e = make_optimizer(eager, CFG, capturable=True)
    graphed = _model("pn_fir_tau_flash", dev)
    opt_g = make_optimizer(graphed, CFG, capturable=True)
    static_x = xs[0].clone()
    g = GraphedStep(graphed, opt_g, static_x, amp=True, warmup=3)  # takes 3 steps on xs[0]
    for _ in range(3):
        train_step(eager, opt_e, xs[0], amp=True)
    torch.cuda.synchronize()
    for i in range(1, 6):
        le = float(train_step(eager, opt_e, xs[i], amp=True))
        torch.cuda.synchronize()
        static_x.copy_(xs[i])
        lg = float(g.replay())
        torch.cuda.synchronize()
        assert abs(le - lg) <= 1e-3 * abs(le), f"replay {i}: eager {le} graph {lg}"
