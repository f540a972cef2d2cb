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
                                                      make_optimizer, train_step, zipf_tokens)
from paper_01_anti_decoy_pnfirtau_amd import causal_fir
from tests.helpers import PARITY_LOG

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
    matches the eager step on the same weights and data (bf16 autocast).  Capture leaves the
    weights and optimizer state as they were, so both start from the same initial model."""
    print("[lm graph]", flush=True)
    xs = _batches(dev, 8, seed=3)
    eager = _model("pn_fir_tau_flash", dev)
    opt_e = make_optimizer(eager, CFG, capturable=True)
    graphed = _model("pn_fir_tau_flash", dev)
    opt_g = make_optimizer(graphed, CFG, capturable=True)
    static_x = xs[0].clone()
    g = GraphedStep(graphed, opt_g, static_x, amp=True, warmup=3)
    for a, b in zip(eager.parameters(), graphed.parameters()):
        assert torch.equal(a, b)
    torch.cuda.synchronize()
    for i in range(0, 5):
        le = float(train_step(eager, opt_e, xs[i], amp=True))
        torch.cuda.synchronize()
        static_x.copy_(xs[i])
        lg = float(g.replay())
        torch.cuda.synchronize()
        assert abs(le - lg) <= 1e-3 * abs(le), f"replay {i}: eager {le} graph {lg}"


def test_graphed_flash_step_matches_eager_reference_module_fp32(dev):
    """The graph-replayed flash training step against the eager PnFirTauMHA model (the
    reference's own attention, restated) in fp32: five replays, each loss within 1e-4
    (relative) of the eager model's on the same data (experiments/exp4c_cuda_graphs.py:81-108
    captures the flash stack the same way)."""
    print("[lm graph vs eager reference fp32]", flush=True)
    xs = _batches(dev, 6, seed=4)
    ref = _model("pn_fir_tau", dev)
    opt_r = make_optimizer(ref, CFG, capturable=True)
    graphed = _model("pn_fir_tau_flash", dev)
    opt_g = make_optimizer(graphed, CFG, capturable=True)
    static_x = xs[0].clone()
    g = GraphedStep(graphed, opt_g, static_x, amp=False, warmup=2)
    for i in range(5):
        lr = float(train_step(ref, opt_r, xs[i], amp=False))
        static_x.copy_(xs[i])
        lg = float(g.replay())
        torch.cuda.synchronize()
        assert abs(lr - lg) <= 1e-4 * abs(lr), f"replay {i}: eager reference {lr} graph {lg}"


# The benchmark's LM workload C3 (D=256, H=4, d_ff=1024, 6 layers, N=512, B=32, vocab 33278)
# and the reference's exp4 shape (experiments/exp4_wikitext2_lm.py:6, :67-88: D=64, H=4,
# 6 layers, d_ff=256, N=256, vocab 23168), dropout 0 so that both variants see the same
# computation.
C3 = dict(cfg=WikiLMConfig(d_model=256, n_heads=4, n_layers=6, d_ff=1024, max_seq=512,
                           dropout=0.0), vocab=33278, batch=32, seq=512)
EXP4 = dict(cfg=WikiLMConfig(d_model=64, n_heads=4, n_layers=6, d_ff=256, max_seq=256,
                             dropout=0.0), vocab=23168, batch=64, seq=256)


def _lm(shape, variant, dev, seed=0):
    torch.manual_seed(seed)
    return WikiLM(shape["vocab"], shape["cfg"], variant).to(dev)


def _grads(model, x, amp):
    model.zero_grad(set_to_none=True)
    loss = lm_loss(model, x, amp)
    loss.backward()
    torch.cuda.synchronize()
    return float(loss.detach()), {n: p.grad.detach().double().clone()
                                  for n, p in model.named_parameters()}


def _rel(a, b):
    """max |a - b| / max |b| per tensor."""
    return {n: (a[n] - b[n]).abs().max().item() / max(b[n].abs().max().item(), 1e-300) for n in b}


def _max_rel(a, b):
    return max(_rel(a, b).values())


def _peak_tie_rows(model, x):
    """Rows of the flash LM's attention layers whose fp32 peak score is tied (Nmax > 1) on
    tokens x: each layer's q, k~, v recomputed from its input and run through the forward
    with statistics."""
    from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import (flash_pn_fir_tau_attention_with_stats,
                                                               hip_causal_fir)

    ties = []

    def hook(mod, inp, out):
        h = inp[0]
        B, N, D = h.shape
        q, k_raw, v = mod.qkv(h).split(D, dim=-1)
        k = mod._split_heads(hip_causal_fir(k_raw, mod.fir_taps))
        st = flash_pn_fir_tau_attention_with_stats(mod._split_heads(q), k, mod._split_heads(v),
                                                   mod.score_tau, gamma=mod.cfg.silence_gamma)
        ties.append(int((st[3] > 1).sum()))

    hs = [blk.attn.register_forward_hook(hook) for blk in model.blocks]
    with torch.no_grad():
        model(x)
    for hnd in hs:
        hnd.remove()
    return sum(ties)


def _tau_conditioning(model64, x):
    """sum_ij |du_ij| of every attention layer of a float64 eager LM on tokens x: the scale
    of the cancelling sum dtau = -sum du.  Each layer's q, k~, v and the gradient reaching
    its attention output are taken from hooks and handed to the float64 oracle."""
    import numpy as np

    from oracle import pnfirtau_oracle as O

    mods = [blk.attn for blk in model64.blocks]
    cap = {}
    hs = []
    for i, mod in enumerate(mods):
        hs.append(mod.register_forward_hook(lambda m, a, o, i=i: cap.__setitem__(("h", i), a[0].detach())))
        hs.append(mod.register_full_backward_hook(
            lambda m, gi, go, i=i: cap.__setitem__(("gy", i), go[0].detach())))
    model64.zero_grad(set_to_none=True)
    lm_loss(model64, x, False).backward()
    for hnd in hs:
        hnd.remove()
    out = []
    with torch.no_grad():
        for i, mod in enumerate(mods):
            h, gy = cap[("h", i)], cap[("gy", i)]
            B, N, D = h.shape
            q, k_raw, v = mod.qkv(h).split(D, dim=-1)
            k = causal_fir(k_raw, mod.fir_taps)
            do = gy @ mod.out.weight  # gradient at the heads' merged output
            heads = lambda t: mod._split_heads(t).cpu().numpy()  # noqa: E731
            *_, dabs = O.flash_bwd(heads(q), heads(k), heads(v), float(mod.score_tau), heads(do),
                                   1.0 / np.sqrt(mod.head_dim), mod.cfg.silence_gamma, True,
                                   return_abs=True)
            out.append(float(dabs))
    model64.zero_grad(set_to_none=True)
    return out


def test_c3_lm_flash_matches_eager_fp32(dev):
    """C3 in fp32, against the same LM evaluated in float64 with the eager PnFirTauMHA: the
    flash LM's step-0 gradient of every parameter is no further from the float64 gradient
    than the fp32 eager LM's is (x2, plus 1e-6 of the tensor's scale), its loss within 1e-6;
    then three AdamW steps' losses within 1e-4 (relative) of the fp32 eager model's.  The
    score_tau gradients are sums with cancellation: their error is bounded by 1e-5 of
    |dtau| + sum |du| (the float64 oracle's sum for that layer), as in the kernel tests.

    The token batch is the first of seeds 0, 1, 2, ... on which no attention row of the fp32
    flash model has two keys tied at its peak: a tie that exists only in fp32 rounding splits
    the peak-gate gradient between the two keys (the tie rule of the reference, whose amax
    backward splits it the same way), where the float64 model gives it to one key -- a
    discontinuity of the gradient, not an error of the kernels.  (Seed 0 has one such row in
    393 216 at layer 1; the tie rule itself is tested against the oracle on planted ties.)"""
    print("[lm C3 fp32]", flush=True)
    fl = _lm(C3, "pn_fir_tau_flash", dev)
    for seed in range(8):
        x0 = zipf_tokens(C3["batch"], C3["seq"], C3["vocab"], seed).to(dev)
        if _peak_tie_rows(fl, x0) == 0:
            break
    else:
        raise AssertionError("no tie-free token batch among 8 seeds")
    xs = [x0] + [zipf_tokens(C3["batch"], C3["seq"], C3["vocab"], 100 + i).to(dev) for i in range(2)]
    del fl
    ref64 = _lm(C3, "pn_fir_tau", dev).double()
    du_abs = _tau_conditioning(ref64, xs[0])
    l64, g64 = _grads(ref64, xs[0], False)
    del ref64
    ref, fl = _lm(C3, "pn_fir_tau", dev), _lm(C3, "pn_fir_tau_flash", dev)
    lr, gr = _grads(ref, xs[0], False)
    lf, gf = _grads(fl, xs[0], False)
    er, ef = _rel(gr, g64), _rel(gf, g64)
    PARITY_LOG.append({"test": "c3_lm_fp32", "what": "step-0 grads, max err / scale vs float64",
                       "eager_fp32": max(er.values()), "flash_fp32": max(ef.values()),
                       "loss": [l64, lr, lf]})
    print(f"[lm C3 fp32] grad error vs float64: eager {max(er.values()):.3g}, flash "
          f"{max(ef.values()):.3g}; loss {l64:.8f} / {lr:.8f} / {lf:.8f}", flush=True)
    assert abs(lf - l64) <= 1e-6 * abs(l64)
    for n in g64:
        if n.endswith("score_tau"):  # a sum with cancellation: bounded against sum |du|
            i = int(n.split(".")[1])
            err = abs(float(gf[n]) - float(g64[n]))
            PARITY_LOG.append({"test": "c3_lm_fp32", "what": n, "abs_err": err,
                               "eager_abs_err": abs(float(gr[n]) - float(g64[n])),
                               "dtau": float(g64[n]), "sum_abs_du": du_abs[i]})
            assert err <= 1e-5 * (abs(float(g64[n])) + du_abs[i]), (n, err, du_abs[i])
            continue
        assert ef[n] <= 2 * er[n] + 1e-6, f"{n}: flash {ef[n]:.3g}, eager {er[n]:.3g}"
    del gr, gf, g64
    opt_r, opt_f = make_optimizer(ref, C3["cfg"]), make_optimizer(fl, C3["cfg"])
    for i, x in enumerate(xs):
        a, b = float(train_step(ref, opt_r, x, amp=False)), float(train_step(fl, opt_f, x, amp=False))
        assert abs(a - b) <= 1e-4 * abs(a), f"step {i}: eager {a} flash {b}"


def test_c3_lm_bf16_flash_vs_fp32_eager(dev):
    """C3 under bf16 autocast: the flash LM's step-0 gradients are as close to the fp32 eager
    LM's as the eager LM's own bf16-autocast gradients are (the reference's bf16 path), and
    its losses over three AdamW steps track the fp32 eager model's within 1e-2."""
    print("[lm C3 bf16]", flush=True)
    xs = [zipf_tokens(C3["batch"], C3["seq"], C3["vocab"], 10 + seed).to(dev) for seed in range(3)]
    ref = _lm(C3, "pn_fir_tau", dev)
    _, g32 = _grads(ref, xs[0], False)
    _, gref16 = _grads(ref, xs[0], True)
    fl = _lm(C3, "pn_fir_tau_flash", dev)
    _, gfl16 = _grads(fl, xs[0], True)
    e_ref, e_fl = _max_rel(gref16, g32), _max_rel(gfl16, g32)
    PARITY_LOG.append({"test": "c3_lm_bf16", "what": "step-0 grads, max err / scale vs fp32 eager",
                       "eager_bf16": e_ref, "flash_bf16": e_fl})
    print(f"[lm C3 bf16] grad error vs fp32 eager: eager bf16 {e_ref:.3g}, flash bf16 {e_fl:.3g}",
          flush=True)
    assert e_fl <= max(1.5 * e_ref, 2e-2)
    del g32, gref16, gfl16
    opt_r, opt_f = make_optimizer(ref, C3["cfg"]), make_optimizer(fl, C3["cfg"])
    for i, x in enumerate(xs):
        a, b = float(train_step(ref, opt_r, x, amp=False)), float(train_step(fl, opt_f, x, amp=True))
        assert abs(a - b) <= 1e-2 * abs(a), f"step {i}: fp32 eager {a} bf16 flash {b}"


@pytest.mark.parametrize("amp,tol", [(False, 1e-3), (True, 2e-2)])
def test_exp4_shape_training_run_tracks_eager(dev, amp, tol):
    """The reference's matched-run protocol (experiments/exp4_wikitext2_lm.py:320-360) at its
    LM shape on synthetic Zipf tokens: 50 AdamW steps of the flash LM (fp32, or bf16 autocast)
    against the fp32 eager PnFirTauMHA LM from the same initial weights; every step's loss
    within `tol` (relative), and both runs learn (final loss below the first)."""
    print(f"[lm exp4 shape amp={amp}]", flush=True)
    ref, fl = _lm(EXP4, "pn_fir_tau", dev), _lm(EXP4, "pn_fir_tau_flash", dev)
    opt_r, opt_f = make_optimizer(ref, EXP4["cfg"]), make_optimizer(fl, EXP4["cfg"])
    worst, la, lb = 0.0, [], []
    for i in range(50):
        x = zipf_tokens(EXP4["batch"], EXP4["seq"], EXP4["vocab"], 100 + i).to(dev)
        a, b = float(train_step(ref, opt_r, x, amp=False)), float(train_step(fl, opt_f, x, amp=amp))
        la.append(a)
        lb.append(b)
        worst = max(worst, abs(a - b) / abs(a))
    PARITY_LOG.append({"test": "exp4_shape_training", "what": f"amp={amp}", "worst_rel": worst,
                       "first": [la[0], lb[0]], "last": [la[-1], lb[-1]]})
    print(f"[lm exp4 amp={amp}] worst per-step loss deviation {worst:.3g}; "
          f"loss {la[0]:.4f} -> {la[-1]:.4f} (eager), {lb[0]:.4f} -> {lb[-1]:.4f} (flash)", flush=True)
    assert worst <= tol
    assert la[-1] < la[0] and lb[-1] < lb[0]
