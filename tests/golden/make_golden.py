"""Write golden vectors from the reference implementation itself.

Run once, in the build container only (the GPU box has no reference tree):

    python tests/golden/make_golden.py /root/reference

It imports the reference's eager module ``src/pnfirtau_attention.py`` (and the
CPU fallback of ``src/triton_pnfirtau.py``) and stores inputs and outputs as
small ``.npz`` fixtures next to this script.  Only data is stored: inputs,
weights, outputs and gradients.  The fixtures pin what no closed form pins:

* ``c1_mha_*``: PnFirTauMHA forward + backward (head split, FIR on K over the
  H*hd channels, mask, gate) at config C1 (B=2, N=128, D=64, H=4) in fp32,
  plus variants (tau != 0, bias, other gate modes) and a bf16 run;
* ``pn_gate``: power_norm_peak_gate outputs and autograd grads for every
  (p, gamma, silence_mode) branch, including planted ties (amax tie split);
* ``fir_eager``: causal_fir in fp32 and bf16 (bf16 rounds the taps first);
* ``scores_fallback``: the eager fallback of triton_pn_fir_tau_scores.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def mha_case(ref, name, *, tau=0.0, bias=False, gamma=0.5, mode="peak", p=10.0,
             dtype=torch.float32, B=2, N=128, D=64, H=4, seed=0, store_w=False):
    cfg = ref.PnFirConfig(d_model=D, n_heads=H, p=p, silence_gamma=gamma, silence_mode=mode,
                          tau_init=tau, bias=bias, dropout=0.0)
    torch.manual_seed(seed)
    m = ref.PnFirTauMHA(cfg)  # default nn.Linear init from the CPU RNG
    m = m.to(dtype)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, N, D, generator=g).to(dtype).requires_grad_(True)
    dout = torch.randn(B, N, D, generator=g).to(dtype)
    out, W = m(x, return_weights=True)
    out.backward(dout)
    rec = {
        "x": _np(x), "dout": _np(dout), "w_qkv": _np(m.qkv.weight), "w_out": _np(m.out.weight),
        "tau": np.array(float(m.score_tau.detach().float())), "taps": _np(m.fir_taps),
        "out": _np(out), "dx": _np(x.grad), "dw_qkv": _np(m.qkv.weight.grad),
        "dw_out": _np(m.out.weight.grad), "dtau": np.array(float(m.score_tau.grad.float())),
        "meta": np.array([B, N, D, H, int(bias)], dtype=np.int64),
        "gamma": np.array(np.nan if gamma is None else gamma), "p": np.array(p),
        "mode": np.array(mode), "dtype": np.array(str(dtype)),
    }
    if store_w:
        rec["W"] = _np(W)
    if bias:
        rec.update(b_qkv=_np(m.qkv.bias), b_out=_np(m.out.bias),
                   db_qkv=_np(m.qkv.bias.grad), db_out=_np(m.out.bias.grad))
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **rec)
    print("wrote", name, tuple(out.shape))


def pn_gate_cases(ref):
    g = torch.Generator().manual_seed(7)
    s = torch.randn(3, 5, 16, generator=g, dtype=torch.float64) * 1.5
    s[0, 0, 3] = s[0, 0, 9] = s[0, 0].abs().max() + 0.25  # planted tie at the peak
    s[1, 2, :] = -0.5  # silent row
    s[2, 1, 4:8] = 2.0  # four-way tie
    dW = torch.randn(3, 5, 16, generator=g, dtype=torch.float64)
    rec = {"s": s.numpy(), "dW": dW.numpy()}
    cases = [(10.0, 0.5, "peak"), (10.0, None, "peak"), (10.0, 0.0, "peak"), (2.0, 0.5, "peak"),
             (3.5, 0.5, "peak"), (10.0, 0.5, "mass_relu"), (10.0, 0.5, "mass_pow"),
             (2.0, 1.25, "mass_pow")]
    for i, (p, gamma, mode) in enumerate(cases):
        x = s.clone().requires_grad_(True)
        w = ref.power_norm_peak_gate(x, p=p, gamma=gamma, silence_mode=mode)
        w.backward(dW)
        rec[f"w_{i}"] = w.detach().numpy()
        rec[f"ds_{i}"] = x.grad.numpy()
    rec["cases"] = np.array([f"{p}|{gamma}|{mode}" for p, gamma, mode in cases])
    np.savez_compressed(os.path.join(HERE, "pn_gate.npz"), **rec)
    print("wrote pn_gate", len(cases))


def fir_cases(ref):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 20, 8, generator=g)
    taps = ref.causal_gaussian_taps(7)
    rec = {"x": x.numpy(), "taps": taps.numpy(), "y_f32": ref.causal_fir(x, taps).numpy()}
    xb = x.to(torch.bfloat16)
    rec["x_bf16"] = _np(xb)
    rec["y_bf16"] = _np(ref.causal_fir(xb, taps))
    rec["taps5"] = ref.causal_gaussian_taps(5, sigma_frac=2.0).numpy()
    rec["taps1"] = ref.causal_gaussian_taps(1).numpy()
    np.savez_compressed(os.path.join(HERE, "fir_eager.npz"), **rec)
    print("wrote fir_eager")


def scores_fallback(tri):
    g = torch.Generator().manual_seed(13)
    raw = torch.randn(2, 3, 24, 24, generator=g) * 3.0
    tau = torch.tensor(0.4)
    rec = {"raw": raw.numpy(), "tau": tau.numpy()}
    for i, (scale, p, gamma, causal) in enumerate([(0.25, 10.0, 0.5, True), (0.5, 2.0, None, False),
                                                   (0.3, 10.0, 0.5, False)]):
        rec[f"w_{i}"] = tri.triton_pn_fir_tau_scores(raw, tau, scale=scale, p=p, gamma=gamma,
                                                     causal_mask=causal).numpy()
        rec[f"args_{i}"] = np.array([scale, p, np.nan if gamma is None else gamma, float(causal)])
    np.savez_compressed(os.path.join(HERE, "scores_fallback.npz"), **rec)
    print("wrote scores_fallback")


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from src import pnfirtau_attention as ref  # noqa: E402

    torch.set_num_threads(4)
    mha_case(ref, "c1_mha_fp32", store_w=True)
    mha_case(ref, "c1_mha_fp32_tau", tau=0.35, seed=3)
    mha_case(ref, "c1_mha_fp32_bias_modes", bias=True, gamma=0.75, mode="mass_pow", p=2.0, seed=5)
    mha_case(ref, "c1_mha_fp32_nogate", gamma=None, seed=9)
    mha_case(ref, "c1_mha_bf16", dtype=torch.bfloat16, seed=17)
    pn_gate_cases(ref)
    fir_cases(ref)
    from src import triton_pnfirtau as tri  # noqa: E402  (CPU tensors take the eager fallback)

    scores_fallback(tri)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
