"""Empty inputs through the drop-in surface on the GPU.

The reference's Triton wrappers launch empty grids for N = 0 or B = 0 and return empty
results (src/triton_pnfirtau.py:629-691, 788-811, 814-983: every grid dimension is a
multiple of B, N or B*H); dtau is the sum over no scores, 0.  The HIP path gives the same
shapes and values without calling into libpnfx.so (whose entry points require N >= 1).
"""
import pytest
import torch

import paper_01_anti_decoy_pnfirtau_amd as P
from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import (flash_pn_fir_tau_attention,
                                                           hip_causal_fir, hip_pn_fir_tau_scores)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 2, 0, 64), (0, 2, 64, 64), (1, 0, 32, 128)])
def test_flash_empty_inputs(dev, dtype, shape):
    print(f"[empty flash {shape} {dtype}]", flush=True)
    q, k, v = (torch.zeros(shape, device=dev, dtype=dtype, requires_grad=True) for _ in range(3))
    tau = torch.tensor(0.25, device=dev, requires_grad=True)
    o = flash_pn_fir_tau_attention(q, k, v, tau)
    assert o.shape == shape and o.dtype == dtype
    o.backward(torch.zeros_like(o))
    torch.cuda.synchronize()
    for t in (q, k, v):
        assert t.grad.shape == shape
    assert tau.grad.item() == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fir_and_rows_empty_inputs(dev, dtype):
    print(f"[empty fir/rows {dtype}]", flush=True)
    taps = P.causal_gaussian_taps(7, device=dev)
    x = torch.zeros((2, 0, 64), device=dev, dtype=dtype, requires_grad=True)
    y = hip_causal_fir(x, taps)
    assert y.shape == (2, 0, 64)
    y.sum().backward()
    assert x.grad.shape == x.shape
    raw = torch.zeros((2, 3, 0, 0), device=dev, dtype=dtype, requires_grad=True)
    tau = torch.tensor(0.1, device=dev, requires_grad=True)
    w = hip_pn_fir_tau_scores(raw, tau)
    assert w.shape == raw.shape
    w.sum().backward()
    torch.cuda.synchronize()
    assert raw.grad.shape == raw.shape and tau.grad.item() == 0.0


@pytest.mark.parametrize("cls", [P.PnFirTauFlashMHA, P.PnFirTauTritonMHA])
def test_mha_empty_sequence(dev, cls):
    """A [B, 0, D] batch through the HIP modules gives [B, 0, D] and zero gradients, as the
    eager reference module does."""
    print(f"[empty mha {cls.__name__}]", flush=True)
    torch.manual_seed(0)
    m = cls(P.PnFirConfig(d_model=64, n_heads=4)).to(dev)
    x = torch.zeros((2, 0, 64), device=dev, requires_grad=True)
    out = m(x)
    assert out.shape == (2, 0, 64)
    out.sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape
    for name, prm in m.named_parameters():
        assert prm.grad is None or float(prm.grad.abs().sum()) == 0.0, name
