"""GPU parity of the row-fused score kernels against the oracle (src/triton_pnfirtau.py:141-303)."""
import numpy as np
import pytest
import torch

from oracle import pnfirtau_oracle as O
from paper_01_anti_decoy_pnfirtau_amd import ops  # noqa: F401  (registers torch.ops.pnfx)
from tests.helpers import BF16_ATOL, F32_TOL, assert_bf16_close, assert_close, seeded, to_np64

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,causal,p,gamma", [(24, True, 10.0, 0.5), (130, True, 10.0, 0.5),
                                              (64, False, 2.0, None), (50, True, 3.5, 0.75),
                                              (512, True, 10.0, 0.5), (5000, True, 10.0, 0.5)])
def test_rows_fwd_bwd_match_oracle(dev, dtype, N, causal, p, gamma):
    print(f"[rows N={N} causal={causal} p={p} gamma={gamma} {dtype}]", flush=True)
    B, H = (2, 2) if N < 1000 else (1, 1)
    raw = seeded((B, H, N, N), 10, dtype, dev, scale=3.0)
    if N >= 24:
        raw[0, 0, 20, :5] = raw[0, 0, 20, 7]  # planted tie at the row peak candidates
    tau = torch.tensor(0.3, device=dev, requires_grad=True)
    scale = 0.25
    rawg = raw.clone().requires_grad_(True)
    from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import hip_pn_fir_tau_scores
    w = hip_pn_fir_tau_scores(rawg, tau, scale=scale, p=p, gamma=gamma, causal_mask=causal)
    dW = seeded(w.shape, 11, dtype, dev)
    w.backward(dW)
    torch.cuda.synchronize()
    rn = to_np64(raw)
    W, M, Z, Nm = O.pn_rows_fwd(rn, 0.3, scale, p, gamma, causal)
    d_raw, dtr = O.pn_rows_bwd(to_np64(dW), rn, 0.3, M, Z, Nm, scale, p, gamma, causal)
    if dtype == torch.float32:  # fp32 bar: 1e-5 (rtol, and atol of the tensor's scale)
        assert_close(to_np64(w), W, F32_TOL, F32_TOL, "W")
        assert_close(to_np64(rawg.grad), d_raw, F32_TOL, F32_TOL, "d_raw")
        tol = F32_TOL
    else:
        assert_bf16_close(to_np64(w), W, "W")
        assert_bf16_close(to_np64(rawg.grad), d_raw, "d_raw")
        tol = BF16_ATOL
    assert abs(float(tau.grad) - dtr.sum()) <= tol * max(1.0, np.abs(dtr).sum())


def test_rows_stats_and_silent_rows(dev):
    raw = seeded((1, 1, 40, 40), 12, torch.float32, dev)
    raw[0, 0, 10] = -5.0  # silent row
    raw[0, 0, 30, :4] = 3.0  # four-way tie at the peak
    tau = torch.tensor(0.1, device=dev)
    w, M, Z, Nm = torch.ops.pnfx.pn_rows_fwd(raw, tau, 1.0, 10.0, 0.5, True, True)
    Wo, Mo, Zo, No = O.pn_rows_fwd(to_np64(raw), 0.1, 1.0, 10.0, 0.5, True)
    assert np.array_equal(Nm.cpu().numpy(), No.reshape(-1))
    assert float(M[10]) == 0.0 and float(Z[10]) == pytest.approx(1e-12) and int(Nm[10]) == 0
    assert int(Nm[30]) == 4
    assert torch.all(w[0, 0, 10] == 0)
    np.testing.assert_allclose(M.cpu().numpy(), Mo.reshape(-1), rtol=1e-6)
    np.testing.assert_allclose(Z.cpu().numpy(), Zo.reshape(-1), rtol=1e-5)
    # row sums equal gate * mass / (mass + 1e-12), i.e. the gate unless the mass is tiny
    np.testing.assert_allclose(w.sum(-1).cpu().numpy().reshape(-1), Wo.sum(-1).reshape(-1), rtol=1e-5, atol=1e-7)


def test_rows_of_length_one_and_many_rows(dev):
    """Score rows of one key (the row's only score is its peak) and a tall stack of short rows."""
    for shape in ((3, 5, 1, 1), (20000, 3, 3)):
        raw = torch.randn(shape, device=dev).to(torch.bfloat16)
        print(f"[rows {tuple(raw.shape)}]", flush=True)
        tau = torch.tensor(0.1, device=dev)
        w, M, Z, Nm = torch.ops.pnfx.pn_rows_fwd(raw, tau, 0.5, 10.0, 0.5, True, False)
        s = raw.float() * 0.5 - 0.1
        u = s.clamp_min(0)
        P = (u ** 10)
        m = u.amax(-1, keepdim=True)
        g = torch.where(m > 0, m / (m + 0.5), torch.zeros_like(m))
        ref = P / (P.sum(-1, keepdim=True) + 1e-12) * g
        torch.testing.assert_close(w.float(), ref, rtol=2e-2, atol=2e-3)
