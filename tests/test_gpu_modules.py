"""GPU drop-in tests: the HIP MHA modules against the reference PnFirTauMHA golden vectors."""
import numpy as np
import pytest
import torch

import paper_01_anti_decoy_pnfirtau_amd as P
from tests.conftest import golden
from oracle import pnfirtau_oracle as O
from tests.helpers import assert_bf16_close, assert_close, assert_sum_close, to_np64
from tests.test_package_cpu import _load_mha, _t

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cls", [P.PnFirTauFlashMHA, P.PnFirTauTritonMHA])
@pytest.mark.parametrize("name", ["c1_mha_fp32", "c1_mha_fp32_tau", "c1_mha_fp32_nogate"])
def test_hip_mha_fp32_matches_reference_golden(dev, cls, name):
    """C1 in fp32: reference parity bar 1e-5 (relative to the tensor's max)."""
    print(f"[mha {cls.__name__} {name}]", flush=True)
    f = golden(name)
    m = _load_mha(cls, f).to(dev)
    x = _t(f["x"]).to(dev).requires_grad_(True)
    out = m(x)
    out.backward(_t(f["dout"]).to(dev))
    torch.cuda.synchronize()
    tol = 1e-5
    B, N, D, H, _ = [int(v) for v in f["meta"]]
    g = float(f["gamma"])
    r = O.mha_fwd_bwd(f["x"], f["w_qkv"], f["w_out"], float(f["tau"]), f["taps"], H, dout=f["dout"],
                      gamma=None if np.isnan(g) else g)
    got = {"out": out, "dx": x.grad, "dw_qkv": m.qkv.weight.grad, "dw_out": m.out.weight.grad}
    for key, t in got.items():
        assert_close(to_np64(t), r[key], tol, tol, key + " vs oracle")
        assert_close(to_np64(t), f[key], tol, tol, key + " vs reference")
    dt = float(m.score_tau.grad)
    assert_sum_close(dt, r["dtau"], r["dtau_abs"], tol, "dtau vs oracle")
    assert_sum_close(dt, float(f["dtau"]), r["dtau_abs"], tol, "dtau vs reference")


def test_flash_mha_return_weights_uses_row_path(dev):
    f = golden("c1_mha_fp32")
    m = _load_mha(P.PnFirTauFlashMHA, f).to(dev)
    out, W = m(_t(f["x"]).to(dev), return_weights=True)
    assert_close(to_np64(W), f["W"], 1e-5, 1e-5, "W")
    assert_close(to_np64(out), f["out"], 1e-5, 1e-5, "out")


@pytest.mark.parametrize("cls", [P.PnFirTauFlashMHA, P.PnFirTauTritonMHA])
def test_hip_mha_bf16_within_bf16_tolerance_of_reference(dev, cls):
    """bf16 weights/activations vs the reference's fp32 result on the same bf16-rounded data."""
    f = golden("c1_mha_fp32")
    m = _load_mha(cls, f)
    mb = _load_mha(cls, f).to(torch.bfloat16).to(dev)
    x32 = _t(f["x"]).bfloat16().float()
    ref = _load_mha(P.PnFirTauMHA, f)
    for p_, pb in zip(ref.parameters(), mb.parameters()):
        p_.data.copy_(pb.data.float().cpu())
    yr = ref(x32)
    yb = mb(_t(f["x"]).bfloat16().to(dev))
    assert_bf16_close(to_np64(yb), to_np64(yr), "out")
