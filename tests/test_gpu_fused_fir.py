"""The flash forward with the causal key FIR fused into its key-tile load (pnfx_flash_fwd_fir)
against the two-launch path it replaces (src/pnfirtau_attention.py:299-315: the FIR, then the
flash forward): O, its bf16 residual, M, Z and the tile mask must agree bit for bit, since the
fused kernel filters each key tile with the FIR kernel's own arithmetic."""
import pytest
import torch

from paper_01_anti_decoy_pnfirtau_amd import ops
from paper_01_anti_decoy_pnfirtau_amd.pnfirtau_attention import causal_gaussian_taps
from tests.helpers import seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,H,N,tau,causal,K,per_head,scale", [
    (1, 2, 200, 0.0, True, 7, False, 0.125),
    (2, 3, 1024, 0.3, True, 7, True, 0.125),
    (1, 2, 130, -0.2, False, 7, False, 0.125),
    (1, 1, 640, 0.1, True, 5, False, 0.1),
    (1, 2, 64, 0.0, True, 3, True, 0.125),
    (1, 1, 7, 0.0, True, 7, False, 0.125),
])
def test_fused_fir_forward_is_bitwise_fir_then_flash(dev, B, H, N, tau, causal, K, per_head, scale):
    D = 64
    q, kraw, v = (seeded((B, H, N, D), s, torch.bfloat16, dev) for s in (11, 12, 13))
    if per_head:
        t = torch.rand(H, K, generator=torch.Generator().manual_seed(14))
        taps = (t / t.sum(-1, keepdim=True)).to(dev)
    else:
        taps = causal_gaussian_taps(K).to(dev)
    t32 = torch.tensor(tau, device=dev)
    k = torch.ops.pnfx.fir_fwd(kraw, taps)
    o, o_lo, M, Z, _, mask = torch.ops.pnfx.flash_fwd(q, k, v, t32, scale, 0.5, True, causal,
                                                       False, False)
    fo, flo, fM, fZ, fmask = ops.flash_fwd_fused_fir(q, kraw, v, t32, taps, scale, 0.5, True, causal)
    torch.cuda.synchronize()
    for name, a, b in (("O", fo, o), ("O_lo", flo, o_lo), ("M", fM, M), ("Z", fZ, Z),
                       ("mask", fmask, mask)):
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.uint8) if b.dtype == torch.bfloat16 else b), name


def test_fused_fir_forward_reads_a_strided_key_view(dev):
    """k_raw as the key slice of a packed qkv projection output ([B, N, 3, H, d])."""
    B, H, N, D = 1, 4, 300, 64
    qkv = seeded((B, N, 3, H, D), 21, torch.bfloat16, dev)
    q, kraw, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    taps = causal_gaussian_taps(7).to(dev)
    t32 = torch.tensor(0.05, device=dev)
    k = torch.ops.pnfx.fir_fwd(kraw.contiguous(), taps)
    o, _, M, _, _, _ = torch.ops.pnfx.flash_fwd(q.contiguous(), k, v.contiguous(), t32, 0.125, 0.5,
                                                True, True, False, False)
    fo, _, fM, _, _ = ops.flash_fwd_fused_fir(q, kraw, v, t32, taps, 0.125, 0.5, True, True)
    torch.cuda.synchronize()
    assert torch.equal(fo.view(torch.uint8), o.view(torch.uint8)) and torch.equal(fM, M)
