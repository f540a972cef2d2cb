"""The flash forward with the causal key FIR fused into its key-tile load (pnfx_flash_fwd_fir).

Against the float64 oracle: the FIR contract of oracle/fir_oracle.c applied to the raw keys,
then the flash forward semantics (src/pnfirtau_attention.py:299-315: the FIR, then
src/triton_pnfirtau.py:313-443), at the bf16 bar for O, 1e-5 for M, the fp32 sum for Z, and
the exact 64x64 tile mask.  Against the two-launch HIP path it replaces: O, its bf16
residual, M, Z and the tile mask bit for bit, since the fused kernel filters each key tile
with the FIR kernel's own arithmetic."""
import numpy as np
import pytest
import torch

from oracle import pnfirtau_oracle as O
from paper_01_anti_decoy_pnfirtau_amd import ops
from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import tile_mask_64
from paper_01_anti_decoy_pnfirtau_amd.pnfirtau_attention import causal_gaussian_taps
from tests.helpers import assert_bf16_close, assert_close, seeded, to_np64

pytestmark = pytest.mark.gpu


CASES = [
    # B, H, N, D, tau, causal, K, per_head, scale
    (1, 2, 200, 64, 0.0, True, 7, False, 0.125),
    (2, 3, 1024, 64, 0.3, True, 7, True, 0.125),
    (1, 2, 130, 64, -0.2, False, 7, False, 0.125),
    (1, 1, 640, 64, 0.1, True, 5, False, 0.1),
    (1, 2, 64, 64, 0.0, True, 3, True, 0.125),
    (1, 1, 7, 64, 0.0, True, 7, False, 0.125),
    (2, 4, 300, 16, 0.0, True, 7, False, 0.25),
    (1, 4, 1000, 16, 0.4, True, 7, True, 0.25),
    (1, 2, 77, 16, -0.1, False, 7, False, 0.3),
    (2, 2, 500, 32, 0.0, True, 7, True, 32 ** -0.5),
    (1, 3, 130, 32, 0.2, False, 5, False, 32 ** -0.5),
]


def _inputs(dev, B, H, N, D, K, per_head):
    q, kraw, v = (seeded((B, H, N, D), s, torch.bfloat16, dev) for s in (11, 12, 13))
    if per_head:
        t = torch.rand(H, K, generator=torch.Generator().manual_seed(14))
        taps = (t / t.sum(-1, keepdim=True)).to(dev)
    else:
        taps = causal_gaussian_taps(K).to(dev)
    return q, kraw, v, taps


def _fir_oracle(kraw, taps):
    """The filtered keys, float64, from the bit-exact FIR contract of oracle/fir_oracle.c."""
    B, H, N, D = kraw.shape
    bits = kraw.detach().cpu().contiguous().reshape(B * H, N, D).view(torch.int16).numpy()
    out = O.fir_contract(bits.view(np.uint16), taps.detach().cpu().numpy())
    return O.bf16_bits_to_f32(out).astype(np.float64).reshape(B, H, N, D)


def _check_against_oracle(fo, fM, fZ, fmask, q, kf, v, tau, scale, causal, slices, what):
    qn, vn = to_np64(q), to_np64(v)
    m64 = tile_mask_64(fmask).cpu().numpy().astype(bool)
    nb = m64.shape[-1]
    for b, h in slices:
        Of, Mo, Zo, _ = O.flash_fwd(qn[b, h], kf[b, h], vn[b, h], tau, scale, 0.5, causal)
        em = O.flash_reference_bf16(qn[b, h], kf[b, h], vn[b, h], tau, np.zeros_like(Of), scale,
                                    0.5, causal)[0]
        assert_bf16_close(to_np64(fo[b, h]), Of, f"{what} O", em)
        assert_close(to_np64(fM[b, h]), Mo, 1e-5, 1e-5, f"{what} M")
        assert_close(to_np64(fZ[b, h]), Zo, 1e-4, 0.0, f"{what} Z")
        act, amb = O.tile_activity(qn[b, h], kf[b, h], tau, scale, causal)
        got = m64[b * fM.shape[1] + h].reshape(nb, nb)
        assert np.array_equal(got[~amb], act[~amb]), f"{what} tile mask"


@pytest.mark.parametrize("B,H,N,D,tau,causal,K,per_head,scale", CASES)
def test_fused_fir_forward_matches_oracle(dev, B, H, N, D, tau, causal, K, per_head, scale):
    print(f"[fused fir oracle B={B} H={H} N={N} D={D} tau={tau} K={K}]", flush=True)
    q, kraw, v, taps = _inputs(dev, B, H, N, D, K, per_head)
    t32 = torch.tensor(tau, device=dev)
    fo, _, fM, fZ, fmask = ops.flash_fwd_fused_fir(q, kraw, v, t32, taps, scale, 0.5, True, causal)
    torch.cuda.synchronize()
    slices = [(b, h) for b in range(B) for h in range(H)]
    _check_against_oracle(fo, fM, fZ, fmask, q, _fir_oracle(kraw, taps), v, tau, scale, causal,
                          slices, "fused")


def test_fused_fir_forward_full_c4_slice_matches_oracle(dev):
    """C4's shape (B=4, H=16, N=8192, d=64) with the reference's shared Gaussian taps, raw
    keys in: one (b, h) slice of the whole launch against the oracle."""
    print("[fused fir C4 slice]", flush=True)
    B, H, N, D = 4, 16, 8192, 64
    g = torch.Generator().manual_seed(31)
    q, kraw, v = [torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
    taps = causal_gaussian_taps(7).to(dev)
    t32 = torch.tensor(0.0, device=dev)
    fo, _, fM, fZ, fmask = ops.flash_fwd_fused_fir(q, kraw, v, t32, taps, 0.125, 0.5, True, True)
    torch.cuda.synchronize()
    b, h = 2, 11
    kf = _fir_oracle(kraw[b:b + 1, h:h + 1], taps)
    sub = lambda t: t[b:b + 1, h:h + 1]  # noqa: E731
    _check_against_oracle(sub(fo), sub(fM), sub(fZ), fmask[b * H + h:b * H + h + 1], sub(q), kf,
                          sub(v), 0.0, 0.125, True, [(0, 0)], "fused C4")


@pytest.mark.parametrize("B,H,N,D,tau,causal,K,per_head,scale", CASES)
def test_fused_fir_forward_is_bitwise_fir_then_flash(dev, B, H, N, D, tau, causal, K, per_head,
                                                     scale):
    q, kraw, v, taps = _inputs(dev, B, H, N, D, K, per_head)
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


def test_module_inference_takes_the_fused_route_bitwise(dev, monkeypatch):
    """PnFirTauFlashMHA under no_grad at a short sequence runs the fused forward
    (hip_pnfirtau.fused_fir_flash_forward) and gives bitwise the output of its two-launch path
    (FIR, then flash: src/pnfirtau_attention.py:299-315); with gradients it keeps the two
    launches; past FUSED_FIR_MAX_N it keeps them too."""
    from paper_01_anti_decoy_pnfirtau_amd import PnFirConfig, PnFirTauFlashMHA, hip_pnfirtau

    calls = []
    real = hip_pnfirtau.fused_fir_flash_forward

    def spy(*a, **k):
        calls.append(a[0].shape)
        return real(*a, **k)

    monkeypatch.setattr(hip_pnfirtau, "fused_fir_flash_forward", spy)
    torch.manual_seed(0)
    m = PnFirTauFlashMHA(PnFirConfig(d_model=64, n_heads=4)).to(dev)
    with torch.no_grad():
        m.score_tau.fill_(0.05)
    x = torch.randn(4, 256, 64, device=dev)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        monkeypatch.setattr(hip_pnfirtau, "FUSED_FIR_INFERENCE", True)
        a = m(x)
        assert len(calls) == 1
        monkeypatch.setattr(hip_pnfirtau, "FUSED_FIR_INFERENCE", False)
        b = m(x)
        assert len(calls) == 1
    assert torch.equal(a, b)
    monkeypatch.setattr(hip_pnfirtau, "FUSED_FIR_INFERENCE", True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        c = m(x.requires_grad_(True))
    assert len(calls) == 1 and torch.equal(c.detach(), a)
    long_x = torch.randn(1, hip_pnfirtau.FUSED_FIR_MAX_N + 1, 64, device=dev)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        m(long_x)
    assert len(calls) == 1


def _random_fused_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rng.choice([16, 32, 64]))
        per_head = bool(rng.random() < 0.5)
        # shared taps are the reference's Gaussian ones, defined for odd lengths only
        K = int(rng.integers(1, 8)) if per_head else int(rng.choice([1, 3, 5, 7]))
        out.append((int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 700)), D,
                    float(np.round(rng.uniform(-0.3, 0.4), 3)), bool(rng.random() < 0.75),
                    K, per_head,
                    float(rng.choice([D ** -0.5, np.round(rng.uniform(0.05, 0.35), 4)]))))
    return out


@pytest.mark.parametrize("seed", [5, 6, 7, 8])
def test_fused_fir_forward_random_sweep(dev, seed):
    """Seeded random shapes (d 16/32/64, N 1..699, K 1..7, shared or per-head taps, tau of
    either sign, causal or not, power-of-two or arbitrary scale), each against the oracle and
    bitwise against the two launches it replaces."""
    for case in _random_fused_cases(30, seed):
        B, H, N, D, tau, causal, K, per_head, scale = case
        print(f"[fused fir random {case}]", flush=True)
        q, kraw, v, taps = _inputs(dev, B, H, N, D, K, per_head)
        t32 = torch.tensor(tau, device=dev)
        fo, flo, fM, fZ, fmask = ops.flash_fwd_fused_fir(q, kraw, v, t32, taps, scale, 0.5, True,
                                                         causal)
        k = torch.ops.pnfx.fir_fwd(kraw, taps)
        o, o_lo, M, Z, _, mask = torch.ops.pnfx.flash_fwd(q, k, v, t32, scale, 0.5, True, causal,
                                                           False, False)
        torch.cuda.synchronize()
        for name, a, b in (("O", fo, o), ("O_lo", flo, o_lo), ("M", fM, M), ("Z", fZ, Z),
                           ("mask", fmask, mask)):
            assert torch.equal(a.view(torch.uint8) if a.dtype == torch.bfloat16 else a,
                               b.view(torch.uint8) if b.dtype == torch.bfloat16 else b), name
        slices = [(b, h) for b in range(B) for h in range(H)]
        _check_against_oracle(fo, fM, fZ, fmask, q, _fir_oracle(kraw, taps), v, tau, scale,
                              causal, slices, "fused random")
