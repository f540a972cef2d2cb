"""GPU parity of the HIP causal FIR against the bit-exact C oracle (oracle/fir_oracle.c)."""
import numpy as np
import pytest
import torch

from oracle import pnfirtau_oracle as O
from paper_01_anti_decoy_pnfirtau_amd import ops  # noqa: F401  (registers torch.ops.pnfx)
from tests.helpers import bf16_bits, seeded

pytestmark = pytest.mark.gpu


def _oracle_bhnc(x: torch.Tensor, taps: torch.Tensor, adjoint=False):
    """Oracle on a [B,H,N,C] (or [B,N,C]) tensor, returned as the same shape."""
    xc = x.detach().cpu().contiguous()
    shp = xc.shape
    x3 = xc.reshape(-1, shp[-2], shp[-1])
    t = taps.detach().cpu().float().numpy()
    if xc.dtype == torch.bfloat16:
        y = O.fir_contract(x3.view(torch.int16).numpy().view(np.uint16), t, adjoint)
        return y.reshape(shp)
    return O.fir_contract(x3.numpy(), t, adjoint).reshape(shp)


def _per_head_taps(H, K, seed):
    g = torch.Generator().manual_seed(seed)
    t = torch.rand(H, K, generator=g)
    return (t / t.sum(-1, keepdim=True)).float()


@pytest.mark.parametrize("adjoint", [False, True])
def test_fir_config2_full_size_bit_exact(dev, adjoint):
    """C2: K [8,8,2048,64] bf16 ~ N(0,1), 7 per-head taps ~ U(0,1) normalised."""
    print(f"[fir c2 adjoint={adjoint}]", flush=True)
    x = seeded((8, 8, 2048, 64), 0, torch.bfloat16, dev)
    taps = _per_head_taps(8, 7, 1).to(dev)
    fn = torch.ops.pnfx.fir_bwd if adjoint else torch.ops.pnfx.fir_fwd
    y = fn(x, taps)
    torch.cuda.synchronize()
    ref = _oracle_bhnc(x.cpu().view(64, 2048, 64), taps.cpu().repeat(8, 1), adjoint)
    assert np.array_equal(bf16_bits(y).reshape(64, 2048, 64), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [1, 5, 7, 33, 130])
def test_fir_mha_layout_strided_view_bit_exact(dev, dtype, N):
    """The reference call site: k_raw is a [B,N,C] column block of the qkv GEMM output."""
    print(f"[fir mha N={N} {dtype}]", flush=True)
    B, C = 3, 64
    qkv = seeded((B, N, 3 * C), 2, dtype, dev)
    k_raw = qkv[..., C:2 * C]
    taps = torch.tensor(O.causal_gaussian_taps(7))
    from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import hip_causal_fir
    y = hip_causal_fir(k_raw, taps.to(dev))
    assert y.shape == (B, N, C) and y.is_contiguous()
    ref = _oracle_bhnc(k_raw.contiguous(), taps)
    got = bf16_bits(y) if dtype == torch.bfloat16 else y.cpu().numpy()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("K", [3, 5, 16])
@pytest.mark.parametrize("C", [64, 13])
def test_fir_general_taps_and_channels(dev, K, C):
    print(f"[fir K={K} C={C}]", flush=True)
    x = seeded((2, 3, 100, C), 3, torch.bfloat16, dev)
    taps = _per_head_taps(3, K, 4).to(dev)
    y = torch.ops.pnfx.fir_fwd(x, taps)
    gy = torch.ops.pnfx.fir_bwd(x, taps)
    xr = x.cpu().reshape(6, 100, C)
    tr = taps.cpu().repeat(2, 1)
    assert np.array_equal(bf16_bits(y).reshape(6, 100, C), _oracle_bhnc(xr, tr))
    assert np.array_equal(bf16_bits(gy).reshape(6, 100, C), _oracle_bhnc(xr, tr, True))


def test_fir_autograd_is_the_adjoint(dev):
    x = seeded((2, 50, 32), 5, torch.float32, dev).requires_grad_(True)
    taps = torch.tensor(O.causal_gaussian_taps(7)).to(dev)
    from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import hip_causal_fir
    y = hip_causal_fir(x, taps)
    g = seeded((2, 50, 32), 6, torch.float32, dev)
    y.backward(g)
    ref = O.fir_contract(g.cpu().numpy(), taps.cpu().numpy(), adjoint=True)
    assert np.array_equal(x.grad.cpu().numpy(), ref)
    lhs = float((y.detach().double() * g.double()).sum())
    rhs = float((x.detach().double() * x.grad.double()).sum())
    assert abs(lhs - rhs) < 1e-4 * max(1.0, abs(lhs))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [1, 6, 9, 37, 130])
def test_fir_adjoint_short_and_ragged_sequences_bit_exact(dev, dtype, N):
    """The 7-tap adjoint where runs of 8 rows straddle both ends of the sequence (the kernel's
    range-tested path) as well as the interior."""
    print(f"[fir adjoint N={N} {dtype}]", flush=True)
    x = seeded((2, 3, N, 64), 9, dtype, dev)
    taps = _per_head_taps(3, 7, 11).to(dev)
    gy = torch.ops.pnfx.fir_bwd(x, taps)
    ref = _oracle_bhnc(x.cpu().reshape(6, N, 64), taps.cpu().repeat(2, 1), True)
    got = bf16_bits(gy) if dtype == torch.bfloat16 else gy.cpu().numpy()
    assert np.array_equal(got.reshape(6, N, 64), ref)


@pytest.mark.parametrize("adjoint", [False, True])
def test_fir_many_slices_take_the_element_kernel_bit_exact(dev, adjoint):
    """More than 65535 (b, h) slices do not fit the vector kernel's second grid dimension:
    the element-per-thread kernel takes them, bit-exact all the same."""
    print(f"[fir 65600 slices adjoint={adjoint}]", flush=True)
    x = seeded((65600, 9, 8), 4, torch.bfloat16, dev)
    taps = torch.tensor(O.causal_gaussian_taps(7)).to(dev)
    fn = torch.ops.pnfx.fir_bwd if adjoint else torch.ops.pnfx.fir_fwd
    y = fn(x, taps)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(y), _oracle_bhnc(x, taps.cpu(), adjoint))
