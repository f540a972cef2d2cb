"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch

from oracle import pnfirtau_oracle as O


def to_np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rel_err(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def assert_close(a, b, rtol, atol, what=""):
    """Elementwise |a - b| <= atol * max|b| + rtol * |b| (atol relative to the tensor's scale)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    scale = max(np.abs(b).max(), 1e-30)
    bad = np.abs(a - b) > atol * scale + rtol * np.abs(b)
    if bad.any():
        i = np.unravel_index(np.argmax(np.abs(a - b) - rtol * np.abs(b)), a.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} elements out of tolerance; "
                             f"worst at {i}: got {a[i]!r} want {b[i]!r} (scale {scale:.3g}, "
                             f"max rel {rel_err(a, b):.3g})")


def seeded(shape, seed, dtype=torch.float32, device="cuda", scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def flash_oracle(q, k, v, tau, dO, scale, gamma, causal):
    """float64 oracle forward + backward on the exact (rounded) device inputs."""
    qn, kn, vn, dn = (to_np64(t) for t in (q, k, v, dO))
    Of, M, Z, Nm = O.flash_fwd(qn, kn, vn, tau, scale, gamma, causal)
    dq, dk, dv, dt = O.flash_bwd(qn, kn, vn, tau, dn, scale, gamma, causal)
    return Of, M, Z, Nm, dq, dk, dv, dt
