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


BF16_RTOL, BF16_ATOL = 2e-2, 2e-3
F32_TOL = 1e-5


def assert_bf16_close(a, b, what=""):
    """bf16 parity bar: max|a-b| <= 2e-2 max|b| and mean|a-b| <= 2e-3 max|b|.

    Both bounds are taken relative to the tensor's scale: in bf16 the error of a
    gradient element is set by the largest terms of its sum (operands rounded to
    8 mantissa bits), not by the element's own magnitude.
    """
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    scale = max(np.abs(b).max(), 1e-30)
    err = np.abs(a - b)
    if err.max() > BF16_RTOL * scale or err.mean() > BF16_ATOL * scale:
        i = np.unravel_index(np.argmax(err), a.shape)
        raise AssertionError(f"{what}: max err {err.max() / scale:.3g}, mean err "
                             f"{err.mean() / scale:.3g} of scale {scale:.3g}; worst at {i}: "
                             f"got {a[i]!r} want {b[i]!r}")


def assert_sum_close(got, want, abs_sum, tol, what=""):
    """A scalar that is a sum with cancellation: |got - want| <= tol * (|want| + sum|terms|)."""
    assert abs(got - want) <= tol * (abs(want) + abs_sum), (what, got, want, abs_sum)


def seeded(shape, seed, dtype=torch.float32, device="cuda", scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def flash_oracle(q, k, v, tau, dO, scale, gamma, causal):
    """float64 oracle forward + backward on the exact (rounded) device inputs."""
    qn, kn, vn, dn = (to_np64(t) for t in (q, k, v, dO))
    Of, M, Z, Nm = O.flash_fwd(qn, kn, vn, tau, scale, gamma, causal)
    dq, dk, dv, dt, dabs = O.flash_bwd(qn, kn, vn, tau, dn, scale, gamma, causal, return_abs=True)
    return Of, M, Z, Nm, dq, dk, dv, dt, dabs
