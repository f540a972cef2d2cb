"""Shared helpers for the GPU parity tests."""
import os

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

# Every bf16 comparison is recorded here (test, tensor, worst ratios, scale); the session
# hook in conftest.py writes the list to $PNFX_PARITY_REPORT when that is set.
PARITY_LOG = []


def _test_name() -> str:
    return os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]


def bf16_ratios(a, b):
    """Worst elementwise ratios of |a - b| to the bf16 bar, and the tensor's scale s = max|b|:
    scaled  = max |a-b| / (2e-3 s + 2e-2 |b|)   (atol taken relative to the tensor's scale),
    literal = max |a-b| / (2e-3   + 2e-2 |b|)   (atol as an absolute 2e-3)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    s = max(float(np.abs(b).max()) if b.size else 0.0, 1e-30)
    err = np.abs(a - b)
    if not err.size:
        return 0.0, 0.0, s
    return (float((err / (BF16_ATOL * s + BF16_RTOL * np.abs(b))).max()),
            float((err / (BF16_ATOL + BF16_RTOL * np.abs(b))).max()), s)


def assert_bf16_close(a, b, what="", ref_rounding=None):
    """bf16 parity bar, elementwise: |a - b| <= 2e-3 max|b| + 2e-2 |b| for every element.

    rtol 2e-2 applies to each element; atol 2e-3 is taken relative to the tensor's scale,
    because in bf16 the error of an element of a sum (a gradient, an attention output) is set
    by the magnitude of the sum's largest terms (its operands carry 8 mantissa bits), not by
    the element's own size.  Both this ratio and the one with an absolute atol of 2e-3 are
    recorded (PARITY_LOG).

    ``ref_rounding``: the same tensor formed with the reference kernels' bf16 rounding points
    (oracle.flash_reference_bf16).  Rounding dS to bf16 before the dQ and dK products, as the
    reference does, puts the odd element of a gradient slightly past 2e-3 max|b|; the bar is
    then the larger of 1 and 1.25x the reference-rounding result's own worst ratio, and both
    ratios are recorded.
    """
    scaled, literal, s = bf16_ratios(a, b)
    entry = {"test": _test_name(), "what": what, "scaled_ratio": scaled,
             "literal_ratio": literal, "scale": s}
    bound = 1.0
    if ref_rounding is not None:
        rs, rl, _ = bf16_ratios(ref_rounding, b)
        entry.update(reference_rounding_scaled_ratio=rs, reference_rounding_literal_ratio=rl)
        bound = max(1.0, 1.25 * rs)
    PARITY_LOG.append(entry)
    if scaled > bound:
        a = np.asarray(a, dtype=np.float64)
        b = np.asarray(b, dtype=np.float64)
        r = np.abs(a - b) / (BF16_ATOL * s + BF16_RTOL * np.abs(b))
        i = np.unravel_index(np.argmax(r), a.shape)
        raise AssertionError(f"{what}: {(r > bound).sum()} / {r.size} elements past the bar "
                             f"({bound:.3g}); worst ratio {scaled:.3g} at {i}: got {a[i]!r} "
                             f"want {b[i]!r} (scale {s:.3g})")


def assert_sum_close(got, want, abs_sum, tol, what=""):
    """A scalar that is a sum with cancellation: |got - want| <= tol * (|want| + sum|terms|)."""
    PARITY_LOG.append({"test": _test_name(), "what": what, "abs_err": abs(got - want),
                       "want": want, "sum_abs_terms": abs_sum,
                       "ratio": abs(got - want) / max(tol * (abs(want) + abs_sum), 1e-300),
                       "literal_ratio": abs(got - want) / (BF16_ATOL + BF16_RTOL * abs(want))})
    assert abs(got - want) <= tol * (abs(want) + abs_sum), (what, got, want, abs_sum)


def flash_reference_rounding(q, k, v, tau, dO, scale, gamma, causal):
    """{"O", "dq", "dk", "dv"} as the reference's bf16 kernels would round them, float64
    otherwise, on the exact (rounded) device inputs; empty for fp32 inputs."""
    if q.dtype != torch.bfloat16:
        return {}
    Of, dq, dk, dv, _ = O.flash_reference_bf16(*(to_np64(t) for t in (q, k, v)), tau,
                                               to_np64(dO), scale, gamma, causal)
    return {"O": Of, "dq": dq, "dk": dk, "dv": dv}


def seeded(shape, seed, dtype=torch.float32, device="cuda", scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(device)


def flash_oracle(q, k, v, tau, dO, scale, gamma, causal):
    """float64 oracle forward + backward on the exact (rounded) device inputs."""
    qn, kn, vn, dn = (to_np64(t) for t in (q, k, v, dO))
    Of, M, Z, Nm = O.flash_fwd(qn, kn, vn, tau, scale, gamma, causal)
    dq, dk, dv, dt, dabs = O.flash_bwd(qn, kn, vn, tau, dn, scale, gamma, causal, return_abs=True)
    return Of, M, Z, Nm, dq, dk, dv, dt, dabs
