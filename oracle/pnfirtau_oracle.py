"""CPU oracle for the pn_fir_tau hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed CPU
baseline), never as something the product path calls.  The product path
(``paper_01_anti_decoy_pnfirtau_amd``) does not import it.

It is a numpy restatement of the reference algorithm, written from the
reference's semantics (file:line citations on each function, relative to the
reference repository root):

* ``causal_gaussian_taps``      src/pnfirtau_attention.py:50-62
* ``fir``                        src/pnfirtau_attention.py:65-74 (math),
                                 src/triton_pnfirtau.py:40-135 (fp32-tap contract;
                                 bit-exact contract lives in ``fir_oracle.c``)
* ``power_norm_peak_gate`` (+bwd) src/pnfirtau_attention.py:87-119
* ``pn_rows_fwd`` / ``pn_rows_bwd`` src/triton_pnfirtau.py:141-303, 694-811
* ``flash_fwd`` / ``flash_bwd``   src/triton_pnfirtau.py:313-621, 814-983
* ``flash_reference_bf16``       the same, with the reference kernels' bf16 rounding points
* ``mha_fwd_bwd``               src/pnfirtau_attention.py:195-247 (PnFirTauMHA)
* ``tile_activity``             experiments/exp4b_mha6_instrumentation.py:80-128

All arithmetic defaults to float64 so that the oracle is a tighter reference
than either the reference GPU path or the HIP path; ``dtype=np.float32`` gives
the same algorithm in single precision (used for the CPU baseline timing).

How each function is pinned (tests/test_oracle.py): taps against the fp32
vector the reference stored in results/exp1_legacy_13stacks.json:29; the FIR
against an impulse response, ``np.convolve`` and the adjoint identity; the
power-norm gate against closed forms (row sum == gate, silent rows),
finite differences and the golden vectors written by
tests/golden/make_golden.py from the reference itself; flash against the
dense composition, the flash identity D = <dO,O>/g and special cases
(N == 1, tau -> +inf, single active key).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

EPS_Z = 1e-12  # src/triton_pnfirtau.py:200, :422; src/pnfirtau_attention.py:107
MASK_FILL = -1e4  # src/pnfirtau_attention.py:237

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_fir.so")
_lib = None


# --------------------------------------------------------------------------
# taps
# --------------------------------------------------------------------------
def causal_gaussian_taps(k: int, sigma_frac: float = 3.0) -> np.ndarray:
    """Half-Gaussian causal taps [k], float32, index k-1 = lag 0 (present).

    Follows src/pnfirtau_attention.py:50-62: dist = (k-1) - t,
    sigma = max((k-1)/sigma_frac, 0.5), w = exp(-0.5 (dist/sigma)^2) / sum(w),
    all in float32.  The exponential is evaluated in float64 and rounded once
    (a correctly rounded expf); the sum is a float32 left-to-right sum and the
    division is float32, which reproduces the reference's stored fp32 vector.
    """
    assert k % 2 == 1 and k >= 1
    sigma = max((k - 1) / sigma_frac, 0.5)
    dist = np.float32(k - 1) - np.arange(k, dtype=np.float32)
    arg = np.float32(-0.5) * (dist / np.float32(sigma)) ** 2  # exact for these small ints
    w = np.exp(arg.astype(np.float64)).astype(np.float32)
    s = np.float32(0.0)
    for v in w:
        s = np.float32(s + v)
    return (w / s).astype(np.float32)


# --------------------------------------------------------------------------
# FIR
# --------------------------------------------------------------------------
def fir(x: np.ndarray, taps: np.ndarray, adjoint: bool = False, per_head: bool = False) -> np.ndarray:
    """Causal depthwise FIR along axis -2 (sequence) in float64.

    x: [..., N, C].  taps: [K] (shared) or [H, K] with per_head=True, where x is
    [B, H, N, C].  y[n] = sum_u h_u x[n-u] with h_u = taps[K-1-u] and x[m<0] = 0
    (src/pnfirtau_attention.py:9-14, :65-74).  adjoint=True applies the
    transpose: gx[n] = sum_u h_u gy[n+u], gy[m>=N] = 0
    (src/triton_pnfirtau.py:89-135).
    """
    x = np.asarray(x, dtype=np.float64)
    taps = np.asarray(taps, dtype=np.float64)
    N = x.shape[-2]
    K = taps.shape[-1]
    y = np.zeros_like(x)
    for u in range(K):
        h = taps[..., K - 1 - u]
        if per_head:
            assert x.ndim == 4 and taps.ndim == 2 and taps.shape[0] == x.shape[1]
            h = h.reshape(1, -1, 1, 1)
        if u >= N:
            break
        if not adjoint:
            y[..., u:, :] += h * x[..., : N - u, :]
        else:
            y[..., : N - u, :] += h * x[..., u:, :]
    return y


def _load_lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build_lib()
        lib = ctypes.CDLL(_LIB_PATH)
        i64, i32 = ctypes.c_int64, ctypes.c_int
        vp = ctypes.c_void_p
        for name in ("oracle_fir_f32", "oracle_fir_bf16"):
            fn = getattr(lib, name)
            fn.argtypes = [vp, vp, i64, i64, i64, vp, i64, i32, i32]
            fn.restype = None
        _lib = lib
    return _lib


def build_lib() -> str:
    """Compile fir_oracle.c into oracle/liboracle_fir.so with gcc."""
    src = os.path.join(_HERE, "fir_oracle.c")
    tmp = _LIB_PATH + ".tmp%d" % os.getpid()
    subprocess.check_call(
        ["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-o", tmp, src, "-lm"]
    )
    os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


def fir_contract(x: np.ndarray, taps: np.ndarray, adjoint: bool = False) -> np.ndarray:
    """Bit-exact fp32-tap FIR contract (see fir_oracle.c) over [BH, N, C].

    x: float32 array, or uint16 array holding bf16 bit patterns.  taps: float32
    [K] or [G, K]; slice bh uses tap row bh % G.  Returns the same dtype as x.
    """
    lib = _load_lib()
    x = np.ascontiguousarray(x)
    assert x.ndim == 3
    taps2 = np.ascontiguousarray(np.asarray(taps, dtype=np.float32).reshape(-1, np.asarray(taps).shape[-1]))
    G, K = taps2.shape
    assert 1 <= K <= 64
    BH, N, C = x.shape
    y = np.empty_like(x)
    if x.dtype == np.float32:
        fn = lib.oracle_fir_f32
    elif x.dtype == np.uint16:
        fn = lib.oracle_fir_bf16
    else:
        raise TypeError("fir_contract takes float32 or bf16 bits (uint16)")
    fn(x.ctypes.data, y.ctypes.data, BH, N, C, taps2.ctypes.data, G, K, int(adjoint))
    return y


# --------------------------------------------------------------------------
# bf16 helpers (bit patterns in uint16)
# --------------------------------------------------------------------------
def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# --------------------------------------------------------------------------
# power-norm peak gate (eager semantics)
# --------------------------------------------------------------------------
def _pow_p(pos: np.ndarray, p: float) -> np.ndarray:
    # src/pnfirtau_attention.py:98-105
    if p == 10.0:
        x2 = pos * pos
        x4 = x2 * x2
        return x4 * x4 * x2
    if p == 2.0:
        return pos * pos
    out = np.zeros_like(pos)
    m = pos > 0
    out[m] = pos[m] ** p
    return out


def _dpow_p(pos: np.ndarray, p: float) -> np.ndarray:
    """d/dpos of _pow_p, zero where pos <= 0 (p > 1)."""
    out = np.zeros_like(pos)
    m = pos > 0
    out[m] = p * pos[m] ** (p - 1.0)
    return out


def _strength(pos, pw, mass, mode):
    if mode == "peak":
        return pos.max(axis=-1, keepdims=True)
    if mode == "mass_relu":
        return pos.sum(axis=-1, keepdims=True)
    if mode == "mass_pow":
        return mass
    raise ValueError(f"unknown silence_mode={mode}")


def power_norm_peak_gate(scores, p=10.0, gamma=0.5, silence_mode="peak", dtype=np.float64):
    """W = relu(s)^p / (sum relu(s)^p + 1e-12) * gate  (src/pnfirtau_attention.py:87-119)."""
    s = np.asarray(scores, dtype=dtype)
    pos = np.maximum(s, 0)
    pw = _pow_p(pos, p)
    mass = pw.sum(axis=-1, keepdims=True)
    w = pw / (mass + dtype(EPS_Z))
    if gamma is not None and gamma > 0:
        st = _strength(pos, pw, mass, silence_mode)
        w = w * (st / (st + dtype(gamma)))
    return w


def power_norm_peak_gate_bwd(scores, dW, p=10.0, gamma=0.5, silence_mode="peak"):
    """Gradient of ``power_norm_peak_gate`` w.r.t. scores, float64.

    Torch autograd semantics of the eager composition: relu'(0) = 0, amax
    splits its gradient evenly over tied maxima.
    """
    s = np.asarray(scores, dtype=np.float64)
    dW = np.asarray(dW, dtype=np.float64)
    pos = np.maximum(s, 0)
    pw = _pow_p(pos, p)
    mass = pw.sum(axis=-1, keepdims=True)
    Zc = mass + EPS_Z
    w = pw / Zc
    has_gate = gamma is not None and gamma > 0
    if has_gate:
        st = _strength(pos, pw, mass, silence_mode)
        g = st / (st + gamma)
        dw = dW * g
        dg = (dW * w).sum(axis=-1, keepdims=True)
        dst = dg * gamma / (st + gamma) ** 2
    else:
        dw = dW
    dpw = (dw - (dw * w).sum(axis=-1, keepdims=True)) / Zc
    if has_gate and silence_mode == "mass_pow":
        dpw = dpw + dst
    dpos = dpw * _dpow_p(pos, p)
    if has_gate and silence_mode == "peak":
        tie = pos == pos.max(axis=-1, keepdims=True)
        dpos = dpos + tie * dst / tie.sum(axis=-1, keepdims=True)
    elif has_gate and silence_mode == "mass_relu":
        dpos = dpos + dst
    return dpos * (s > 0)


# --------------------------------------------------------------------------
# row-fused score kernel semantics (src/triton_pnfirtau.py:141-303)
# --------------------------------------------------------------------------
def _row_valid(N, causal):
    if causal:
        return np.arange(N)[None, :] <= np.arange(N)[:, None]
    return np.ones((N, N), dtype=bool)


def pn_rows_fwd(raw, tau, scale=1.0, p=10.0, gamma=0.5, causal=True, dtype=np.float64):
    """Row kernel forward: returns (W, M, Z, Nmax) for raw [..., N, N].

    s = raw*scale - tau; u = relu on valid (col <= row if causal) entries;
    silent rows (peak <= 0) give W = 0, M = 0, Z = 1e-12, Nmax = 0
    (src/triton_pnfirtau.py:170-212).
    """
    raw = np.asarray(raw, dtype=dtype)
    N = raw.shape[-1]
    assert raw.shape[-2] == N
    valid = _row_valid(N, causal)
    s = raw * dtype(scale) - dtype(tau)
    u = np.where(valid & (s > 0), s, 0).astype(dtype)
    peak = u.max(axis=-1)
    if p == 10.0 or p == 2.0:
        pw = _pow_p(u, p)
    else:
        pw = np.zeros_like(u)
        m = u > 0
        pw[m] = np.exp(np.log(u[m]) * p)
    mass = pw.sum(axis=-1)
    z = mass + dtype(EPS_Z)
    has_gamma = gamma is not None and gamma > 0
    gate = peak / (peak + dtype(gamma)) if has_gamma else np.ones_like(peak)
    W = pw * (gate / z)[..., None]
    nmax = (u == peak[..., None]).sum(axis=-1).astype(np.int32)
    silent = peak <= 0
    W[silent] = 0
    z = np.where(silent, dtype(EPS_Z), z)
    nmax = np.where(silent, 0, nmax).astype(np.int32)
    peak = np.where(silent, 0, peak)
    return W, peak, z, nmax


def pn_rows_bwd(dW, raw, tau, M, Z, Nmax, scale=1.0, p=10.0, gamma=0.5, causal=True):
    """Row kernel backward, float64: returns (d_raw, dtau_rows) (src/triton_pnfirtau.py:214-303)."""
    raw = np.asarray(raw, dtype=np.float64)
    dy = np.asarray(dW, dtype=np.float64)
    N = raw.shape[-1]
    valid = _row_valid(N, causal)
    s = raw * scale - float(tau)
    u = np.where(valid & (s > 0), s, 0.0)
    dy = np.where(valid, dy, 0.0)
    M = np.asarray(M, dtype=np.float64)[..., None]
    Z = np.asarray(Z, dtype=np.float64)[..., None]
    nm = np.asarray(Nmax, dtype=np.float64)[..., None]
    if p == 10.0:
        upm1 = u**9
    elif p == 2.0:
        upm1 = u
    else:
        upm1 = np.where(u > 0, np.exp(np.log(np.where(u > 0, u, 1.0)) * (p - 1.0)), 0.0)
    pw = upm1 * u
    what = pw / Z
    dot = (dy * what).sum(axis=-1, keepdims=True)
    has_gamma = gamma is not None and gamma > 0
    if has_gamma:
        gate = M / (M + gamma)
        dgate = gamma / ((M + gamma) ** 2)
        du_gate = np.where(u == M, dot * dgate / np.maximum(nm, 1.0), 0.0)
    else:
        gate = np.ones_like(M)
        du_gate = 0.0
    du_norm = (p * gate / Z) * upm1 * (dy - dot)
    du = np.where(u > 0, du_norm + du_gate, 0.0)
    silent = M[..., 0] <= 0
    du[silent] = 0.0
    return du * scale, -du.sum(axis=-1)


def eager_scores(raw, tau, scale=1.0, p=10.0, gamma=0.5, causal=True):
    """Eager fallback of triton_pn_fir_tau_scores (src/triton_pnfirtau.py:802-811), float64."""
    s = np.asarray(raw, dtype=np.float64) * scale - float(tau)
    if causal:
        N = s.shape[-1]
        s = np.where(np.triu(np.ones((N, N), dtype=bool), 1), MASK_FILL, s)
    return power_norm_peak_gate(s, p=p, gamma=gamma, silence_mode="peak")


# --------------------------------------------------------------------------
# flash semantics (src/triton_pnfirtau.py:313-621)
# --------------------------------------------------------------------------
def _flash_scores(q, k, tau, scale, causal, dtype):
    N = q.shape[-2]
    Nk = k.shape[-2]
    s = np.matmul(q.astype(dtype), np.swapaxes(k.astype(dtype), -1, -2)) * dtype(scale) - dtype(tau)
    if causal:
        valid = np.arange(Nk)[None, :] <= np.arange(N)[:, None]
    else:
        valid = np.ones((N, Nk), dtype=bool)
    return s, valid


def flash_fwd(q, k, v, tau, scale=None, gamma=0.5, causal=True, dtype=np.float64,
              p_bf16=False):
    """Flash forward semantics on [..., N, d]: returns (O, M, Z, Nmax).

    u = relu(q k^T * scale - tau) on valid entries; P = u^10; Z = sum P + 1e-12;
    M = max u; Nmax = #(u == M) when M > 0 else 0; gate = M/(M+gamma) (0 when
    M <= 0); O = (P v) * gate / Z  (src/triton_pnfirtau.py:383-443).

    ``p_bf16``: P rounded to bf16 before it weights v and enters Z -- the weights a bf16
    kernel multiplies v by (src/triton_pnfirtau.py:417-420); the reference's kernel sums the
    unrounded P into its mass (:405), the default here.  Each rounded term is within
    the bf16 unit roundoff 2^-8 of P.
    """
    q = np.asarray(q)
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s, valid = _flash_scores(q, np.asarray(k), tau, scale, causal, dtype)
    u = np.where(valid & (s > 0), s, 0).astype(dtype)
    P = _pow_p(u, 10.0)
    if p_bf16:
        P = round_bf16(P).astype(dtype)
    mass = P.sum(axis=-1)
    Z = mass + dtype(EPS_Z)
    M = u.max(axis=-1)
    nmax = np.where(M > 0, (u == M[..., None]).sum(axis=-1), 0).astype(np.int32)
    has_gamma = gamma is not None and gamma > 0
    if has_gamma:
        gate = np.where(M > 0, M / (M + dtype(gamma)), 0).astype(dtype)
    else:
        gate = np.where(M > 0, 1, 0).astype(dtype)
    O = np.matmul(P, np.asarray(v).astype(dtype)) * (gate / Z)[..., None]
    return O, M, Z, nmax


def flash_bwd(q, k, v, tau, dO, scale=None, gamma=0.5, causal=True, return_abs=False,
              dtype=np.float64):
    """Flash backward semantics, float64: returns (dq, dk, dv, dtau).

    Recomputes u from q, k; w = u^10 g/Z; dv = w^T dO; dW = dO v^T;
    D = sum_j dW_ij P_ij / Z_i (equal to <dO_i, O_i>/g_i, the flash identity);
    du = 1[u>0] [(10 g/Z) u^9 (dW - D) + 1[u == M] D gamma/(M+gamma)^2 / Nmax];
    dS = du*scale; dq = dS k; dk = dS^T q; dtau = -sum du
    (src/triton_pnfirtau.py:530-602, :959).
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    dO = np.asarray(dO, dtype=dtype)
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s, valid = _flash_scores(q, k, tau, scale, causal, dtype)
    u = np.where(valid & (s > 0), s, dtype(0))
    P = _pow_p(u, 10.0)
    Z = (P.sum(axis=-1) + EPS_Z)[..., None]
    M = u.max(axis=-1)[..., None]
    nmax = (u == M).sum(axis=-1, keepdims=True)
    has_gamma = gamma is not None and gamma > 0
    g = np.where(M > 0, M / (M + gamma), 0.0) if has_gamma else np.where(M > 0, 1.0, 0.0)
    w = P * g / Z
    dv = np.matmul(np.swapaxes(w, -1, -2), dO)
    dW = np.matmul(dO, np.swapaxes(v, -1, -2))
    D = (dW * P / Z).sum(axis=-1, keepdims=True)
    du = (10.0 * g / Z) * u**9 * (dW - D)
    if has_gamma:
        tie = (u == M) & (M > 0)
        du = du + np.where(tie, D * gamma / (M + gamma) ** 2 / np.maximum(nmax, 1), 0.0)
    du = np.where(u > 0, du, 0.0)
    dS = du * scale
    dq = np.matmul(dS, k)
    dk = np.matmul(np.swapaxes(dS, -1, -2), q)
    if return_abs:  # sum |du|: the conditioning scale of the dtau sum
        return dq, dk, dv, -du.sum(), np.abs(du).sum()
    return dq, dk, dv, -du.sum()


def flash_reference_bf16(q, k, v, tau, dO, scale=None, gamma=0.5, causal=True):
    """The reference kernels' bf16 rounding points, float64 everywhere else: returns
    (O, dq, dk, dv, dtau) as the reference's bf16 forward and backward would form them.

    Forward (src/triton_pnfirtau.py:405, :417-420, :422-429): P = u^10 weights v after
    rounding to bf16, the mass sums the unrounded P, and O is stored in bf16.  Backward
    (:566-571, :575-577, :590-600): w = u^10 g/Z is rounded to bf16 for dV; D = <dO, O>/g
    uses the stored bf16 O; dS = du * scale is rounded to bf16 for dK and dQ; dtau = -sum du
    is not rounded.  Inputs are taken as given (already bf16-valued).  This is the error a
    bf16 kernel with the reference's structure carries, for comparison with the HIP kernels'.
    """
    q, k, v, dO = (np.asarray(t, dtype=np.float64) for t in (q, k, v, dO))
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s, valid = _flash_scores(q, k, tau, scale, causal, np.float64)
    u = np.where(valid & (s > 0), s, 0.0)
    P = _pow_p(u, 10.0)
    Z = (P.sum(axis=-1) + EPS_Z)[..., None]
    M = u.max(axis=-1)[..., None]
    nmax = (u == M).sum(axis=-1, keepdims=True)
    has_gamma = gamma is not None and gamma > 0
    g = np.where(M > 0, M / (M + gamma), 0.0) if has_gamma else np.where(M > 0, 1.0, 0.0)
    rb = lambda a: round_bf16(a).astype(np.float64)  # noqa: E731
    O = rb(np.matmul(rb(P), v) * (g / Z))
    w = P * g / Z
    dv = np.matmul(np.swapaxes(rb(w), -1, -2), dO)
    dW = np.matmul(dO, np.swapaxes(v, -1, -2))
    D = np.where(g > 0, (dO * O).sum(axis=-1, keepdims=True) / np.where(g > 0, g, 1.0), 0.0)
    du = (10.0 * g / Z) * u**9 * (dW - D)
    if has_gamma:
        tie = (u == M) & (M > 0)
        du = du + np.where(tie, D * gamma / (M + gamma) ** 2 / np.maximum(nmax, 1), 0.0)
    du = np.where(u > 0, du, 0.0)
    dS = rb(du * scale)
    dq = np.matmul(dS, k)
    dk = np.matmul(np.swapaxes(dS, -1, -2), q)
    return O, dq, dk, dv, -du.sum()


def tile_activity(q, k, tau, scale=None, causal=True, tile=64):
    """Per 64x64 tile activity of the flash skip rule, float64.

    Returns (active, ambiguous), each [..., ceil(N/tile), ceil(Nk/tile)] bool.
    A tile is active when max over its valid entries of relu(q.k*scale - tau)
    is > 0 (src/triton_pnfirtau.py:395-400; the 64x64 convention of
    experiments/exp4b_mha6_instrumentation.py:96-111).  Tiles entirely above
    the causal diagonal are reported inactive.  ``ambiguous`` flags tiles whose
    max score is within a rounding bound of zero, i.e. whose activity could
    flip under a different (but correct) fp32 accumulation order.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s, valid = _flash_scores(q, k, tau, scale, causal, np.float64)
    d = q.shape[-1]
    bound = (np.matmul(np.abs(q), np.swapaxes(np.abs(k), -1, -2)) * scale * (d + 2) * 2.0**-23
             + (abs(float(tau)) + np.abs(s)) * 2.0**-22)
    s = np.where(valid, s, -np.inf)
    N, Nk = s.shape[-2], s.shape[-1]
    nr, nc = -(-N // tile), -(-Nk // tile)
    pad_r, pad_c = nr * tile - N, nc * tile - Nk
    lead = s.shape[:-2]
    sp = np.pad(s, [(0, 0)] * len(lead) + [(0, pad_r), (0, pad_c)], constant_values=-np.inf)
    bp = np.pad(np.where(valid, bound, 0.0), [(0, 0)] * len(lead) + [(0, pad_r), (0, pad_c)])
    sp = sp.reshape(lead + (nr, tile, nc, tile))
    bp = bp.reshape(lead + (nr, tile, nc, tile))
    tmax = sp.max(axis=(-3, -1))
    bmax = bp.max(axis=(-3, -1))
    active = tmax > 0
    ambiguous = np.isfinite(tmax) & (np.abs(tmax) <= bmax)
    return active, ambiguous


# --------------------------------------------------------------------------
# PnFirTauMHA dense composition, forward + backward (src/pnfirtau_attention.py:195-247)
# --------------------------------------------------------------------------
def mha_fwd_bwd(x, w_qkv, w_out, tau, taps, n_heads, dout=None, b_qkv=None, b_out=None,
                p=10.0, gamma=0.5, silence_mode="peak", causal=True):
    """Forward (and backward when ``dout`` is given) of PnFirTauMHA with dropout 0, float64.

    qkv = x W_qkv^T (+b); q, k, v = the three D-wide column blocks of qkv
    (reshape(B, N, 3, H, hd).unbind(2), src/pnfirtau_attention.py:221-222);
    k is filtered along N over all H*hd channels with shared taps (:223-225);
    scores = q k^T / sqrt(hd) - tau, then entries above the diagonal set to
    -1e4 (:231-237); W = power_norm_peak_gate (:239-241); out = (W v) W_out^T.
    Returns dict with out, W and (if dout) dx, dw_qkv, dw_out, dtau (+ biases).
    """
    x = np.asarray(x, dtype=np.float64)
    Wq = np.asarray(w_qkv, dtype=np.float64)
    Wo = np.asarray(w_out, dtype=np.float64)
    B, N, D = x.shape
    H = n_heads
    hd = D // H
    scale = 1.0 / np.sqrt(hd)
    qkv = x @ Wq.T
    if b_qkv is not None:
        qkv = qkv + np.asarray(b_qkv, dtype=np.float64)
    q_f, k_raw, v_f = qkv[..., :D], qkv[..., D : 2 * D], qkv[..., 2 * D :]
    k_f = fir(k_raw, taps) if np.asarray(taps).size > 1 else k_raw

    def heads(t):
        return t.reshape(B, N, H, hd).transpose(0, 2, 1, 3)

    q, k, v = heads(q_f), heads(k_f), heads(v_f)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale - float(tau)
    masked = np.triu(np.ones((N, N), dtype=bool), 1) if causal else np.zeros((N, N), dtype=bool)
    s = np.where(masked, MASK_FILL, s)
    Wt = power_norm_peak_gate(s, p, gamma, silence_mode)
    o = np.matmul(Wt, v)
    o_flat = o.transpose(0, 2, 1, 3).reshape(B, N, D)
    out = o_flat @ Wo.T
    if b_out is not None:
        out = out + np.asarray(b_out, dtype=np.float64)
    res = {"out": out, "W": Wt}
    if dout is None:
        return res
    dout = np.asarray(dout, dtype=np.float64)
    res["dw_out"] = dout.reshape(-1, D).T @ o_flat.reshape(-1, D)
    if b_out is not None:
        res["db_out"] = dout.reshape(-1, D).sum(axis=0)
    do = heads(dout @ Wo)
    dWt = np.matmul(do, np.swapaxes(v, -1, -2))
    dv = np.matmul(np.swapaxes(Wt, -1, -2), do)
    ds = power_norm_peak_gate_bwd(s, dWt, p, gamma, silence_mode)
    ds = np.where(masked, 0.0, ds)
    res["dtau"] = -ds.sum()
    res["dtau_abs"] = np.abs(ds).sum()
    draw = ds * scale
    dq = np.matmul(draw, k)
    dk = np.matmul(np.swapaxes(draw, -1, -2), q)

    def flat(t):
        return t.transpose(0, 2, 1, 3).reshape(B, N, D)

    dk_raw = fir(flat(dk), taps, adjoint=True) if np.asarray(taps).size > 1 else flat(dk)
    dqkv = np.concatenate([flat(dq), dk_raw, flat(dv)], axis=-1)
    res["dx"] = dqkv @ Wq
    res["dw_qkv"] = dqkv.reshape(-1, 3 * D).T @ x.reshape(-1, D)
    if b_qkv is not None:
        res["db_qkv"] = dqkv.reshape(-1, 3 * D).sum(axis=0)
    return res
