"""Pins the CPU oracle (oracle/) against the reference's own vectors and the mathematics.

Every function of the oracle is checked against at least one of: a golden vector
written from the reference (tests/golden/make_golden.py), a vector the reference
repository itself stores, a closed form, an independent library routine, or
finite differences -- chosen so that a dropped term, a wrong sign or index or a
transposed operand fails.
"""
import numpy as np
import pytest

from oracle import pnfirtau_oracle as O
from tests.conftest import golden

# results/exp1_legacy_13stacks.json:29 of the reference: taps present -> past
REF_TAPS_PRESENT_TO_PAST = [0.33288270235061646, 0.2937679588794708, 0.2019035667181015,
                            0.10807118564844131, 0.04505077376961708, 0.014625845476984978,
                            0.003697992768138647]


def test_taps_match_reference_results_vector_bit_exact():
    t = O.causal_gaussian_taps(7)
    assert t.dtype == np.float32
    assert t[::-1].tolist() == REF_TAPS_PRESENT_TO_PAST


def test_taps_other_sizes_match_golden():
    # The oracle sums the exponentials left to right in fp32; the reference's library
    # reduction may order the sum differently, which moves a tap by at most an ulp or two.
    f = golden("fir_eager")
    np.testing.assert_allclose(O.causal_gaussian_taps(5, sigma_frac=2.0), f["taps5"], rtol=3e-7, atol=0)
    assert O.causal_gaussian_taps(1).tolist() == f["taps1"].tolist() == [1.0]


def test_fir_impulse_response_pins_tap_indexing():
    taps = O.causal_gaussian_taps(7)
    x = np.zeros((1, 20, 3), np.float32)
    x[0, 5, :] = 1.0
    y = O.fir_contract(x, taps)
    for u in range(7):
        assert np.all(y[0, 5 + u] == taps[6 - u])  # lag u carries taps[K-1-u]
    assert np.all(y[0, :5] == 0) and np.all(y[0, 12:] == 0)
    yb = O.fir_contract(O.f32_to_bf16_bits(x), taps)
    for u in range(7):
        assert np.all(yb[0, 5 + u] == O.f32_to_bf16_bits(taps[6 - u : 7 - u]))


def test_fir_matches_numpy_convolve_and_float64_restatement():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 50, 4)).astype(np.float32)
    taps = O.causal_gaussian_taps(7)
    h = taps[::-1].astype(np.float64)  # lag order
    ref = np.stack([np.stack([np.convolve(x[b, :, c].astype(np.float64), h)[:50] for c in range(4)], -1)
                    for b in range(3)])
    assert np.abs(O.fir(x, taps) - ref).max() < 1e-12
    assert np.abs(O.fir_contract(x, taps) - ref).max() < 2e-6


def test_fir_adjoint_identity_and_causality():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 40, 5))
    g = rng.standard_normal((2, 40, 5))
    taps = O.causal_gaussian_taps(7)
    lhs = (O.fir(x, taps) * g).sum()
    rhs = (x * O.fir(g, taps, adjoint=True)).sum()
    assert abs(lhs - rhs) < 1e-10
    xf = np.ascontiguousarray(x.astype(np.float32))
    x2 = xf.copy()
    x2[:, 30:] += 5.0
    assert np.array_equal(O.fir_contract(xf, taps)[:, :30], O.fir_contract(x2, taps)[:, :30])
    ga = np.ascontiguousarray(g.astype(np.float32))
    g2 = ga.copy()
    g2[:, :10] += 5.0
    assert np.array_equal(O.fir_contract(ga, taps, adjoint=True)[:, 10:],
                          O.fir_contract(g2, taps, adjoint=True)[:, 10:])


def test_fir_contract_per_head_rows_and_eager_golden():
    f = golden("fir_eager")
    y = O.fir_contract(f["x"], f["taps"])
    assert np.abs(y - f["y_f32"]).max() < 1e-6
    rng = np.random.default_rng(2)
    x = rng.standard_normal((6, 30, 8)).astype(np.float32)
    taps = rng.uniform(0, 1, (3, 7)).astype(np.float32)
    taps /= taps.sum(-1, keepdims=True)
    y = O.fir_contract(x, taps)
    ref = O.fir(x.reshape(2, 3, 30, 8), taps, per_head=True).reshape(6, 30, 8)
    assert np.abs(y - ref).max() < 2e-6


@pytest.mark.parametrize("i", range(8))
def test_power_norm_gate_matches_reference_golden(i):
    f = golden("pn_gate")
    p, g, m = str(f["cases"][i]).split("|")
    p, g = float(p), (None if g == "None" else float(g))
    w = O.power_norm_peak_gate(f["s"], p, g, m)
    ds = O.power_norm_peak_gate_bwd(f["s"], f["dW"], p, g, m)
    assert np.abs(w - f[f"w_{i}"]).max() < 1e-14
    assert np.abs(ds - f[f"ds_{i}"]).max() < 1e-12


def test_power_norm_closed_forms():
    rng = np.random.default_rng(3)
    s = rng.standard_normal((4, 33)) * 2
    s[1] = -np.abs(s[1]) - 0.1  # silent row
    w = O.power_norm_peak_gate(s, 10.0, 0.5, "peak")
    peak = np.maximum(s, 0).max(-1)
    np.testing.assert_allclose(w.sum(-1), peak / (peak + 0.5), rtol=1e-12, atol=1e-15)
    assert np.all(w[1] == 0)
    # p = 10 by squaring agrees with pow
    pos = np.maximum(s, 0)
    np.testing.assert_allclose(O._pow_p(pos, 10.0), pos**10, rtol=1e-14)


@pytest.mark.parametrize("mode", ["peak", "mass_relu", "mass_pow"])
def test_power_norm_backward_finite_differences(mode):
    rng = np.random.default_rng(4)
    s = rng.standard_normal((2, 9)) + 0.3
    dW = rng.standard_normal((2, 9))
    ds = O.power_norm_peak_gate_bwd(s, dW, 10.0, 0.5, mode)
    eps = 1e-6
    num = np.zeros_like(s)
    for idx in np.ndindex(s.shape):
        sp, sm = s.copy(), s.copy()
        sp[idx] += eps
        sm[idx] -= eps
        num[idx] = ((O.power_norm_peak_gate(sp, 10.0, 0.5, mode) - O.power_norm_peak_gate(sm, 10.0, 0.5, mode)) * dW).sum() / (2 * eps)
    np.testing.assert_allclose(ds, num, rtol=1e-5, atol=1e-7)


def test_rows_kernel_semantics_equal_eager_and_reference_fallback():
    f = golden("scores_fallback")
    raw, tau = f["raw"], float(f["tau"])
    for i in range(3):
        scale, p, g, causal = f[f"args_{i}"]
        g = None if np.isnan(g) else float(g)
        w_ref = f[f"w_{i}"]
        w_e = O.eager_scores(raw, tau, scale, p, g, bool(causal))
        assert np.abs(w_e - w_ref).max() < 1e-6
        W, M, Z, Nm = O.pn_rows_fwd(raw, tau, scale, p, g, bool(causal))
        assert np.abs(W - w_ref).max() < 1e-6
    # backward of the row semantics equals the eager gradient (peak mode)
    rng = np.random.default_rng(5)
    raw = rng.standard_normal((3, 16, 16)) * 3
    raw[0, 4, :3] = raw[0, 4, 2]  # tie at a row peak
    dW = rng.standard_normal((3, 16, 16))
    W, M, Z, Nm = O.pn_rows_fwd(raw, 0.2, 0.5, 10.0, 0.5, True)
    d_raw, dtr = O.pn_rows_bwd(dW, raw, 0.2, M, Z, Nm, 0.5, 10.0, 0.5, True)
    s = raw * 0.5 - 0.2
    s = np.where(np.triu(np.ones((16, 16), bool), 1), O.MASK_FILL, s)
    ds = O.power_norm_peak_gate_bwd(s, dW, 10.0, 0.5, "peak")
    ds = np.where(np.triu(np.ones((16, 16), bool), 1), 0.0, ds)
    np.testing.assert_allclose(d_raw, ds * 0.5, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dtr.sum(), -ds.sum(), rtol=1e-9)


def _rand_qkv(rng, B, H, N, d):
    return [rng.standard_normal((B, H, N, d)) for _ in range(3)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("gamma", [0.5, None])
def test_flash_semantics_equal_dense_composition(causal, gamma):
    rng = np.random.default_rng(6)
    q, k, v = _rand_qkv(rng, 2, 2, 40, 8)
    dO = rng.standard_normal(q.shape)
    tau, scale = 0.1, 1 / np.sqrt(8)
    Of, M, Z, Nm = O.flash_fwd(q, k, v, tau, scale, gamma, causal)
    s = q @ np.swapaxes(k, -1, -2) * scale - tau
    if causal:
        s = np.where(np.triu(np.ones((40, 40), bool), 1), O.MASK_FILL, s)
    W = O.power_norm_peak_gate(s, 10.0, gamma, "peak")
    np.testing.assert_allclose(Of, W @ v, rtol=1e-10, atol=1e-13)
    dq, dk, dv, dtau = O.flash_bwd(q, k, v, tau, dO, scale, gamma, causal)
    dW = dO @ np.swapaxes(v, -1, -2)
    ds = O.power_norm_peak_gate_bwd(s, dW, 10.0, gamma, "peak")
    if causal:
        ds = np.where(np.triu(np.ones((40, 40), bool), 1), 0.0, ds)
    np.testing.assert_allclose(dv, np.swapaxes(W, -1, -2) @ dO, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dq, ds * scale @ k, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, np.swapaxes(ds * scale, -1, -2) @ q, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dtau, -ds.sum(), rtol=1e-9)


def test_flash_identity_D_equals_dO_dot_O_over_gate():
    rng = np.random.default_rng(7)
    q, k, v = _rand_qkv(rng, 1, 1, 30, 8)
    dO = rng.standard_normal(q.shape)
    Of, M, Z, Nm = O.flash_fwd(q, k, v, 0.0, None, 0.5, True)
    s = q @ np.swapaxes(k, -1, -2) / np.sqrt(8)
    u = np.where(np.tril(np.ones((30, 30), bool)) & (s > 0), s, 0)
    what = u**10 / Z[..., None]
    D_direct = ((dO @ np.swapaxes(v, -1, -2)) * what).sum(-1)
    g = M / (M + 0.5)
    live = M > 0
    assert live.sum() > 20
    np.testing.assert_allclose(((dO * Of).sum(-1))[live] / g[live], D_direct[live], rtol=1e-10)


def test_flash_special_cases():
    rng = np.random.default_rng(8)
    # N == 1: O = g * v0 with g = u/(u+gamma)
    q, k, v = _rand_qkv(rng, 1, 1, 1, 4)
    q[...] = np.abs(q) + 0.5
    k[...] = np.abs(k) + 0.5
    Of, M, Z, Nm = O.flash_fwd(q, k, v, 0.0, 0.5, 0.5, True)
    u = (q * k).sum() * 0.5
    np.testing.assert_allclose(Of[0, 0, 0], u / (u + 0.5) * v[0, 0, 0] * u**10 / (u**10 + 1e-12), rtol=1e-12)
    assert Nm[0, 0, 0] == 1
    # tau -> +inf: everything silent, zero output and grads, no active tiles
    q, k, v = _rand_qkv(rng, 1, 2, 70, 4)
    Of, M, Z, Nm = O.flash_fwd(q, k, v, 1e6)
    assert np.all(Of == 0) and np.all(M == 0) and np.all(Nm == 0)
    dq, dk, dv, dt = O.flash_bwd(q, k, v, 1e6, rng.standard_normal(q.shape))
    assert np.all(dq == 0) and np.all(dk == 0) and np.all(dv == 0) and dt == 0
    act, amb = O.tile_activity(q, k, 1e6)
    assert not act.any() and not amb.any()
    # one active key per row: O = g * v_j
    q = np.zeros((1, 1, 3, 2)); k = np.zeros((1, 1, 3, 2)); v = rng.standard_normal((1, 1, 3, 2))
    q[..., 0] = 1.0; k[0, 0, 1, 0] = 2.0
    Of, M, Z, Nm = O.flash_fwd(q, k, v, 0.0, 1.0, 0.5, True)
    np.testing.assert_allclose(Of[0, 0, 2], 2.0 / 2.5 * v[0, 0, 1] * 2.0**10 / (2.0**10 + 1e-12), rtol=1e-12)
    assert np.all(Of[0, 0, 0] == 0)


def test_flash_bf16_weights_option_known_answers():
    """p_bf16 rounds P = u^10 to bf16 before it weights v and enters Z.  One key with
    u = 1.5: P = 1.5^10 = 57.665..., whose bf16 value is 231/128 * 32 = 57.75 (rounding u
    instead of P would leave 57.665).  Powers of two are exact in bf16, so u in {0.5, 1, 2}
    gives bitwise the unrounded result."""
    q = np.ones((1, 1, 1, 1)); k = np.full((1, 1, 1, 1), 1.5); v = np.full((1, 1, 1, 1), 3.0)
    Of, M, Z, Nm = O.flash_fwd(q, k, v, 0.0, 1.0, None, True, p_bf16=True)
    assert Z[0, 0, 0] == 57.75 + 1e-12
    assert abs(Of[0, 0, 0, 0] - 3.0 * 57.75 / (57.75 + 1e-12)) <= 1e-14
    assert O.flash_fwd(q, k, v, 0.0, 1.0, None, True)[2][0, 0, 0] == 1.5**10 + 1e-12
    q = np.ones((1, 1, 3, 1)); k = np.array([0.5, 1.0, 2.0]).reshape(1, 1, 3, 1)
    v = np.arange(3.0).reshape(1, 1, 3, 1)
    a = O.flash_fwd(q, k, v, 0.0, 1.0, 0.5, True, p_bf16=True)
    b = O.flash_fwd(q, k, v, 0.0, 1.0, 0.5, True)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    # on random rows the rounded mass stays within the bf16 rounding of its terms
    rng = np.random.default_rng(9)
    q, k, v = _rand_qkv(rng, 1, 2, 64, 8)
    Zr = O.flash_fwd(q, k, v, 0.0, p_bf16=True)[2]
    Ze = O.flash_fwd(q, k, v, 0.0)[2]
    assert np.all(np.abs(Zr - Ze) <= 2.0**-8 * Ze)  # bf16 unit roundoff
    assert np.any(Zr != Ze)


def test_flash_reference_bf16_rounding_points_known_answers():
    """One query, one key (d = 1, q = k = 1, v = 3, dO = 1, scale 1, tau 0, gamma 0.5): u = 1,
    P = 1, g = 2/3, O = 2, D = <dO, O>/g = 3 = dW, so du is the tie term alone,
    3 * 0.5 / 1.5^2 = 2/3.  The reference's kernels round dS = 2/3 and w = g/Z ~ 2/3 to bf16,
    0.66796875 (= 171/256): dq = dk = dv = 0.66796875, while dtau = -2/3 is not rounded.
    The float64 oracle gives 2/3 for all three."""
    one = np.ones((1, 1, 1, 1))
    O_, dq, dk, dv, dt = O.flash_reference_bf16(one, one, 3 * one, 0.0, one, 1.0, 0.5, True)
    assert O_[0, 0, 0, 0] == 2.0
    assert dq[0, 0, 0, 0] == dk[0, 0, 0, 0] == dv[0, 0, 0, 0] == 171 / 256
    assert abs(dt + 2 / 3) < 1e-12
    eq, ek, ev, et = O.flash_bwd(one, one, 3 * one, 0.0, one, 1.0, 0.5, True)
    # (the 1e-12 in Z leaves dW - D = 3e-12, hence the 1e-10)
    assert abs(eq[0, 0, 0, 0] - 2 / 3) < 1e-10 and abs(ek[0, 0, 0, 0] - 2 / 3) < 1e-10
    assert abs(ev[0, 0, 0, 0] - 2 / 3) < 1e-10 and abs(et - dt) < 1e-10
    # on random inputs it stays within bf16 rounding of the exact gradients
    rng = np.random.default_rng(10)
    q, k, v = _rand_qkv(rng, 1, 1, 48, 8)
    d = rng.standard_normal(q.shape)
    _, rq, rk, rv, rt = O.flash_reference_bf16(q, k, v, 0.0, d)
    xq, xk, xv, xt = O.flash_bwd(q, k, v, 0.0, d)
    for a, b in ((rq, xq), (rk, xk), (rv, xv)):
        assert np.abs(a - b).max() <= 0.05 * np.abs(b).max() and np.any(a != b)


def test_flash_reference_bf16_rounding_points_two_keys():
    """Two queries, two keys (d = 1, q = (0, 1), k = (1, 1/2), v = (3, 5), dO = 1, scale 1,
    tau 0, gamma 0.5, causal).  Row 0 is silent (s = 0).  Row 1: u = (1, 1/2),
    P = (1, 2^-10), Z = 1025/1024, M = 1, g = 2/3, one tie (key 0).
    * O = (3 + 5 / 1024) g / Z = 6154/3075 = 2.0013..., stored in bf16 as 2.0.
    * w = P g / Z = (2048/3075, 2/3075), rounded to bf16 for dV: 0.66796875 and
      0.000652313232421875 (= 171/256 and 171/262144).
    * D = <dO, O>/g with the stored O: 3 = dW_0, so du_0 is the tie term alone,
      3 * 0.5 / 1.5^2 = 2/3, and du_1 = (10 g / Z) 2^-9 (5 - 3) = 0.0260162...; dS = du rounded
      to bf16: 0.66796875 and 0.0260009765625 (= 213/8192).
    * dq_1 = dS_0 k_0 + dS_1 k_1 = 0.68096923828125, dk = dS (q_1 = 1), dv = bf16(w), and
      dtau = -(du_0 + du_1) is not rounded.
    Each value is written out by hand from the reference's rounding points
    (src/triton_pnfirtau.py:417-420 O and its bf16 store, :566-571 w, :598-600 dS)."""
    q = np.array([0.0, 1.0]).reshape(1, 1, 2, 1)
    k = np.array([1.0, 0.5]).reshape(1, 1, 2, 1)
    v = np.array([3.0, 5.0]).reshape(1, 1, 2, 1)
    dO = np.ones((1, 1, 2, 1))
    O_, dq, dk, dv, dt = O.flash_reference_bf16(q, k, v, 0.0, dO, 1.0, 0.5, True)
    assert O_[0, 0, 0, 0] == 0.0 and O_[0, 0, 1, 0] == 2.0
    assert dq[0, 0, 0, 0] == 0.0 and dq[0, 0, 1, 0] == 0.68096923828125
    assert dk[0, 0, 0, 0] == 171 / 256 and dk[0, 0, 1, 0] == 213 / 8192
    assert dv[0, 0, 0, 0] == 171 / 256 and dv[0, 0, 1, 0] == 171 / 262144
    du1 = (10 * (2 / 3) / (1025 / 1024 + 1e-12)) * 2.0**-9 * 2.0
    assert dt == pytest.approx(-(2 / 3 + du1), rel=1e-12)
    # the exact gradients differ from every rounded one above
    eq, ek, ev, _ = O.flash_bwd(q, k, v, 0.0, dO, 1.0, 0.5, True)
    assert ek[0, 0, 1, 0] != dk[0, 0, 1, 0] and ev[0, 0, 0, 0] != dv[0, 0, 0, 0]


def test_tile_activity_closed_form_all_active():
    # every causal tile active: fully-silent fraction of the nb^2 grid is (nb-1)/(2nb)
    # (0.46875 at nb = 16, the exp4b convention, results/exp4b_mha6_instrumentation.json:24-157)
    N, d = 1024, 4
    q = np.ones((1, 1, N, d)); k = np.ones((1, 1, N, d))
    act, amb = O.tile_activity(q, k, -1.0, tile=64)
    nb = N // 64
    assert act.sum() == nb * (nb + 1) // 2
    assert 1 - act.mean() == pytest.approx((nb - 1) / (2 * nb)) == pytest.approx(0.46875)
    assert not amb.any()


def test_tile_activity_planted_zero_key_blocks():
    rng = np.random.default_rng(9)
    N, d = 512, 8
    q, k, _ = _rand_qkv(rng, 1, 1, N, d)
    silent_blocks = [j for j in range(N // 64) if j % 2 == 0]
    for j in silent_blocks:
        k[..., 64 * j : 64 * j + 64, :] = 0
    act, amb = O.tile_activity(q, k, 0.25)
    assert not amb.any()
    for j in range(N // 64):
        col = act[0, 0, j:, j]
        assert (not col.any()) if j in silent_blocks else col.all()


@pytest.mark.parametrize("name", ["c1_mha_fp32", "c1_mha_fp32_tau", "c1_mha_fp32_bias_modes", "c1_mha_fp32_nogate"])
def test_mha_oracle_matches_reference_golden(name):
    f = golden(name)
    B, N, D, H, bias = [int(x) for x in f["meta"]]
    g = float(f["gamma"])
    r = O.mha_fwd_bwd(f["x"], f["w_qkv"], f["w_out"], float(f["tau"]), f["taps"], H, dout=f["dout"],
                      b_qkv=f["b_qkv"] if bias else None, b_out=f["b_out"] if bias else None,
                      p=float(f["p"]), gamma=None if np.isnan(g) else g, silence_mode=str(f["mode"]))
    keys = ["out", "dx", "dw_qkv", "dw_out", "dtau"] + (["db_qkv", "db_out"] if bias else [])
    for key in keys:
        ref = f[key]
        err = np.abs(r[key] - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 2e-5, (key, err)
    if "W" in f:
        assert np.abs(r["W"] - f["W"]).max() < 1e-6


def test_golden_comparison_detects_planted_oracle_mistakes():
    """Mutations of the oracle (reversed taps, swapped q/k blocks) must fail the golden check."""
    f = golden("c1_mha_fp32")
    B, N, D, H, _ = [int(x) for x in f["meta"]]
    args = dict(dout=f["dout"])
    good = O.mha_fwd_bwd(f["x"], f["w_qkv"], f["w_out"], 0.0, f["taps"], H, **args)
    bad_taps = O.mha_fwd_bwd(f["x"], f["w_qkv"], f["w_out"], 0.0, f["taps"][::-1].copy(), H, **args)
    wq = f["w_qkv"].copy()
    wq[:D], wq[D:2 * D] = f["w_qkv"][D:2 * D], f["w_qkv"][:D]
    bad_split = O.mha_fwd_bwd(f["x"], wq, f["w_out"], 0.0, f["taps"], H, **args)
    ref = f["out"]
    assert np.abs(good["out"] - ref).max() < 1e-5
    assert np.abs(bad_taps["out"] - ref).max() > 1e-3
    assert np.abs(bad_split["out"] - ref).max() > 1e-3
