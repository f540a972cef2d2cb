"""CPU-side tests of the product package: eager primitives against the reference's golden
vectors, module drop-in properties, and the C ABI library surface (no GPU compute)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import paper_01_anti_decoy_pnfirtau_amd as P
from paper_01_anti_decoy_pnfirtau_amd import _lib
from tests.conftest import ROOT, golden


def _t(a):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a))


def test_taps_bit_exact_vs_reference_vector():
    t = P.causal_gaussian_taps(7)
    assert t.flip(0).tolist() == [0.33288270235061646, 0.2937679588794708, 0.2019035667181015,
                                  0.10807118564844131, 0.04505077376961708, 0.014625845476984978,
                                  0.003697992768138647]
    f = golden("fir_eager")
    assert P.causal_gaussian_taps(5, sigma_frac=2.0).tolist() == f["taps5"].tolist()


def test_eager_fir_matches_reference_golden_bit_exact():
    f = golden("fir_eager")
    taps = _t(f["taps"])
    assert torch.equal(P.causal_fir(_t(f["x"]), taps), _t(f["y_f32"]))
    yb = P.causal_fir(_t(f["x_bf16"]), taps)
    assert torch.equal(yb.view(torch.int16), _t(f["y_bf16"]).view(torch.int16))


@pytest.mark.parametrize("i", range(8))
def test_eager_power_norm_matches_reference_golden(i):
    f = golden("pn_gate")
    p, g, m = str(f["cases"][i]).split("|")
    s = _t(f["s"]).clone().requires_grad_(True)
    w = P.power_norm_peak_gate(s, float(p), None if g == "None" else float(g), m)
    w.backward(_t(f["dW"]))
    assert torch.equal(w.detach(), _t(f[f"w_{i}"]))
    assert torch.allclose(s.grad, _t(f[f"ds_{i}"]), rtol=0, atol=1e-15)


def test_unknown_silence_mode_raises():
    with pytest.raises(ValueError):
        P.power_norm_peak_gate(torch.randn(2, 4), silence_mode="nope")


def test_cpu_row_scores_follow_reference_fallback():
    from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import triton_pn_fir_tau_scores

    f = golden("scores_fallback")
    raw, tau = _t(f["raw"]), _t(f["tau"])
    for i in range(3):
        scale, p, g, causal = f[f"args_{i}"]
        w = triton_pn_fir_tau_scores(raw, tau, scale=float(scale), p=float(p),
                                     gamma=None if np.isnan(g) else float(g), causal_mask=bool(causal))
        assert torch.equal(w, _t(f[f"w_{i}"]))


def _load_mha(cls, f, dtype=torch.float32):
    B, N, D, H, bias = [int(x) for x in f["meta"]]
    g = float(f["gamma"])
    cfg = P.PnFirConfig(d_model=D, n_heads=H, p=float(f["p"]), silence_gamma=None if np.isnan(g) else g,
                        silence_mode=str(f["mode"]), bias=bool(bias))
    m = cls(cfg)
    sd = {"qkv.weight": _t(f["w_qkv"]), "out.weight": _t(f["w_out"]),
          "score_tau": _t(f["tau"]).reshape(()).float(), "fir_taps": _t(f["taps"]).float()}
    if bias:
        sd.update({"qkv.bias": _t(f["b_qkv"]), "out.bias": _t(f["b_out"])})
    m.load_state_dict(sd)
    return m.to(dtype)


@pytest.mark.parametrize("name", ["c1_mha_fp32", "c1_mha_fp32_tau", "c1_mha_fp32_bias_modes", "c1_mha_fp32_nogate"])
def test_eager_mha_matches_reference_golden(name):
    f = golden(name)
    m = _load_mha(P.PnFirTauMHA, f)
    x = _t(f["x"]).clone().requires_grad_(True)
    out, W = m(x, return_weights=True)
    out.backward(_t(f["dout"]))
    assert torch.allclose(out, _t(f["out"]), rtol=0, atol=1e-6)
    assert torch.allclose(x.grad, _t(f["dx"]), rtol=0, atol=1e-5)
    assert torch.allclose(m.qkv.weight.grad, _t(f["dw_qkv"]), rtol=0, atol=1e-4)
    assert torch.allclose(m.out.weight.grad, _t(f["dw_out"]), rtol=0, atol=1e-4)
    assert abs(float(m.score_tau.grad) - float(f["dtau"])) <= 1e-6 * max(1.0, abs(float(f["dtau"])))


def test_state_dict_keys_and_subclassing_match_reference():
    cfg = P.PnFirConfig()
    for cls in (P.PnFirTauMHA, P.PnFirTauTritonMHA, P.PnFirTauFlashMHA):
        m = cls(cfg)
        assert list(m.state_dict().keys()) == ["score_tau", "fir_taps", "qkv.weight", "out.weight"]
        assert isinstance(m, P.PnFirTauMHA)
        assert m.score_tau.shape == () and m.fir_taps.shape == (7,)
    mb = P.PnFirTauMHA(P.PnFirConfig(bias=True))
    assert set(mb.state_dict()) == {"score_tau", "qkv.weight", "qkv.bias", "out.weight", "out.bias", "fir_taps"}


def test_default_init_consumes_rng_like_reference():
    f = golden("c1_mha_fp32")
    torch.manual_seed(0)
    m = P.PnFirTauMHA(P.PnFirConfig(d_model=64, n_heads=4, dropout=0.0))
    assert torch.equal(m.qkv.weight.detach(), _t(f["w_qkv"]))
    assert torch.equal(m.out.weight.detach(), _t(f["w_out"]))


def _header_symbols():
    txt = open(os.path.join(ROOT, "include", "pnfx.h")).read()
    return sorted(set(re.findall(r"\b(pnfx_\w+)\s*\(", txt)))


def test_c_abi_library_exports_every_declared_symbol():
    syms = _header_symbols()
    assert syms == sorted(_lib.exported_symbols())
    lib = _lib.lib()
    for s in syms:
        assert hasattr(lib, s), s
    assert lib.pnfx_abi_version() == _lib.ABI_VERSION


def test_c_abi_rejects_bad_arguments_without_touching_the_gpu():
    lib = _lib.lib()
    rc = lib.pnfx_flash_fwd(*([None, 0, 0, 0] * 4), None, None, None, None, None, None, 0,
                            1, 1, 8, 48, None, 0.125, 0.5, 1, 1, 1, None)
    assert rc == -1 and b"head dim" in lib.pnfx_last_error()
    # a bf16 row stride the tile loads' 32-bit row offsets cannot span
    fake16 = ctypes.c_void_p(256)
    ok = [fake16, 64 * 8, 64 * 8, 64]
    rc = lib.pnfx_flash_fwd(*ok, fake16, 64 * 8, 64 * 8, 1 << 25, *ok, *ok, None, fake16, fake16,
                            None, None, None, 0, 1, 1, 8, 64, fake16, 0.125, 0.5, 1, 1, 1, None)
    assert rc == -1 and b"k row stride" in lib.pnfx_last_error()
    rc = lib.pnfx_fir_fwd(None, 0, 0, 0, None, 1, 1, 4, 8, None, 1, 7, 1, None)
    assert rc == -1 and b"null" in lib.pnfx_last_error()
    rc = lib.pnfx_fir_fwd(ctypes.c_void_p(16), 0, 0, 0, ctypes.c_void_p(16), 1, 1, 4, 8,
                          ctypes.c_void_p(16), 1, 17, 1, None)
    assert rc == -1 and b"K=17" in lib.pnfx_last_error()
    need = lib.pnfx_flash_bwd_workspace_size(4, 16, 8192, 64)
    assert need >= 4 * 16 * 8192 * 32
    # the no-allocation backward refuses a shape past its scratch before any device call
    rc = lib.pnfx_flash_bwd_noalloc(*([None, 0, 0, 0] * 4), None, None, 0, 0, 0, None, None, None,
                                    *([None, 0, 0, 0] * 3), None, 4, 16, 16384, 64, None, 0.125,
                                    0.5, 1, 1, 1, None)
    assert rc == -1 and b"scratch" in lib.pnfx_last_error()
    # the fused-FIR forward: bf16, d = 64 and K <= 7 only, refused before any device call
    fake = ctypes.c_void_p(256)
    args = ([fake, 64 * 8, 64 * 8, 64] * 4 + [fake, fake, fake, None, 1, 1, 8, 64, fake, 0.125,
                                              0.5, 1, 1, fake, 1])
    rc = lib.pnfx_flash_fwd_fir(*args, 8, 1, None)
    assert rc == -1 and b"K=8" in lib.pnfx_last_error()
    rc = lib.pnfx_flash_fwd_fir(*args, 7, 0, None)
    assert rc == -1 and b"bf16 only" in lib.pnfx_last_error()


@pytest.mark.parametrize("B,H,N,D", [(4, 16, 8192, 64), (8, 8, 4096, 128), (1, 3, 520, 128),
                                     (2, 4, 1000, 32), (1, 1, 70000, 16)])
def test_backward_workspace_holds_only_what_the_kernels_use(B, H, N, D):
    """The backward workspace is the sum of its parts, each rounded up to 256 bytes: eight fp32
    row-constant planes, one fp64 tau partial per dQ wave (32 rows per wave for d <= 64, 16 at
    d = 128, four waves per workgroup), the bf16 copy Q 2^-e, one activity byte per 64-key tile,
    and the activity/tie map (a byte per 32-row group and 64-key tile) only where the dQ kernel
    writes it: d <= 64 and N <= 65536.  At d = 128 (16 rows per dQ wave) no map bytes are held,
    which keeps C5 well inside the no-allocation entry point's scratch."""
    r = lambda x: (x + 255) // 256 * 256  # noqa: E731
    rows_per_wg = 128 if D <= 64 else 64
    want = (r(B * H * N * 8 * 4) + r(B * H * -(-N // rows_per_wg) * 4 * 8) + r(B * H * N * D * 2)
            + r(B * H * -(-N // 64)))
    if D <= 64 and N <= 65536:
        want += r(B * H * -(-N // 32) * -(-N // 64))
    lib = _lib.lib()
    assert lib.pnfx_flash_bwd_workspace_size(B, H, N, D) == want
    if (B, H, N, D) == (8, 8, 4096, 128):
        assert want < _lib.PNFX_NOALLOC_SCRATCH_BYTES


def test_hip_ops_refuse_cpu_tensors():
    from paper_01_anti_decoy_pnfirtau_amd import ops  # noqa: F401

    q = torch.randn(1, 1, 8, 16)
    with pytest.raises(Exception):
        torch.ops.pnfx.flash_fwd(q, q, q, torch.tensor(0.0), 0.25, 0.5, True, True, False, False)
    with pytest.raises(RuntimeError):
        P.flash_pn_fir_tau_attention(q, q, q, torch.tensor(0.0))


def test_wikilm_variants_share_init_and_train_on_cpu():
    """The LM consumer (experiments/exp4_wikitext2_lm.py:183-247) builds the same weights for
    every attention variant from one seed and ties the head to the embedding.  Off-GPU the
    row-fused variant takes the eager path, so its training steps agree exactly with the eager
    model's; the flash variant has no CPU route (as in the reference) and raises."""
    from paper_01_anti_decoy_pnfirtau_amd.wikilm import WikiLM, WikiLMConfig, make_optimizer, train_step

    cfg = WikiLMConfig(d_model=32, n_heads=4, n_layers=2, d_ff=64, max_seq=32, dropout=0.0)
    x = torch.randint(0, 50, (2, 32), generator=torch.Generator().manual_seed(0))
    losses, states = {}, {}
    for variant in ("pn_fir_tau", "pn_fir_tau_triton", "pn_fir_tau_flash"):
        torch.manual_seed(0)
        m = WikiLM(50, cfg, variant)
        assert m.head.weight is m.embed.weight
        states[variant] = {k: v.clone() for k, v in m.state_dict().items()}
        opt = make_optimizer(m, cfg)
        if variant == "pn_fir_tau_flash":
            with pytest.raises(RuntimeError, match="GPU only"):
                train_step(m, opt, x, amp=False)
            continue
        losses[variant] = [float(train_step(m, opt, x, amp=False)) for _ in range(2)]
    ref = states["pn_fir_tau"]
    for variant, st in states.items():
        assert st.keys() == ref.keys()
        for k in ref:
            assert torch.equal(st[k], ref[k]), (variant, k)
    assert losses["pn_fir_tau_triton"] == losses["pn_fir_tau"]
    assert losses["pn_fir_tau"][1] < losses["pn_fir_tau"][0]
    with pytest.raises(ValueError):
        WikiLM(50, cfg, "softmax")


def test_flash_op_checks_operand_agreement_on_the_host():
    """k and v of another shape, dtype or device than q are refused before any kernel is
    called (the kernels read all three with q's element size and extents)."""
    from paper_01_anti_decoy_pnfirtau_amd import ops

    q = torch.randn(1, 2, 8, 16)
    ops._check_qkv(q, q.clone(), q.clone())
    with pytest.raises(TypeError):
        ops._check_qkv(q, q.to(torch.bfloat16), q)
    with pytest.raises(ValueError):
        ops._check_qkv(q, q, q[:, :, :4])
    with pytest.raises(ValueError):
        ops._check_qkv(q, q.to("meta"), q)


def test_fake_kernels_give_the_output_layouts():
    """Under FakeTensorMode (what torch.compile traces with) every pnfx op returns tensors of
    the real kernels' shapes, dtypes and memory order without touching a device: O as
    [B, H, N, D] or, with o_bnhd, as a [B, H, N, D] view of [B, N, H, D] rows; M and Z fp32
    [B, H, N]; Nmax int32 only when asked for; the tile mask [B*H, ceil(N/32), ceil(N/64)];
    the backward's gradients contiguous and dtau one fp32; the FIR and row ops shape-true."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from paper_01_anti_decoy_pnfirtau_amd import ops  # noqa: F401  (registers the fakes)

    B, H, N, D = 2, 3, 100, 64
    with FakeTensorMode(allow_non_fake_inputs=True):
        q = torch.empty(B, H, N, D, dtype=torch.bfloat16, device="cuda")
        tau = torch.empty((), device="cuda")
        o, o_lo, M, Z, Nm, mask = torch.ops.pnfx.flash_fwd(q, q, q, tau, 0.125, 0.5, True,
                                                           True, False, True)
        assert o.shape == o_lo.shape == (B, H, N, D) and o.is_contiguous()
        assert M.shape == Z.shape == (B, H, N) and M.dtype == Z.dtype == torch.float32
        assert Nm.shape == (B, H, N) and Nm.dtype == torch.int32
        assert mask.shape == (B * H, 4, 2) and mask.dtype == torch.uint8
        ob = torch.ops.pnfx.flash_fwd(q, q, q, tau, 0.125, 0.5, True, True, True, False)
        assert ob[0].shape == (B, H, N, D) and ob[0].transpose(1, 2).is_contiguous()
        assert ob[4].numel() == 0  # no tie counts unless asked for
        dq, dk, dv, dt = torch.ops.pnfx.flash_bwd(q, q, q, tau, o, o_lo, o, M, Z, mask, 0.125,
                                                  0.5, True, True)
        assert dq.shape == dk.shape == dv.shape == (B, H, N, D) and dq.is_contiguous()
        assert dt.shape == (1,) and dt.dtype == torch.float32
        f = torch.ops.pnfx.flash_fwd_fir(q, q, q, tau, torch.empty(7, device="cuda"), 0.125,
                                         0.5, True, True)
        assert [t.shape for t in f] == [(B, H, N, D)] * 2 + [(B, H, N)] * 2 + [(B * H, 4, 2)]
        x = torch.empty(B, N, 192, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.pnfx.fir_fwd(x, torch.empty(7, device="cuda")).shape == x.shape
        raw = torch.empty(B, H, N, N, device="cuda")
        w, Mr, Zr, Nr = torch.ops.pnfx.pn_rows_fwd(raw, tau, 0.125, 10.0, 0.5, True, True)
        assert w.shape == raw.shape and Mr.shape == Zr.shape == Nr.shape == (B * H * N,)
        d_raw, dtr = torch.ops.pnfx.pn_rows_bwd(w, raw, tau, Mr, Zr, Nr, 0.125, 10.0, 0.5, True,
                                                True)
        assert d_raw.shape == raw.shape and dtr.shape == (B * H * N,)


def test_tile_mask_shape_and_its_length_limit():
    """The forward's silence map is [B*H, ceil(N/32), ceil(N/64)] bytes -- N^2/2048 per (b, h) --
    and is not formed past MASK_MAX_N (the backward then recomputes every tile)."""
    from paper_01_anti_decoy_pnfirtau_amd import ops

    assert ops._mask_shape(2, 3, 100) == (6, 4, 2)
    assert ops._mask_shape(1, 1, ops.MASK_MAX_N) == (1, ops.MASK_MAX_N // 32, ops.MASK_MAX_N // 64)
    assert ops._mask_shape(1, 1, ops.MASK_MAX_N + 1) == (0, 0, 0)


@pytest.mark.parametrize("K", [1, 5, 7])
def test_fir_entry_point_takes_eager_path_on_cpu(K):
    """triton_causal_fir on a CPU tensor is the eager causal_fir (src/triton_pnfirtau.py:687-691),
    bit for bit the reference's golden for K = 7 in fp32 and bf16."""
    from paper_01_anti_decoy_pnfirtau_amd.hip_pnfirtau import triton_causal_fir

    f = golden("fir_eager")
    taps = {1: _t(f["taps1"]), 5: _t(f["taps5"]), 7: _t(f["taps"])}[K]
    for x in (_t(f["x"]), _t(f["x_bf16"])):
        assert torch.equal(triton_causal_fir(x, taps), P.causal_fir(x, taps))
    if K == 7:
        assert torch.equal(triton_causal_fir(_t(f["x"]), taps), _t(f["y_f32"]))
        assert torch.equal(triton_causal_fir(_t(f["x_bf16"]), taps).view(torch.int16),
                           _t(f["y_bf16"]).view(torch.int16))


def test_missing_libraries_fail_loudly(monkeypatch):
    """The product path has no fallback: without libpnfx.so (the C ABI) or _pnfx_torch.so (the
    operator registration) loading raises PnfxError instead of running anything else."""
    from paper_01_anti_decoy_pnfirtau_amd import _lib, ops
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libpnfx.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.PnfxError, match="not built"):
        _lib.lib()
    monkeypatch.undo()
    monkeypatch.setattr(ops, "TORCH_OPS_PATH", "/nonexistent/_pnfx_torch.so")
    with pytest.raises(_lib.PnfxError, match="not built"):
        ops._load()
