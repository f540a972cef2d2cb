"""torch.library.opcheck over the C++-registered pnfx operators: the schema's mutation and
aliasing claims, the autograd registration, the fake (meta) kernels against the real
kernels' outputs, and tracing through AOTAutograd with dynamic shapes -- what torch.compile
relies on.  Small shapes; bf16 and fp32."""
import pytest
import torch

from paper_01_anti_decoy_pnfirtau_amd import ops  # noqa: F401  (loads the ops and fakes)
from tests.helpers import seeded

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_opcheck_flash_forward_and_backward(dev, dtype):
    B, H, N, D = 1, 2, 80, 64
    q, k, v, dO = (seeded((B, H, N, D), 300 + i, dtype, dev) for i in range(4))
    tau = torch.tensor(0.05, device=dev)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    torch.library.opcheck(torch.ops.pnfx.flash_fwd.default,
                          (qg, kg, vg, tau, 0.125, 0.5, True, True, False, False))
    torch.library.opcheck(torch.ops.pnfx.flash_fwd.default,
                          (q, k, v, tau, 0.125, 0.5, True, True, True, True))
    o, o_lo, M, Z, _, mask = torch.ops.pnfx.flash_fwd(q, k, v, tau, 0.125, 0.5, True, True,
                                                      False, False)
    torch.library.opcheck(torch.ops.pnfx.flash_bwd.default,
                          (q, k, v, tau, o, o_lo, dO, M, Z, mask, 0.125, 0.5, True, True))


def test_opcheck_fused_fir_forward(dev):
    B, H, N, D = 2, 2, 90, 32
    q, kr, v = (seeded((B, H, N, D), 310 + i, torch.bfloat16, dev) for i in range(3))
    taps = torch.rand(7, device=dev)
    tau = torch.tensor(0.0, device=dev)
    torch.library.opcheck(torch.ops.pnfx.flash_fwd_fir.default,
                          (q, kr, v, tau, taps, D ** -0.5, 0.5, True, True, False))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_opcheck_fir_and_row_scores(dev, dtype):
    x = seeded((2, 70, 48), 320, dtype, dev).requires_grad_(True)
    taps = torch.rand(7, device=dev)
    torch.library.opcheck(torch.ops.pnfx.fir_fwd.default, (x, taps))
    torch.library.opcheck(torch.ops.pnfx.fir_bwd.default, (x.detach(), taps))
    raw = seeded((1, 2, 40, 40), 321, dtype, dev).requires_grad_(True)
    tau = torch.tensor(0.1, device=dev)
    torch.library.opcheck(torch.ops.pnfx.pn_rows_fwd.default,
                          (raw, tau, 0.125, 10.0, 0.5, True, True))
    w, M, Z, Nm = torch.ops.pnfx.pn_rows_fwd(raw.detach(), tau, 0.125, 10.0, 0.5, True, True)
    torch.library.opcheck(torch.ops.pnfx.pn_rows_bwd.default,
                          (torch.randn_like(w), raw.detach(), tau, M, Z, Nm, 0.125, 10.0, 0.5,
                           True, True))


def test_tau_on_the_host_is_moved_to_the_device(dev):
    """The kernels read tau on the device: a CPU (or bf16) tau tensor is brought to the
    operands' device as fp32 by the op, and its gradient comes back on tau's own device."""
    B, H, N, D = 1, 2, 70, 64
    q, k, v, dO = (seeded((B, H, N, D), 330 + i, torch.bfloat16, dev) for i in range(4))
    outs = []
    for tau in (torch.tensor(0.05, device=dev), torch.tensor(0.05), torch.tensor(0.05).bfloat16()):
        t = tau.clone().requires_grad_(True)
        o = torch.ops.pnfx.flash_fwd(q, k, v, t, 0.125, 0.5, True, True, False, False)[0]
        o.backward(dO)
        assert t.grad.device == tau.device and t.grad.dtype == tau.dtype
        outs.append((o, float(t.grad)))
    for o, g in outs[1:2]:  # a CPU fp32 tau: exactly the device result
        assert torch.equal(o, outs[0][0]) and g == outs[0][1]
    # bf16 tau: 0.05 rounds to bf16, so only closeness
    assert torch.allclose(outs[2][0].float(), outs[0][0].float(), atol=2e-2, rtol=2e-2)


def test_inference_call_skips_the_graph_and_matches(dev):
    """With grad mode off (or no input requiring a gradient) the op runs below autograd
    without a graph node: outputs carry no grad_fn and equal those of the recorded call."""
    B, H, N, D = 1, 2, 96, 64
    q, k, v = (seeded((B, H, N, D), 340 + i, torch.bfloat16, dev) for i in range(3))
    tau = torch.tensor(0.02, device=dev)
    qg = q.clone().requires_grad_(True)
    rec = torch.ops.pnfx.flash_fwd(qg, k, v, tau, 0.125, 0.5, True, True, False, False)
    assert rec[0].grad_fn is not None
    with torch.no_grad():
        inf = torch.ops.pnfx.flash_fwd(qg, k, v, tau, 0.125, 0.5, True, True, False, False)
    plain = torch.ops.pnfx.flash_fwd(q, k, v, tau, 0.125, 0.5, True, True, False, False)
    for outs in (inf, plain):
        assert all(not t.requires_grad and t.grad_fn is None for t in outs)
        assert all(torch.equal(a, b) for a, b in zip(outs, rec))
    x = seeded((2, 50, 32), 343, torch.bfloat16, dev)
    taps = torch.rand(7, device=dev)
    y_rec = torch.ops.pnfx.fir_fwd(x.clone().requires_grad_(True), taps)
    with torch.no_grad():
        y_inf = torch.ops.pnfx.fir_fwd(x, taps)
    assert y_rec.grad_fn is not None and y_inf.grad_fn is None and torch.equal(y_rec, y_inf)
    raw = seeded((1, 2, 40, 40), 344, torch.bfloat16, dev)
    with torch.inference_mode():
        w_inf = torch.ops.pnfx.pn_rows_fwd(raw, tau, 0.125, 10.0, 0.5, True, True)
    w_rec = torch.ops.pnfx.pn_rows_fwd(raw.clone().requires_grad_(True), tau, 0.125, 10.0, 0.5,
                                       True, True)
    assert w_rec[0].grad_fn is not None and w_inf[0].grad_fn is None
    assert all(torch.equal(a, b) for a, b in zip(w_inf, w_rec))


def test_backward_ops_refuse_statistics_of_another_shape(dev):
    """The backward ops index the forward's statistics and tile mask by row: tensors of
    another size, type or layout are refused on the host, before any launch."""
    B, H, N, D = 1, 2, 96, 64
    q, k, v, dO = (seeded((B, H, N, D), 350 + i, torch.bfloat16, dev) for i in range(4))
    tau = torch.tensor(0.0, device=dev)
    o, o_lo, M, Z, _, mask = torch.ops.pnfx.flash_fwd(q, k, v, tau, 0.125, 0.5, True, True,
                                                      False, False)
    bwd = torch.ops.pnfx.flash_bwd

    def call(M_=M, Z_=Z, mask_=mask):
        return bwd(q, k, v, tau, o, o_lo, dO, M_, Z_, mask_, 0.125, 0.5, True, True)

    ref = call()
    with pytest.raises(ValueError, match="M must be"):
        call(M_=M[..., :-1].contiguous())
    with pytest.raises(TypeError, match="Z is"):
        call(Z_=Z.double())
    with pytest.raises(ValueError, match="M must be"):
        call(M_=M.transpose(1, 2).contiguous().transpose(1, 2))  # right size, not contiguous
    with pytest.raises(ValueError, match="mask must be"):
        call(mask_=mask[:, :-1].contiguous())
    # no mask at all is allowed (every causal tile recomputed), with the same results
    assert all(torch.equal(a, b) for a, b in zip(call(mask_=mask[:0]), ref))
    raw = seeded((1, 2, 40, 40), 355, torch.bfloat16, dev)
    w, Mr, Zr, Nm = torch.ops.pnfx.pn_rows_fwd(raw, tau, 0.125, 10.0, 0.5, True, True)
    rbwd = torch.ops.pnfx.pn_rows_bwd
    with pytest.raises(TypeError, match="Nmax is"):
        rbwd(torch.ones_like(w), raw, tau, Mr, Zr, Nm.float(), 0.125, 10.0, 0.5, True, True)
    with pytest.raises(ValueError, match="dw has shape"):
        rbwd(torch.ones_like(w)[..., :-1], raw, tau, Mr, Zr, Nm, 0.125, 10.0, 0.5, True, True)


@pytest.mark.parametrize("training", [True, False])
def test_module_compiles_without_graph_breaks(dev, training):
    """PnFirTauFlashMHA under torch.compile (AOTAutograd, no code generation) traces the pnfx
    ops into one graph, and the compiled forward (and backward) give the eager results."""
    from paper_01_anti_decoy_pnfirtau_amd import PnFirConfig, PnFirTauFlashMHA
    torch.manual_seed(7)
    m = PnFirTauFlashMHA(PnFirConfig(d_model=64, n_heads=4)).to(dev).bfloat16()
    with torch.no_grad():
        m.score_tau.fill_(0.05)
    x = seeded((2, 96, 64), 360, torch.bfloat16, dev)
    torch._dynamo.reset()
    cm = torch.compile(m, backend="aot_eager", fullgraph=True, dynamic=False)
    if training:
        outs = []
        for f in (m, cm):
            xg = x.clone().requires_grad_(True)
            m.zero_grad(set_to_none=True)
            y = f(xg)
            y.float().square().sum().backward()
            outs.append((y, xg.grad, m.qkv.weight.grad, m.score_tau.grad))
        for a, b in zip(*outs):
            assert torch.equal(a, b)
    else:
        with torch.no_grad():
            assert torch.equal(m(x), cm(x))


def test_backward_gradients_follow_the_inputs_dimension_order(dev):
    """For q/k/v that are head views of [B,N,H*D] rows (as the modules split a qkv projection)
    the gradients come back as views of [B,N,H,D] memory, so that merging their heads is free;
    values are those of the contiguous call, and opcheck holds the fake kernel to the layout."""
    B, H, N, D = 2, 4, 80, 32
    qkv = seeded((B, N, 3, H, D), 370, torch.bfloat16, dev)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    dO = seeded((B, H, N, D), 374, torch.bfloat16, dev)
    tau = torch.tensor(0.01, device=dev)
    fwd = torch.ops.pnfx.flash_fwd(q, k, v, tau, D ** -0.5, 0.5, True, True, False, False)
    o, o_lo, M, Z, _, mask = fwd
    args = (o, o_lo, dO, M, Z, mask, D ** -0.5, 0.5, True, True)
    grads = torch.ops.pnfx.flash_bwd(q, k, v, tau, *args)
    qc, kc, vc = (t.contiguous() for t in (q, k, v))
    ref = torch.ops.pnfx.flash_bwd(qc, kc, vc, tau, *args)
    for g, r in zip(grads[:3], ref[:3]):
        assert g.transpose(1, 2).is_contiguous() and r.is_contiguous()
        assert torch.equal(g, r)
    assert torch.equal(grads[3], ref[3])
    torch.library.opcheck(torch.ops.pnfx.flash_bwd.default, (q, k, v, tau, *args))
