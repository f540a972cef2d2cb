"""pnfx_flash_bwd_noalloc (the backward with the library-held scratch instead of a workspace)
against pnfx_flash_bwd through the C ABI: bitwise the same dQ, dK, dV and dtau on consecutive
calls of decreasing size -- the scratch keeps the previous call's contents, so this also shows
that nothing stale is read -- and a shape past the scratch size is refused."""
import numpy as np
import pytest
import torch

from paper_01_anti_decoy_pnfirtau_amd import _lib, ops
from tests.helpers import seeded

pytestmark = pytest.mark.gpu


def _call(entry, q, k, v, o, o_lo, dO, M, Z, mask, tau, scale, code):
    lib = _lib.lib()
    B, H, N, D = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    dt = torch.empty(1, device=q.device)
    pre = (*ops._ptr4(q), *ops._ptr4(k), *ops._ptr4(v), *ops._ptr4(o),
           o_lo.data_ptr() if o_lo.numel() else None, *ops._ptr4(dO), M.data_ptr(), Z.data_ptr(),
           mask.data_ptr(), *ops._ptr4(dq), *ops._ptr4(dk), *ops._ptr4(dv), dt.data_ptr())
    post = (B, H, N, D, tau.data_ptr(), scale, 0.5, 1, 1, code,
            torch.cuda.current_stream().cuda_stream)
    if entry == "noalloc":
        rc = lib.pnfx_flash_bwd_noalloc(*pre, *post)
    else:
        nbytes = lib.pnfx_flash_bwd_workspace_size(B, H, N, D)
        ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
        rc = lib.pnfx_flash_bwd(*pre, ws.data_ptr(), nbytes, *post)
    assert rc == 0, lib.pnfx_last_error()
    torch.cuda.synchronize()
    return dq, dk, dv, dt


# consecutive calls, each smaller than the one before
CALLS = [
    # B, H, N, D, dtype, tau, zeroed 64-key blocks
    (2, 4, 1000, 64, torch.bfloat16, 0.25, (0, 2, 3, 7, 12)),
    (1, 3, 520, 128, torch.bfloat16, 0.0, ()),
    (1, 2, 300, 64, torch.float32, 0.1, (1,)),
    (1, 1, 70, 16, torch.bfloat16, 0.0, ()),
]


def test_noalloc_backward_matches_workspace_backward(dev):
    print("[noalloc]", flush=True)
    for i, (B, H, N, D, dtype, tau_val, blocks) in enumerate(CALLS):
        print(f"[noalloc call {i}: B={B} H={H} N={N} D={D} {dtype}]", flush=True)
        q, k, v, dO = (seeded((B, H, N, D), 200 + 4 * i + j, dtype, dev) for j in range(4))
        for j in blocks:
            k[:, :, 64 * j:64 * j + 64] = 0
        tau = torch.tensor(tau_val, device=dev)
        scale = 1.0 / np.sqrt(D)
        o, o_lo, M, Z, _, mask = torch.ops.pnfx.flash_fwd(q, k, v, tau, scale, 0.5, True, True,
                                                          False, False)
        code = _lib.PNFX_BF16 if dtype == torch.bfloat16 else _lib.PNFX_F32
        want = _call("workspace", q, k, v, o, o_lo, dO, M, Z, mask, tau.reshape(1), scale, code)
        got = _call("noalloc", q, k, v, o, o_lo, dO, M, Z, mask, tau.reshape(1), scale, code)
        for name, a, b in zip(("dq", "dk", "dv", "dtau"), got, want):
            assert torch.equal(a, b), (i, name)
        assert torch.any(got[0] != 0)


def test_noalloc_backward_refuses_shapes_past_its_scratch(dev):
    lib = _lib.lib()
    B, H, N, D = 4, 16, 16384, 64
    need = lib.pnfx_flash_bwd_workspace_size(B, H, N, D)
    assert need > _lib.PNFX_NOALLOC_SCRATCH_BYTES
    assert lib.pnfx_flash_bwd_workspace_size(4, 16, 8192, 64) <= _lib.PNFX_NOALLOC_SCRATCH_BYTES
    p = torch.empty(16, device=dev)
    args = [p.data_ptr(), 0, 0, 0] * 4 + [None] + [p.data_ptr(), 0, 0, 0] + [p.data_ptr()] * 3 \
        + [p.data_ptr(), 0, 0, 0] * 3 + [p.data_ptr()]
    rc = lib.pnfx_flash_bwd_noalloc(*args, B, H, N, D, p.data_ptr(), 0.125, 0.5, 1, 1,
                                    _lib.PNFX_BF16, torch.cuda.current_stream().cuda_stream)
    assert rc == -1 and b"scratch" in lib.pnfx_last_error()
