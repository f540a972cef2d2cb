"""The diagnostic pipe probe (pnfx_probe_pipe_overlap) runs and reports three timings."""
import ctypes
import math

import pytest
import torch

from paper_01_anti_decoy_pnfirtau_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("waves,big", [(1, 0), (2, 1)])
def test_pipe_probe_reports_three_timings(dev, waves, big):
    print(f"[pipe probe waves={waves} big={big}]", flush=True)
    L = _lib.lib()
    out = torch.empty(256 * 512, device=dev)
    ms = (ctypes.c_float * 3)()
    _lib.check(L.pnfx_probe_pipe_overlap(waves, big, 8, 32, 200, out.data_ptr(), ms,
                                         torch.cuda.current_stream().cuda_stream),
               "pnfx_probe_pipe_overlap")
    assert all(math.isfinite(ms[i]) and ms[i] > 0 for i in range(3))
    # both streams together take at least as long as the longer one alone (loose: timing noise)
    assert ms[2] > 0.5 * max(ms[0], ms[1])
    assert torch.isfinite(out).all()
