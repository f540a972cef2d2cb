"""MI355X-native pn_fir_tau attention hot path (gfx950 HIP kernels behind a C ABI).

Drop-in surface of the reference package (``src/__init__.py`` plus the
accelerated modules of ``src/pnfirtau_attention.py`` and the entry points of
``src/triton_pnfirtau.py``).  Importing the package does not load the HIP
library; the first accelerated call does, and raises if it is not built.
"""
from .pnfirtau_attention import (
    PnFirConfig,
    PnFirTauFlashMHA,
    PnFirTauMHA,
    PnFirTauTritonMHA,
    causal_fir,
    causal_gaussian_taps,
    power_norm_peak_gate,
)

__all__ = [
    "PnFirConfig",
    "PnFirTauMHA",
    "PnFirTauTritonMHA",
    "PnFirTauFlashMHA",
    "causal_fir",
    "causal_gaussian_taps",
    "power_norm_peak_gate",
    "hip_causal_fir",
    "hip_pn_fir_tau_scores",
    "flash_pn_fir_tau_attention",
    "triton_causal_fir",
    "triton_pn_fir_tau_scores",
]


def __getattr__(name):
    # The HIP entry points import torch.library registrations lazily.
    if name in ("hip_causal_fir", "hip_pn_fir_tau_scores", "flash_pn_fir_tau_attention",
                "triton_causal_fir", "triton_pn_fir_tau_scores"):
        from . import hip_pnfirtau

        return getattr(hip_pnfirtau, name)
    raise AttributeError(name)
