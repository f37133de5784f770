"""MI355X-native token sampling for Chenxing.

The sampler (``chenxing/core/sampler.py``) and the speculative-decoding verify
step (``chenxing/engine/speculative.py:145-171``) run as fused HIP kernels for
gfx950 behind a C-ABI (``include/cx_sampler.h``); this package is the Python
host side with the reference's call signatures.
"""
from .params import SamplingParams, RowParams

__all__ = ["SamplingParams", "RowParams", "Sampler", "SpeculativeDecoder",
           "decode_step_batched", "scheduler_step_batched"]


def __getattr__(name):
    if name == "Sampler":
        from .sampler import Sampler
        return Sampler
    if name == "SpeculativeDecoder":
        from .speculative import SpeculativeDecoder
        return SpeculativeDecoder
    if name in ("decode_step_batched", "scheduler_step_batched"):
        from . import decode
        return getattr(decode, name)
    raise AttributeError(name)
