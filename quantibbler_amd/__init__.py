"""quantibbler_amd -- MI355X (gfx950) implementation of quantibbler-kernels'
two hot paths behind the reference's own API surface:

* the binary latent-factor linear (decode GEMV, prefill GEMM) over 1-bit
  sign matrices: ``FactorLayer`` / ``FactorSet`` and the packed products of
  ``kernels`` (the ``quantibbler_kernels`` PyO3 names);
* SageAttention: ``GpuContext.attention_sage`` (the reference's [SA] s4
  scheme) and ``GpuContext.attention_sage_blk_dev`` (block-scaled INT8 Q/K,
  fp16 P.V).

All compute runs in libqbk.so (hand-written HIP, C ABI in include/qbk.h).
"""
from ._lib import DeviceError, InitError, KernelError, load as _load_lib  # noqa: F401
from .gpu import (AttentionShape, DecoderBlock, FactorLayer, FactorSet, GpuContext,  # noqa: F401
                  LmHead, SageDecodeState, gpu_available)

_load_lib()

__version__ = "0.1.0"
