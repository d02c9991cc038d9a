"""MI355X (gfx950) W8A8 quantized linear path for nanopointllm.

Public surface:

* :mod:`nanopointllm_amd.w8a8` - the ``nanopointllm.compression.w8a8``
  contract functions executed by HIP kernels (quantize / scale / QDQ /
  integer linear) plus the low-level fused linear entry points.
* :mod:`nanopointllm_amd.linear` - ``W8A8Linear``, ``W8A8PackedQKV``,
  ``W8A8GateUpSiluMul`` and ``W8A8MLP`` modules for the lightweight runner's
  projection call sites.
* :mod:`nanopointllm_amd.package` - schema-1.0 quantized tensor package.
* :mod:`nanopointllm_amd.inject` - swaps the dense projections of a LLaMA
  model for the W8A8 modules.

All GPU work goes through ``libw8a8_gfx950.so`` (C ABI in
``include/w8a8_gfx950.h``); there is no CPU or torch fallback.
"""
from . import _lib
from ._lib import LIB_PATH

__all__ = ["LIB_PATH", "load_library"]


def load_library():
    """Load ``libw8a8_gfx950.so`` (raises ``RuntimeError`` if it is missing)."""
    return _lib.load()
