"""MI355X (gfx950) W8A8 quantized linear path for nanopointllm.

Public surface:

* :mod:`nanopointllm_amd.w8a8` - the ``nanopointllm.compression.w8a8``
  contract functions executed by HIP kernels (quantize / scale / QDQ /
  integer linear) plus the low-level fused linear entry points.
* :mod:`nanopointllm_amd.linear` - ``W8A8Linear``, ``W8A8PackedQKV``,
  ``W8A8GateUpSiluMul`` and ``W8A8MLP`` modules for the lightweight runner's
  projection call sites.
* :mod:`nanopointllm_amd.package` - schema-1.0 quantized tensor package
  (per-tensor and per-token variants).
* :mod:`nanopointllm_amd.weight_cache` - offline cache of quantized, packed
  weights with checksums.
* :mod:`nanopointllm_amd.inject` - swaps the dense projections of a LLaMA
  model for the W8A8 modules, plus the packed call-site helpers.
* :mod:`nanopointllm_amd.runner` - a decoder stack in the shape of
  ``LightweightLlamaRunner`` on the W8A8 modules, capturable in a HIP graph.
* :mod:`nanopointllm_amd.calibration` - activation range collection, QDQ
  hooks, weight fake-quant and SmoothQuant smoothing.
* :mod:`nanopointllm_amd.integer_epilogues` - the int32 -> int8
  multiplier/shift requant and int32 -> bf16 single-rounding dequant of the
  reference's accelerator model.

All GPU work goes through ``libw8a8_gfx950.so`` (C ABI in
``include/w8a8_gfx950.h``); there is no CPU or torch fallback.
"""
from . import _lib
from ._lib import LIB_PATH

__all__ = ["LIB_PATH", "load_library"]


def load_library():
    """Load ``libw8a8_gfx950.so`` (raises ``RuntimeError`` if it is missing)."""
    return _lib.load()
