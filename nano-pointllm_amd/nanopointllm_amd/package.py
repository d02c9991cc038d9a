"""Quantized linear tensor package, schema 1.0 (byte-compatible reader/writer).

On-disk format of ``nanopointllm/compression/quantized_tensor_package.py``
(write :46-140, load :143-186, validation :189-213): a directory holding
row-major little-endian payload files and a ``metadata.json`` manifest with
``schema_version "1.0"``, ``package_type``, ``shape {m, n, k}``,
``numerical_contract`` and, per tensor, ``{file, dtype, shape, order,
bytes, sha256}``.  The manifest is written with ``indent=2, sort_keys=True``
and a trailing newline so a package written here hashes identically to one
written by the reference.

The per-token variant (``PACKAGE_TYPE_PER_TOKEN``) keeps every file and key
and stores one activation scale per row.  Host-side file I/O only (numpy +
hashlib); :func:`to_device_weight` hands the int8 weight to the GPU kernels.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

SCHEMA_VERSION = "1.0"
PACKAGE_TYPE = "smoothquant_static_a8_per_output_w8_linear"
# Per-token variant: the same files, with activation_scale.fp16 holding one
# scale per activation row ([m]) - the dynamic per-token contract
# (w8a8.py:106-115) that the reference's package cannot express.
PACKAGE_TYPE_PER_TOKEN = "smoothquant_dynamic_per_token_a8_per_output_w8_linear"

_FILES = {
    "activation": "activation.int8",
    "weight": "weight.int8",
    "activation_scale": "activation_scale.fp16",
    "weight_scale": "weight_scale.fp16",
    "smooth_scale": "smooth_scale.fp16",
    "output_scale": "output_scale.fp16",
    "bias": "bias.fp16",
}
_REQUIRED = ("activation", "weight", "activation_scale", "weight_scale", "smooth_scale")
_NUMERICAL_CONTRACT = {
    "activation": "symmetric_per_tensor_int8[-127,127]",
    "weight": "symmetric_per_output_int8[-127,127]",
    "scale_storage": "IEEE754_binary16_little_endian",
    "accumulator": "signed_int32",
    "rounding": "round_to_nearest_ties_to_even",
    "layout": "row_major",
}
_I8 = np.dtype("i1")
_F16 = np.dtype("<f2")


@dataclass(frozen=True)
class QuantizedLinearTensors:
    """Validated contents of one package (``QuantizedLinearTensors``, :16-43)."""

    activation: np.ndarray
    weight: np.ndarray
    activation_scale: np.ndarray
    weight_scale: np.ndarray
    smooth_scale: np.ndarray
    output_scale: np.ndarray | None
    bias: np.ndarray | None
    metadata: dict[str, Any]

    @property
    def m(self) -> int:
        return int(self.activation.shape[0])

    @property
    def n(self) -> int:
        return int(self.weight.shape[0])

    @property
    def k(self) -> int:
        return int(self.weight.shape[1])

    @property
    def per_token(self) -> bool:
        return self.metadata.get("package_type") == PACKAGE_TYPE_PER_TOKEN

    def output_golden(self) -> np.ndarray:
        """The binary32 linear output of the package's integer contract:
        ``f32(acc) * s_a * s_w (+ bias)`` with s_a per tensor or per row."""
        acc = self.integer_golden().astype(np.float32)
        sa = self.activation_scale.astype(np.float32)
        out = acc * (sa[:, None] if self.per_token else sa[0])
        out = out * self.weight_scale.astype(np.float32)[None, :]
        if self.bias is not None:
            out = out + self.bias.astype(np.float32)[None, :]
        return out.astype(np.float32)

    def integer_golden(self) -> np.ndarray:
        """Host int32 accumulators ``activation @ weight.T`` (exact)."""
        a = self.activation.astype(np.int64)
        w = self.weight.astype(np.int64)
        return (a @ w.T).astype(np.int32)


def _as_array(values, dtype: np.dtype, name: str, ndim: int) -> np.ndarray:
    arr = np.asarray(values)
    if arr.ndim != ndim:
        raise ValueError(f"{name} must have {ndim} dimensions")
    if not np.all(np.isfinite(arr)):
        raise ValueError(f"{name} contains non-finite values")
    return np.ascontiguousarray(arr.astype(dtype, copy=False))


def write_quantized_linear_package(directory, *, activation, weight, activation_scale,
                                   weight_scale, smooth_scale, output_scale=None, bias=None,
                                   provenance: dict[str, Any] | None = None,
                                   per_token: bool = False) -> dict[str, Any]:
    """Write a schema-1.0 package and return its manifest.

    ``per_token`` writes the per-token variant (``PACKAGE_TYPE_PER_TOKEN``):
    ``activation_scale`` then holds one scale per activation row."""
    root = Path(directory)
    root.mkdir(parents=True, exist_ok=True)
    act = _as_array(activation, _I8, "activation", 2)
    wgt = _as_array(weight, _I8, "weight", 2)
    if act.shape[1] != wgt.shape[1]:
        raise ValueError("activation and weight K dimensions differ")
    a_scale = _as_array(np.asarray(activation_scale).reshape(-1), _F16, "activation_scale", 1)
    if per_token and a_scale.shape != (act.shape[0],):
        raise ValueError("activation_scale must contain one FP16 value per activation row")
    if not per_token and a_scale.shape != (1,):
        raise ValueError("activation_scale must contain exactly one FP16 value")
    w_scale = _as_array(weight_scale, _F16, "weight_scale", 1)
    s_scale = _as_array(smooth_scale, _F16, "smooth_scale", 1)
    if w_scale.shape != (wgt.shape[0],):
        raise ValueError("weight_scale must contain one value per output")
    if s_scale.shape != (wgt.shape[1],):
        raise ValueError("smooth_scale must contain one value per input channel")
    if np.any(a_scale <= 0) or np.any(w_scale <= 0):
        raise ValueError("quantization scales must be positive")
    if np.any(s_scale <= 0):
        raise ValueError("SmoothQuant scales must be positive")
    arrays: dict[str, np.ndarray] = {
        "activation": act, "weight": wgt, "activation_scale": a_scale,
        "weight_scale": w_scale, "smooth_scale": s_scale,
    }
    if output_scale is not None:
        o_scale = _as_array(np.asarray(output_scale).reshape(-1), _F16, "output_scale", 1)
        if o_scale.shape != (1,) or np.any(o_scale <= 0):
            raise ValueError("output_scale must contain one positive FP16 value")
        arrays["output_scale"] = o_scale
    if bias is not None:
        b = _as_array(bias, _F16, "bias", 1)
        if b.shape != (wgt.shape[0],):
            raise ValueError("bias must contain one value per output")
        arrays["bias"] = b

    entries = {}
    for name, arr in arrays.items():
        payload = arr.tobytes(order="C")
        (root / _FILES[name]).write_bytes(payload)
        entries[name] = {
            "file": _FILES[name],
            "dtype": arr.dtype.str,
            "shape": list(arr.shape),
            "order": "C",
            "bytes": len(payload),
            "sha256": hashlib.sha256(payload).hexdigest(),
        }
    manifest = {
        "schema_version": SCHEMA_VERSION,
        "package_type": PACKAGE_TYPE_PER_TOKEN if per_token else PACKAGE_TYPE,
        "shape": {"m": int(act.shape[0]), "n": int(wgt.shape[0]), "k": int(wgt.shape[1])},
        "numerical_contract": _contract(per_token),
        "tensors": entries,
        "provenance": provenance or {},
    }
    (root / "metadata.json").write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n",
                                        encoding="utf-8")
    return manifest


def _contract(per_token: bool) -> dict[str, str]:
    contract = dict(_NUMERICAL_CONTRACT)
    if per_token:
        contract["activation"] = "symmetric_per_token_int8[-127,127]"
    return contract


def _read_entry(root: Path, name: str, entry: dict[str, Any]) -> np.ndarray:
    payload = (root / entry["file"]).read_bytes()
    if len(payload) != int(entry["bytes"]):
        raise ValueError(f"{name} byte count mismatch")
    if hashlib.sha256(payload).hexdigest() != entry["sha256"]:
        raise ValueError(f"{name} SHA256 mismatch")
    dtype = np.dtype(entry["dtype"])
    shape = tuple(int(v) for v in entry["shape"])
    if int(np.prod(shape, dtype=np.int64)) * dtype.itemsize != len(payload):
        raise ValueError(f"{name} metadata size mismatch")
    return np.frombuffer(payload, dtype=dtype).reshape(shape).copy()


def load_quantized_linear_package(directory) -> QuantizedLinearTensors:
    """Load a package, verifying every checksum and shape before returning."""
    root = Path(directory)
    manifest = json.loads((root / "metadata.json").read_text(encoding="utf-8"))
    if manifest.get("schema_version") != SCHEMA_VERSION:
        raise ValueError("unsupported quantized tensor package schema")
    package_type = manifest.get("package_type", PACKAGE_TYPE)
    if package_type not in (PACKAGE_TYPE, PACKAGE_TYPE_PER_TOKEN):
        raise ValueError(f"unsupported quantized tensor package type: {package_type}")
    per_token = package_type == PACKAGE_TYPE_PER_TOKEN
    entries = manifest.get("tensors", {})
    missing = sorted(set(_REQUIRED) - set(entries))
    if missing:
        raise ValueError(f"quantized tensor package is missing {missing}")
    arrays = {name: _read_entry(root, name, entry) for name, entry in entries.items()}
    shape = manifest.get("shape", {})
    m, n, k = int(shape["m"]), int(shape["n"]), int(shape["k"])
    if arrays["activation"].shape != (m, k):
        raise ValueError("activation shape does not match package shape")
    if arrays["weight"].shape != (n, k):
        raise ValueError("weight shape does not match package shape")
    if arrays["activation_scale"].shape != ((m,) if per_token else (1,)):
        raise ValueError("activation_scale shape must be [m]" if per_token
                         else "activation_scale shape must be [1]")
    if arrays["weight_scale"].shape != (n,):
        raise ValueError("weight_scale shape does not match N")
    if arrays["smooth_scale"].shape != (k,):
        raise ValueError("smooth_scale shape does not match K")
    output_scale = arrays.get("output_scale")
    bias = arrays.get("bias")
    if output_scale is not None and output_scale.shape != (1,):
        raise ValueError("output_scale shape must be [1]")
    if bias is not None and bias.shape != (n,):
        raise ValueError("bias shape does not match N")
    return QuantizedLinearTensors(
        activation=arrays["activation"], weight=arrays["weight"],
        activation_scale=arrays["activation_scale"], weight_scale=arrays["weight_scale"],
        smooth_scale=arrays["smooth_scale"], output_scale=output_scale, bias=bias,
        metadata=manifest,
    )


def to_device_weight(package: QuantizedLinearTensors, device="cuda"):
    """Pack the package's int8 weight and scales for the GPU kernels."""
    import torch

    from .linear import PackedW8A8Weight

    q = torch.from_numpy(package.weight).to(device)
    s = torch.from_numpy(package.weight_scale.astype(np.float32)).to(device)
    b = None if package.bias is None else torch.from_numpy(
        package.bias.astype(np.float32)).to(device)
    return PackedW8A8Weight.from_int8(q, s, b)


def package_integer_golden_gpu(package: QuantizedLinearTensors, device="cuda"):
    """int32 accumulators of the package computed by the HIP GEMM/GEMV."""
    import torch

    from . import w8a8

    w = to_device_weight(package, device)
    a = torch.from_numpy(package.activation).to(device)
    return w8a8.gemm_i32(a, w.packed, package.n)
