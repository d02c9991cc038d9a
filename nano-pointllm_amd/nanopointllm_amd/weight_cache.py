"""Offline cache of packed W8A8 weights (pre-quantized, pre-packed MFMA tiles).

Quantizing a weight per output row and packing it into 16x64 tiles is
deterministic, so it can be done once and stored.  One cache entry is a
directory in the manifest style of the schema-1.0 tensor package
(``metadata.json`` with ``indent=2, sort_keys=True``; per file ``{file,
dtype, shape, order, bytes, sha256}``):

* ``packed.int8``   - the tiles exactly as ``w8a8_pack_rows`` lays them out:
  tile (rb, kb) of 16 rows x 64 K at byte (rb * ceil(K/64) + kb) * 1024, lane
  slot l = r + 16 g holding row 16 rb + r, k 64 kb + 16 g .. +15 (the register
  image of a ``v_mfma_i32_16x16x64_i8`` operand), zero padded;
* ``scale.fp32``    - per-output scales in packed row order;
* ``bias.fp32``     - optional, in packed row order;
* the manifest records N, K, the row layout (as-is, or gate/up interleaved)
  and, optionally, the sha256 of the source weight so a stale entry is caught.

Every payload's sha256 is checked before anything is uploaded to the GPU.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path
from typing import Any

import numpy as np
import torch

from . import _lib

CACHE_SCHEMA_VERSION = "1.0"
CACHE_TYPE = "w8a8_gfx950_packed_per_output_weight"
TILE_FORMAT = "16x64_int8_tiles_mfma_i32_16x16x64_i8_operand"
_LAYOUTS = {_lib.ROWS_AS_IS: "rows_as_is", _lib.ROWS_INTERLEAVE_HALVES: "gate_up_interleaved"}


def source_sha256(weight: torch.Tensor) -> str:
    """sha256 of a weight's bytes (contiguous, host copy, its own dtype)."""
    t = weight.detach().contiguous().cpu()
    return hashlib.sha256(t.view(torch.uint8).numpy().tobytes()).hexdigest()


def _entry(root: Path, name: str, arr: np.ndarray) -> dict[str, Any]:
    payload = np.ascontiguousarray(arr).tobytes(order="C")
    (root / name).write_bytes(payload)
    return {"file": name, "dtype": arr.dtype.str, "shape": list(arr.shape), "order": "C",
            "bytes": len(payload), "sha256": hashlib.sha256(payload).hexdigest()}


def save_packed_weight(directory, weight, *, source: torch.Tensor | None = None,
                       provenance: dict[str, Any] | None = None) -> dict[str, Any]:
    """Write one :class:`PackedW8A8Weight` and return its manifest."""
    root = Path(directory)
    root.mkdir(parents=True, exist_ok=True)
    tensors = {
        "packed": _entry(root, "packed.int8", weight.packed.detach().cpu().numpy()),
        "scale": _entry(root, "scale.fp32",
                        weight.scale.detach().float().cpu().numpy().astype("<f4")),
    }
    if weight.bias is not None:
        tensors["bias"] = _entry(root, "bias.fp32",
                                 weight.bias.detach().float().cpu().numpy().astype("<f4"))
    manifest = {
        "schema_version": CACHE_SCHEMA_VERSION,
        "cache_type": CACHE_TYPE,
        "tile_format": TILE_FORMAT,
        "row_layout": _LAYOUTS[weight.layout],
        "shape": {"n": int(weight.out_features), "k": int(weight.in_features)},
        "source_sha256": None if source is None else source_sha256(source),
        "tensors": tensors,
        "provenance": provenance or {},
    }
    (root / "metadata.json").write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n",
                                        encoding="utf-8")
    return manifest


def _read(root: Path, name: str, entry: dict[str, Any]) -> np.ndarray:
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


def load_packed_weight(directory, device="cuda", *, source: torch.Tensor | None = None,
                       shape: tuple[int, int] | None = None, layout: int | None = None):
    """Load one cache entry, checking every checksum (and, with ``source``,
    that it was made from that weight) before uploading it.  ``shape`` (N, K)
    and ``layout`` are checked against the manifest first: a cache directory
    reused for a model of other dimensions must not hand out a weight of the
    wrong shape."""
    from .linear import PackedW8A8Weight

    root = Path(directory)
    manifest = json.loads((root / "metadata.json").read_text(encoding="utf-8"))
    if manifest.get("schema_version") != CACHE_SCHEMA_VERSION or \
            manifest.get("cache_type") != CACHE_TYPE or manifest.get("tile_format") != TILE_FORMAT:
        raise ValueError("unsupported packed weight cache entry")
    entry_layout = {v: k for k, v in _LAYOUTS.items()}.get(manifest.get("row_layout"))
    if entry_layout is None:
        raise ValueError("unknown row layout in packed weight cache entry")
    n, k = int(manifest["shape"]["n"]), int(manifest["shape"]["k"])
    if shape is not None and (n, k) != (int(shape[0]), int(shape[1])):
        raise ValueError(f"packed weight cache entry has shape {(n, k)}, expected "
                         f"{(int(shape[0]), int(shape[1]))}")
    if layout is not None and entry_layout != layout:
        raise ValueError("packed weight cache entry has a different row layout")
    layout = entry_layout
    if source is not None:
        if manifest.get("source_sha256") != source_sha256(source):
            raise ValueError("packed weight cache entry was made from a different weight")
    entries = manifest["tensors"]
    packed = _read(root, "packed", entries["packed"])
    scale = _read(root, "scale", entries["scale"])
    bias = _read(root, "bias", entries["bias"]) if "bias" in entries else None
    if packed.dtype != np.int8 or packed.size != int(_lib.load().w8a8_packed_bytes(n, k)):
        raise ValueError("packed tile payload does not match the shape")
    if scale.shape != (n,) or (bias is not None and bias.shape != (n,)):
        raise ValueError("scale/bias must have one value per output")
    return PackedW8A8Weight(
        torch.from_numpy(packed).to(device), torch.from_numpy(scale).float().to(device),
        None if bias is None else torch.from_numpy(bias).float().to(device), n, k, layout)


def cached(directory, key: str, build, *, source: torch.Tensor | None = None,
           verify_source: bool = False, device="cuda", layout: int | None = None):
    """Load ``directory/key`` if it exists, else ``build()`` the packed weight
    and store it there (with the sha256 of ``source``).  A loaded entry's N, K
    must match ``source``'s shape and its row layout ``layout`` (cheap manifest
    checks, always made); ``verify_source`` also checks it against ``source``'s
    sha256 (it hashes the source weight)."""
    entry = Path(directory) / key
    if (entry / "metadata.json").exists():
        shape = None
        if source is not None:
            flat = source.reshape(source.shape[0], -1)
            shape = (int(flat.shape[0]), int(flat.shape[1]))
        return load_packed_weight(entry, device, source=source if verify_source else None,
                                  shape=shape, layout=layout)
    weight = build()
    save_packed_weight(entry, weight, source=source)
    return weight
