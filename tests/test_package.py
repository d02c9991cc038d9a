"""Schema-1.0 quantized tensor package (host I/O), mirroring the reference's
tests/test_quantized_tensor_package.py with its fixture values."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from nanopointllm_amd.package import (
    load_quantized_linear_package, write_quantized_linear_package,
)

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
PKG = GOLDEN["package"]


def _write(path, **override):
    args = dict(
        activation=np.array(PKG["activation"], np.int8),
        weight=np.array(PKG["weight"], np.int8),
        activation_scale=np.array([PKG["activation_scale"]], np.float16),
        weight_scale=np.array(PKG["weight_scale"], np.float16),
        smooth_scale=np.array(PKG["smooth_scale"], np.float16),
        output_scale=np.array([PKG["output_scale"]], np.float16),
        provenance=PKG["provenance"],
    )
    args.update(override)
    return write_quantized_linear_package(path, **args)


def test_round_trip_and_integer_golden(tmp_path):
    _write(tmp_path)
    pkg = load_quantized_linear_package(tmp_path)
    np.testing.assert_array_equal(pkg.activation, np.array(PKG["activation"], np.int8))
    np.testing.assert_array_equal(pkg.weight, np.array(PKG["weight"], np.int8))
    np.testing.assert_array_equal(pkg.integer_golden(),
                                  np.array(PKG["derived_integer_golden"], np.int32))
    meta = json.loads((tmp_path / "metadata.json").read_text())
    assert meta["shape"] == PKG["asserted_shape"]
    assert len(meta["tensors"]["weight"]["sha256"]) == PKG["asserted_sha256_hex_length"]
    assert float(pkg.output_scale[0]) == PKG["output_scale"]
    assert (pkg.m, pkg.n, pkg.k) == (2, 3, 4)


def test_manifest_layout_is_byte_stable(tmp_path):
    manifest = _write(tmp_path)
    text = (tmp_path / "metadata.json").read_text()
    assert text == json.dumps(manifest, indent=2, sort_keys=True) + "\n"
    assert manifest["schema_version"] == "1.0"
    assert manifest["package_type"] == "smoothquant_static_a8_per_output_w8_linear"
    w = manifest["tensors"]["weight"]
    payload = (tmp_path / "weight.int8").read_bytes()
    assert w == {"file": "weight.int8", "dtype": "|i1", "shape": [3, 4], "order": "C",
                 "bytes": 12, "sha256": hashlib.sha256(payload).hexdigest()}
    assert manifest["tensors"]["weight_scale"]["dtype"] == "<f2"
    assert payload == np.array(PKG["weight"], np.int8).tobytes()


def test_rejects_corruption(tmp_path):
    _write(tmp_path)
    path = tmp_path / "weight.int8"
    data = bytearray(path.read_bytes())
    data[0] ^= 1
    path.write_bytes(data)
    with pytest.raises(ValueError, match="SHA256 mismatch"):
        load_quantized_linear_package(tmp_path)


def test_rejects_incompatible_shapes(tmp_path):
    with pytest.raises(ValueError, match="K dimensions differ"):
        write_quantized_linear_package(
            tmp_path, activation=np.ones((1, 4), np.int8), weight=np.ones((3, 8), np.int8),
            activation_scale=1.0, weight_scale=np.ones(3), smooth_scale=np.ones(8))


def test_rejects_bad_scales_and_truncation(tmp_path):
    with pytest.raises(ValueError, match="positive"):
        _write(tmp_path, weight_scale=np.array([0.25, 0.0, 1.0], np.float16))
    with pytest.raises(ValueError, match="exactly one"):
        _write(tmp_path, activation_scale=np.array([1.0, 2.0], np.float16))
    _write(tmp_path)
    (tmp_path / "activation.int8").write_bytes(b"\x00")
    with pytest.raises(ValueError, match="byte count mismatch"):
        load_quantized_linear_package(tmp_path)


def test_per_token_variant_round_trip_and_golden(tmp_path):
    """Per-token package type: the same files and keys, one activation scale
    per row; the output golden applies each row's scale."""
    from nanopointllm_amd.package import PACKAGE_TYPE_PER_TOKEN

    sa = np.array([0.125, 0.5], np.float16)
    manifest = _write(tmp_path, activation_scale=sa, per_token=True)
    assert manifest["package_type"] == PACKAGE_TYPE_PER_TOKEN
    assert manifest["numerical_contract"]["activation"] == "symmetric_per_token_int8[-127,127]"
    assert manifest["tensors"]["activation_scale"]["shape"] == [2]
    pkg = load_quantized_linear_package(tmp_path)
    assert pkg.per_token
    acc = np.array(PKG["derived_integer_golden"], np.float32)
    ws = np.array(PKG["weight_scale"], np.float16).astype(np.float32)
    exp = (acc * sa.astype(np.float32)[:, None]) * ws[None, :]
    np.testing.assert_array_equal(pkg.output_golden(), exp.astype(np.float32))
    # a static package's golden uses its single scale
    static_dir = tmp_path / "static"
    _write(static_dir)
    spkg = load_quantized_linear_package(static_dir)
    assert not spkg.per_token
    np.testing.assert_array_equal(
        spkg.output_golden(),
        ((acc * np.float32(np.float16(PKG["activation_scale"]))) * ws[None, :]).astype(np.float32))


def test_per_token_variant_rejects_wrong_scale_count_and_unknown_type(tmp_path):
    with pytest.raises(ValueError, match="one FP16 value per activation row"):
        _write(tmp_path, activation_scale=np.array([0.1], np.float16), per_token=True)
    _write(tmp_path / "ok", activation_scale=np.array([0.1, 0.2], np.float16), per_token=True)
    meta_path = tmp_path / "ok" / "metadata.json"
    meta = json.loads(meta_path.read_text())
    meta["package_type"] = "something_else"
    meta_path.write_text(json.dumps(meta, indent=2, sort_keys=True) + "\n")
    with pytest.raises(ValueError, match="unsupported quantized tensor package type"):
        load_quantized_linear_package(tmp_path / "ok")
