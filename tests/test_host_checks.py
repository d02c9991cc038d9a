"""Host-side refusals that must happen before any launch (no GPU needed):
the linear wrappers refuse an activation whose K differs from the packed
weight's and buffers shorter than N x K implies, and the packed weight cache
refuses an entry whose manifest shape or row layout differs from the weight
it stands for."""
from __future__ import annotations

import json

import pytest
import torch

from nanopointllm_amd import _lib, w8a8
from nanopointllm_amd import weight_cache as WC


def _packed(n: int, k: int) -> torch.Tensor:
    return torch.zeros(w8a8.packed_bytes(n, k), dtype=torch.int8)


def test_wrong_k_is_refused():
    w = _packed(64, 256)
    s = torch.ones(64)
    w8a8._check_operands(256, w, s, None, 64, 256)        # matching K passes
    with pytest.raises(ValueError, match="shapes do not match"):
        w8a8._check_operands(250, w, s, None, 64, 256)    # same 64-column round-up
    with pytest.raises(ValueError, match="shapes do not match"):
        w8a8._check_operands(320, w, s, None, 64, None)   # more K than packed
    with pytest.raises(ValueError, match="shapes do not match"):
        w8a8._check_operands(256, w, s, None, 80, None)   # more outputs than packed


def test_short_scale_bias_and_bad_dtypes_are_refused():
    w = _packed(64, 256)
    with pytest.raises(ValueError, match="one value per output"):
        w8a8._check_operands(256, w, torch.ones(63), None, 64, 256)
    with pytest.raises(ValueError, match="one value per output"):
        w8a8._check_operands(256, w, torch.ones(64), torch.ones(10), 64, 256)
    with pytest.raises(ValueError, match="float32"):
        w8a8._check_operands(256, w, torch.ones(64, dtype=torch.float16), None, 64, 256)
    with pytest.raises(ValueError, match="int8"):
        w8a8._check_operands(256, w.to(torch.uint8), torch.ones(64), None, 64, 256)


def _fake_entry(root, n, k, layout="rows_as_is"):
    root.mkdir(parents=True)
    manifest = {"schema_version": WC.CACHE_SCHEMA_VERSION, "cache_type": WC.CACHE_TYPE,
                "tile_format": WC.TILE_FORMAT, "row_layout": layout,
                "shape": {"n": n, "k": k}, "source_sha256": None, "tensors": {},
                "provenance": {}}
    (root / "metadata.json").write_text(json.dumps(manifest))


def test_cache_entry_of_other_shape_is_refused(tmp_path):
    _fake_entry(tmp_path / "proj", 64, 256)
    never = lambda: pytest.fail("a cached entry exists; nothing should be built")  # noqa: E731
    with pytest.raises(ValueError, match="shape"):
        WC.cached(tmp_path, "proj", never, source=torch.zeros(64, 512))
    with pytest.raises(ValueError, match="shape"):
        WC.cached(tmp_path, "proj", never, source=torch.zeros(128, 256))
    with pytest.raises(ValueError, match="row layout"):
        WC.cached(tmp_path, "proj", never, source=torch.zeros(64, 256),
                  layout=_lib.ROWS_INTERLEAVE_HALVES)
