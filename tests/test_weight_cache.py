"""Offline packed-weight cache: entries load back bit-identically, a model
injected from the cache matches one quantized from scratch without running
any quantization, and corrupted or stale entries are refused."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

sys.path.insert(0, str(Path(__file__).parent))


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def test_entry_round_trip(cuda, tmp_path):
    from nanopointllm_amd import _lib, weight_cache as WC
    from nanopointllm_amd.linear import PackedW8A8Weight

    g = torch.Generator().manual_seed(1)
    w = (torch.randn(96, 300, generator=g) * 0.05).to(torch.float16).to(cuda)
    b = torch.randn(96, generator=g).to(cuda)
    note("weight cache round trip")
    for layout in (_lib.ROWS_AS_IS, _lib.ROWS_INTERLEAVE_HALVES):
        p = PackedW8A8Weight.from_float(w, b, layout=layout)
        d = tmp_path / str(layout)
        manifest = WC.save_packed_weight(d, p, source=w)
        assert manifest["tensors"]["packed"]["bytes"] == _lib.load().w8a8_packed_bytes(96, 300)
        q = WC.load_packed_weight(d, cuda, source=w)
        assert torch.equal(q.packed, p.packed) and torch.equal(q.scale, p.scale)
        assert torch.equal(q.bias, p.bias) and q.layout == layout
        assert (q.out_features, q.in_features) == (96, 300)
    with pytest.raises(ValueError, match="different weight"):
        WC.load_packed_weight(tmp_path / "0", cuda, source=w * 2)
    blob = tmp_path / "0" / "packed.int8"
    raw = bytearray(blob.read_bytes())
    raw[7] ^= 1
    blob.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="SHA256 mismatch"):
        WC.load_packed_weight(tmp_path / "0", cuda)


def test_inject_from_cache_skips_quantization(cuda, tmp_path, monkeypatch):
    from nanopointllm_amd import linear
    from nanopointllm_amd.inject import inject_w8a8, packed_mlp_decode, project_qkv_decode_packed
    from test_gpu_inject import _model

    cache = tmp_path / "cache"
    first = _model(cuda)
    note("inject building the cache")
    inject_w8a8(first, weight_cache=cache)
    entries = sorted(p.parent.name for p in cache.rglob("metadata.json"))
    # per layer: packed QKV, q/k/v/o, packed gate/up, gate/up/down (down shared)
    assert len(entries) == 2 * 9

    second = _model(cuda)

    def no_quantization(*args, **kwargs):
        raise AssertionError("quantized although the cache holds the weight")

    monkeypatch.setattr(linear.PackedW8A8Weight, "from_float", no_quantization)
    note("inject from the cache")
    inject_w8a8(second, weight_cache=cache, verify_source=True)
    x = torch.randn(1, 3, 256, generator=torch.Generator().manual_seed(5)).to(torch.float16)
    x = x.to(cuda)
    for a, b in zip(first.model.layers, second.model.layers):
        for t1, t2 in zip(project_qkv_decode_packed(x, a.self_attn.w8a8_qkv),
                          project_qkv_decode_packed(x, b.self_attn.w8a8_qkv)):
            assert torch.equal(t1, t2)
        assert torch.equal(packed_mlp_decode(x, a.mlp.w8a8_mlp), packed_mlp_decode(x, b.mlp.w8a8_mlp))
        assert torch.equal(a.self_attn.o_proj(x[0]), b.self_attn.o_proj(x[0]))
