"""Two-phase per-token dynamic requantization of the SiLU*mul output
(``w8a8_gateup_silu_mul``; dynamic_per_token_activation_qdq, w8a8.py:106-115,
applied to the down projection's input of the packed MLP,
lightweight_runner.py:344-379).

Bars, on every kernel route (fused decode GEMV, int8-in GEMV, GEMV at
M = 40, MFMA GEMM):
* h bit-equal to the plain SiLU*mul linear on the same inputs;
* hq and its scales bit-exact against the oracle's per-token quantization of
  the GPU's own h, call after call (nothing is carried between calls);
* the down projection on hq bit-exact against the oracle;
* graph replays equal the eager result, replay after replay.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _gateup(inter: int, k: int, seed: int, cuda):
    from nanopointllm_amd import _lib
    from nanopointllm_amd.linear import PackedW8A8Weight

    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(2 * inter, k, generator=g) * 0.02).to(torch.float16)
    b = torch.randn(2 * inter, generator=g) * 0.1
    p = PackedW8A8Weight.from_float(w.to(cuda), b.to(cuda), layout=_lib.ROWS_INTERLEAVE_HALVES)
    return p


CASES = [
    # (label, m, inter, k, int8 x)
    ("fused-decode", 1, 2752, 4096, False),
    ("fused-decode", 8, 2752, 4096, False),
    ("fused-decode-16", 16, 2752, 4096, False),
    ("gemv-i8", 8, 264, 512, True),
    ("gemv", 40, 2752, 1024, False),
    ("gemm", 567, 2752, 1024, False),
    ("gemm-i8", 200, 520, 704, True),
    # int8 rows with K > 8192: the fused kernel's stream on int8 x.
    ("fused-i8-deep", 8, 1376, 11008, True),
    ("fused-i8-deep", 3, 1376, 9216, True),
]


@pytest.mark.parametrize("label,m,inter,k,int8_x", CASES)
def test_two_phase_matches_plain_silu_and_oracle(cuda, label, m, inter, k, int8_x):
    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    p = _gateup(inter, k, seed=m + inter, cuda=cuda)
    x = (W.decode_activations(m, k, seed=m) if m <= 16
         else W.prefill_activations(m, k, seed=m, point_tokens=m // 2)).to(cuda)
    sx = None
    if int8_x:
        x, sx = w8a8.quant_rows(x)
    note(f"two-phase {label} m={m} n={2 * inter} k={k}")
    if int8_x:
        plain = w8a8.linear_i8in(x, sx, p.packed, p.scale, p.bias, p.out_features,
                                 epilogue=_lib.EPI_SILU_MUL, out_dtype=torch.float16)
    else:
        plain = w8a8.linear_dynamic(x, p.packed, p.scale, p.bias, p.out_features,
                                    epilogue=_lib.EPI_SILU_MUL)
    h = plain.cpu().numpy()
    eq, es = O.dynamic_per_token_quant(h.astype(np.float32))
    for _ in range(2):
        out = w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, p.bias, p.out_features,
                                             x_scale=sx, in_features=k)
        np.testing.assert_array_equal(out.h.cpu().numpy(), h)
        np.testing.assert_array_equal(out.hq.cpu().numpy(), eq)
        np.testing.assert_array_equal(out.scale.cpu().numpy(), es[:, 0])


@pytest.mark.parametrize("m", [8, 567])
def test_mlp_two_phase_chain_equals_plain_dynamic_chain(cuda, m):
    """W8A8MLP's two-phase chain gives the same bits as gate/up -> fp16 h ->
    down with its own per-token quantization, and down on the GPU's int8 h
    is exact against the oracle."""
    from nanopointllm_amd import linear
    import workloads as W

    inter, k = 2752, 1024
    g = torch.Generator().manual_seed(9)
    mods = [torch.nn.Linear(k, inter, bias=False), torch.nn.Linear(k, inter, bias=False),
            torch.nn.Linear(inter, k, bias=False)]
    for mod in mods:
        mod.weight.data = (torch.randn(*mod.weight.shape, generator=g) * 0.02).to(
            torch.float16).to(cuda)
    mlp = linear.W8A8MLP(*mods, two_phase=True)
    x = (W.decode_activations(m, k, seed=3) if m <= 16 else
         W.prefill_activations(m, k, seed=3)).to(cuda)
    note(f"mlp two-phase chain m={m}")
    y = mlp(x)
    mlp.two_phase = False
    y_plain = mlp(x)
    mlp.two_phase = True
    np.testing.assert_array_equal(y.cpu().numpy(), y_plain.cpu().numpy())
    out = mlp.gate_up.forward_two_phase(x)
    _, qd, sd = O.per_output_weight_qdq(mods[2].weight.detach().float().cpu().numpy())
    exp, _ = O.linear_from_quantized(out.hq.cpu().numpy(), out.scale.cpu().numpy(), qd, sd)
    np.testing.assert_array_equal(y.cpu().numpy(), exp.astype(np.float16))


def test_two_phase_graph_replays(cuda):
    """Captured in a graph and replayed with eager work between replays:
    every replay equals the eager result."""
    from nanopointllm_amd import w8a8
    import workloads as W

    p = _gateup(2752, 4096, seed=5, cuda=cuda)
    x = W.decode_activations(8, 4096, seed=6).to(cuda)
    eager = w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, None, p.out_features)
    note("two-phase graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, None, p.out_features)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, None, p.out_features)
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.hq, eager.hq) and torch.equal(out.scale, eager.scale), rep
        assert torch.equal(out.h, eager.h), rep
        _ = (x.float() * 2).sum().item()   # eager work between replays


def test_two_phase_argument_checks(cuda):
    from nanopointllm_amd import w8a8

    p = _gateup(264, 512, seed=1, cuda=cuda)
    x = torch.zeros(4, 512, dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError, match="shapes do not match"):
        w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, None, p.out_features,
                                       in_features=448)
    with pytest.raises(ValueError, match="per-row scales"):
        w8a8.gateup_silu_mul_two_phase(x.to(torch.int8), p.packed, p.scale, None,
                                       p.out_features)
    with pytest.raises(ValueError, match="even"):
        w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, None, p.out_features - 1)


# Full-size LLaMA-7B packed gate/up (22016 x 4096): the GEMM tiles the
# library picks at these row counts, each run with the per-block maxima of h.
FULL_M = [560, 567, 768, 1024, 2048]


@pytest.fixture(scope="module")
def gateup_full(cuda):
    return _gateup(11008, 4096, seed=77, cuda=cuda)


@pytest.fixture(scope="module")
def down_full(cuda):
    from nanopointllm_amd.linear import PackedW8A8Weight

    g = torch.Generator().manual_seed(78)
    w = (torch.randn(4096, 11008, generator=g) * 0.02).to(torch.float16)
    _, qd, sd = O.per_output_weight_qdq(w.float().numpy())
    return PackedW8A8Weight.from_float(w.to(cuda)), qd, sd


def test_full_size_tiles_are_covered():
    from gemm_tiles import gemm_config

    tiles = {gemm_config(m, 22016) for m in FULL_M}
    assert len(tiles) >= 4, tiles


@pytest.mark.parametrize("m", FULL_M)
def test_two_phase_full_size_gateup(cuda, gateup_full, down_full, m):
    """h equals the plain SiLU*mul linear, hq and its scales are bit-exact
    against the oracle's per-token quantization of that h, and the down
    projection on hq is exact against the oracle (on a sample of rows)."""
    from gemm_tiles import gemm_config
    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    p = gateup_full
    x = W.prefill_activations(m, 4096, seed=m, point_tokens=min(513, m - 7)).to(cuda)
    note(f"two-phase full size m={m} tile={gemm_config(m, 22016)}")
    plain = w8a8.linear_dynamic(x, p.packed, p.scale, p.bias, p.out_features,
                                epilogue=_lib.EPI_SILU_MUL)
    out = w8a8.gateup_silu_mul_two_phase(x, p.packed, p.scale, p.bias, p.out_features)
    h = plain.cpu().numpy()
    np.testing.assert_array_equal(out.h.cpu().numpy(), h)
    eq, es = O.dynamic_per_token_quant(h.astype(np.float32))
    hq = out.hq.cpu().numpy()
    np.testing.assert_array_equal(hq, eq)
    np.testing.assert_array_equal(out.scale.cpu().numpy(), es[:, 0])
    dp, qd, sd = down_full
    y = w8a8.linear_i8in(out.hq, out.scale.reshape(-1), dp.packed, dp.scale, None,
                         dp.out_features, out_dtype=torch.float16).cpu().numpy()
    rows = np.unique(np.linspace(0, m - 1, 48).astype(int))
    exp, _ = O.linear_from_quantized(hq[rows], es[rows], qd, sd)
    np.testing.assert_array_equal(y[rows], exp.astype(np.float16))
