"""Calibration, fake-quant and comparison API on the GPU (a7, a9, a11 of the
W8A8 contract, nanopointllm/compression/w8a8.py:65-91, 142-262, 265-447).

Bars: groupwise weight QDQ and every integer result bit-exact against the
oracle; SmoothQuant preserves the linear's product up to fp32 rounding; the
calibrated static scales equal ``static_activation_scale`` of the observed
absmax; QDQ hooks produce the oracle's QDQ values.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import w8a8_oracle as O

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


@pytest.mark.parametrize("shape,group", [((64, 512), 128), ((37, 300), 128), ((16, 100), 1000),
                                         ((8, 4, 96), 32)])
def test_groupwise_weight_qdq_exact(cuda, shape, group):
    from nanopointllm_amd import w8a8

    w = torch.randn(*shape, generator=torch.Generator().manual_seed(shape[0])) * 0.05
    w = w.to(torch.float16)
    note(f"groupwise {shape} g={group}")
    deq, q, s = w8a8.groupwise_weight_qdq(w.to(cuda), group_size=group)
    edeq, eq, es = O.groupwise_weight_qdq(w.float().numpy(), group_size=group)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    np.testing.assert_array_equal(s.cpu().numpy(), es)
    np.testing.assert_array_equal(deq.float().cpu().numpy(), edeq.astype(np.float16))
    assert deq.dtype == torch.float16 and deq.shape == w.shape


def test_compare_linear_report(cuda):
    from nanopointllm_amd import w8a8

    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 5, 256, generator=g)
    w = torch.randn(96, 256, generator=g) * 0.05
    b = torch.randn(96, generator=g)
    absmax = x.abs().max()
    scale = torch.tensor(float(O.static_activation_scale(absmax.numpy())))
    note("compare_linear_bf16_qdq_integer")
    rep = w8a8.compare_linear_bf16_qdq_integer(x.to(cuda), w.to(cuda),
                                               activation_scale=scale.to(cuda), bias=b.to(cuda))
    eout, eacc = O.integer_linear_per_output(x.numpy(), w.numpy(),
                                             activation_scale=scale.numpy(), bias=b.numpy())
    assert rep["shape"] == {"input": [3, 5, 256], "weight": [96, 256], "output": [3, 5, 96]}
    assert rep["accumulator_min"] == int(eacc.min()) and rep["accumulator_max"] == int(eacc.max())
    assert rep["worst_case_accumulator_bound"] == 256 * 127 ** 2
    assert rep["arithmetic_contract"]["bias_application"] == "floating_point_after_dequantization"
    # integer vs fp32 is the quantization error, stable to the fp32 rounding of
    # the dense product; integer vs fp32 QDQ is rounding noise only.
    fp32 = x.numpy().reshape(-1, 256).astype(np.float64) @ w.numpy().astype(np.float64).T
    err = O.tensor_error((fp32 + b.numpy()).reshape(3, 5, 96), eout.reshape(3, 5, 96))
    for key, val in rep["metrics"]["integer_vs_fp32"].items():
        assert val == pytest.approx(err[key], rel=2e-3), key
    scale_out = float(np.abs(eout).max())
    assert rep["metrics"]["integer_vs_qdq_fp32"]["max_abs"] < 1e-4 * scale_out
    assert set(rep["metrics"]) == {"bf16_vs_fp32", "qdq_bf16_vs_qdq_fp32", "integer_vs_qdq_fp32",
                                   "integer_vs_qdq_bf16", "integer_vs_fp32"}


def _linear(k, n, seed, cuda, dtype=torch.float16):
    lin = nn.Linear(k, n, bias=False)
    lin.weight.data = (torch.randn(n, k, generator=torch.Generator().manual_seed(seed))
                       * 0.05).to(dtype)
    return lin.to(cuda)


def test_sequential_qdq_dynamic_and_static_with_smoothing(cuda):
    from nanopointllm_amd import calibration as C

    lin = _linear(300, 64, 1, cuda)
    x = (torch.randn(7, 300, generator=torch.Generator().manual_seed(2)) * 3).to(torch.float16)
    smooth = (torch.rand(300, generator=torch.Generator().manual_seed(3)) + 0.5)
    smooth = smooth.to(torch.float16).float()
    seen = {}
    # a forward hook sees the input after every pre-hook replaced it
    lin.register_forward_hook(lambda m, inp, out: seen.__setitem__("x", inp[0].clone()))
    note("SequentialActivationQDQ dynamic")
    with C.SequentialActivationQDQ({"l": lin}, mode="dynamic_per_token",
                                   input_smoothing_scales={"l": smooth}):
        lin(x.to(cuda))
    xs = O.smooth_divide(x.float().numpy(), smooth.numpy(), "f16")
    eq, es = O.dynamic_per_token_quant(xs)
    np.testing.assert_array_equal(seen["x"].float().cpu().numpy(),
                                  O.round16(eq.astype(np.float32) * es, "f16"))
    static = torch.tensor(float(O.static_activation_scale(np.abs(xs).max())))
    note("SequentialActivationQDQ static")
    with C.SequentialActivationQDQ({"l": lin}, mode="static", static_scales={"l": static},
                                   input_smoothing_scales={"l": smooth}):
        lin(x.to(cuda))
    eqs = O.quantize_symmetric(xs, static.numpy())
    np.testing.assert_array_equal(seen["x"].float().cpu().numpy(),
                                  O.round16(eqs.astype(np.float32) * static.numpy(), "f16"))
    with pytest.raises(ValueError):
        C.SequentialActivationQDQ({"l": lin}, mode="static")


def test_smoothquant_transform_then_w8a8_linear(cuda):
    """apply_smoothquant_transform keeps x @ W^T (x/s @ (W*s)^T), and the W8A8
    linear with the smoothing vector and the calibrated static scale equals
    the oracle's static integer linear on x/s."""
    from nanopointllm_amd import calibration as C
    from nanopointllm_amd.linear import W8A8Linear

    k, n = 512, 128
    lin = _linear(k, n, 5, cuda, dtype=torch.float32)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(9, k, generator=g)
    x[:, :6] *= 30                                       # outlier channels
    x16 = x.to(torch.float16)
    w_before = lin.weight.detach().clone()
    note("ActivationAbsmaxCollector + apply_smoothquant_transform")
    with C.ActivationAbsmaxCollector({"l": lin}) as col:
        lin(x16.float().to(cuda))
    assert col.tensor_absmax["l"] == pytest.approx(float(x16.float().abs().max()))
    np.testing.assert_array_equal(col.channel_absmax["l"].numpy(),
                                  x16.float().abs().amax(0).numpy())
    assert col.samples["l"] == 9
    smooth, act = C.apply_smoothquant_transform({"l": lin}, col.channel_absmax, alpha=0.5)
    s = smooth["l"]
    assert torch.equal(s, s.to(torch.float16).float())   # stored as binary16
    before = x16.float().to(cuda) @ w_before.t()
    after = (x16.float().to(cuda) / s.to(cuda)) @ lin.weight.t()
    torch.testing.assert_close(after, before, rtol=1e-4, atol=1e-4)
    post = float((col.channel_absmax["l"] / s).amax())
    assert float(act["l"]) == float(O.static_activation_scale(np.float32(post)))

    mod = W8A8Linear.from_linear(lin.half(), smooth=s.to(cuda), static_scale=float(act["l"]))
    y = mod(x16.to(cuda))
    xs = O.smooth_divide(x16.float().numpy(), s.numpy(), "f16")
    _, qw, sw = O.per_output_weight_qdq(lin.weight.detach().float().cpu().numpy())
    xq = O.quantize_symmetric(xs, act["l"].numpy())
    acc = O.int32_matmul_f64(xq, qw)
    exp = O.dequant_epilogue(acc, np.float32(act["l"]), sw).astype(np.float16)
    np.testing.assert_array_equal(y.float().cpu().numpy(), exp.astype(np.float32))


def test_apply_weight_qdq_reports(cuda):
    from nanopointllm_amd import calibration as C

    a, b = _linear(200, 48, 7, cuda), _linear(300, 40, 8, cuda)
    wa, wb = a.weight.detach().float().cpu().numpy(), b.weight.detach().float().cpu().numpy()
    note("apply_weight_qdq")
    rep = C.apply_weight_qdq({"a": a}, granularity="per_output")
    rep.update(C.apply_weight_qdq({"b": b}, granularity="group", group_size=64))
    np.testing.assert_array_equal(a.weight.detach().float().cpu().numpy(),
                                  O.per_output_weight_qdq(wa)[0].astype(np.float16))
    np.testing.assert_array_equal(b.weight.detach().float().cpu().numpy(),
                                  O.groupwise_weight_qdq(wb, 64)[0].astype(np.float16))
    assert rep["a"]["scale_shape"] == [48] and rep["b"]["scale_shape"] == [40, 5]
    assert rep["b"]["group_size"] == 64 and rep["a"]["group_size"] is None
    assert -127 <= rep["a"]["quantized_min"] < 0 < rep["a"]["quantized_max"] <= 127
    with pytest.raises(ValueError):
        C.apply_weight_qdq({"a": a}, granularity="tensor")


def test_calibrate_h_scales_feeds_the_int8_chain(cuda):
    """calibrate_h_scales observes h = SiLU(g) * u at each down projection and
    returns static_activation_scale(absmax); the int8 chain then runs."""
    from nanopointllm_amd import calibration as C
    from nanopointllm_amd.inject import inject_w8a8, packed_mlp_decode
    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent))
    from test_gpu_inject import _model

    model = _model(cuda)
    inject_w8a8(model)
    g = torch.Generator().manual_seed(3)
    batches = [torch.randn(1, 4, 256, generator=g).to(torch.float16).to(cuda) for _ in range(3)]
    hs = {}
    for idx, layer in enumerate(model.model.layers):
        mlp = layer.mlp.w8a8_mlp
        hs[idx] = max(float(mlp.gate_up(b[0]).float().abs().max()) for b in batches)

    def run():
        for b in batches:
            for layer in model.model.layers:
                packed_mlp_decode(b, layer.mlp.w8a8_mlp)

    note("calibrate_h_scales")
    scales = C.calibrate_h_scales(model, run)
    assert set(scales) == {0, 1}
    for idx, s in scales.items():
        assert s == float(O.static_activation_scale(np.float32(hs[idx])))
        mlp = model.model.layers[idx].mlp.w8a8_mlp
        assert mlp.h_scale is None                       # restored
        mlp.h_scale = s
        out = packed_mlp_decode(batches[0], mlp)
        assert out.shape == (1, 4, 256) and torch.isfinite(out.float()).all()


# ------------------------------------ the reference's own calibration tests
# (tests/test_w8a8_contract.py:79-160), on the GPU path.
def test_sequential_activation_qdq_propagates_to_later_layer(cuda):
    from nanopointllm_amd import calibration as C, w8a8

    model = nn.Sequential(nn.Linear(4, 4, bias=False), nn.Linear(4, 2, bias=False)).to(cuda)
    modules = {"first": model[0], "second": model[1]}
    values = torch.tensor([[0.03, -0.7, 1.1, 4.3]], device=cuda)
    note("sequential QDQ propagation")
    with C.ActivationAbsmaxCollector(modules) as collector:
        baseline = model(values)
    scales = collector.static_scales()
    captured = []
    handle = model[1].register_forward_pre_hook(
        lambda _m, inputs: captured.append(inputs[0].detach().clone()))
    try:
        with C.SequentialActivationQDQ(modules, mode="static", static_scales=scales):
            candidate = model(values)
    finally:
        handle.remove()
    first_q = w8a8.static_activation_qdq(values, scales["first"].to(cuda))
    np.testing.assert_array_equal(
        first_q.cpu().numpy(),
        O.quantize_symmetric(values.cpu().numpy(), scales["first"].numpy()).astype(np.float32)
        * scales["first"].numpy())
    torch.testing.assert_close(captured[0], model[0](first_q))
    assert not torch.equal(candidate, baseline)


def test_apply_weight_qdq_changes_all_selected_modules(cuda):
    from nanopointllm_amd import calibration as C

    model = nn.Sequential(nn.Linear(7, 5), nn.Linear(5, 3)).to(cuda)
    originals = [m.weight.detach().clone() for m in model]
    note("apply_weight_qdq group 4")
    report = C.apply_weight_qdq({"first": model[0], "second": model[1]}, granularity="group",
                                group_size=4)
    assert set(report) == {"first", "second"}
    assert all(not torch.equal(m.weight, w) for m, w in zip(model, originals))
    for m, w in zip(model, originals):
        np.testing.assert_array_equal(m.weight.detach().cpu().numpy(),
                                      O.groupwise_weight_qdq(w.cpu().numpy(), 4)[0])


def test_smoothquant_transform_is_exact_before_qdq_for_linear_and_conv(cuda):
    from nanopointllm_amd import calibration as C

    torch.manual_seed(8)
    linear = nn.Linear(5, 3).to(cuda)
    x = torch.randn(2, 4, 5, device=cuda)
    ref = linear(x)
    note("smoothquant linear + conv")
    with C.ActivationAbsmaxCollector({"linear": linear}) as col:
        linear(x)
    smoothing, act = C.apply_smoothquant_transform({"linear": linear}, col.channel_absmax,
                                                   alpha=0.5)
    torch.testing.assert_close(linear(x / smoothing["linear"].to(cuda)), ref, rtol=2e-3,
                               atol=2e-3)
    assert act["linear"].numel() == 1
    conv = nn.Conv1d(4, 6, 1).to(cuda)
    xc = torch.randn(2, 4, 7, device=cuda)
    refc = conv(xc)
    with C.ActivationAbsmaxCollector({"conv": conv}) as col:
        conv(xc)
    np.testing.assert_array_equal(col.channel_absmax["conv"].numpy(),
                                  xc.abs().amax(dim=(0, 2)).cpu().numpy())
    smoothing, _ = C.apply_smoothquant_transform({"conv": conv}, col.channel_absmax, alpha=0.5)
    torch.testing.assert_close(conv(xc / smoothing["conv"].to(cuda).reshape(1, 4, 1)), refc,
                               rtol=2e-3, atol=2e-3)


def test_invalid_contract_arguments_fail_closed(cuda):
    from nanopointllm_amd import calibration as C, w8a8

    with pytest.raises(ValueError, match="positive"):
        w8a8.quantize_symmetric(torch.ones(1, device=cuda), torch.tensor(0.0, device=cuda))
    with pytest.raises(ValueError, match="group_size"):
        w8a8.groupwise_weight_qdq(torch.ones(2, 2, device=cuda), group_size=0)
    with pytest.raises(ValueError, match="alpha"):
        C.apply_smoothquant_transform({}, {}, alpha=1.1)
