"""Host-side calibration API that needs no GPU: the SmoothQuant hardware
report (nanopointllm/compression/w8a8.py:217-251), checked against the
reference's own test (tests/test_w8a8_contract.py:138-151) and the report's
closed-form totals."""
from __future__ import annotations

import torch
import torch.nn as nn


def test_smoothquant_hardware_report_refuses_independent_qkv_fold_claim():
    from nanopointllm_amd.calibration import smoothquant_hardware_report

    modules = {
        "layers.0.self_attn.q_proj": nn.Linear(4, 4),
        "layers.0.self_attn.k_proj": nn.Linear(4, 4),
        "layers.0.mlp.down_proj": nn.Linear(4, 4),
    }
    rep = smoothquant_hardware_report(modules, {name: torch.ones(4) for name in modules})
    assert rep["runtime_overhead_zero"] is False
    assert rep["total_storage_bytes_fp16"] == 24
    assert rep["modules"]["layers.0.self_attn.q_proj"]["offline_fold_status"].startswith(
        "not_foldable_independently")


def test_smoothquant_hardware_report_statuses_and_totals():
    from nanopointllm_amd.calibration import smoothquant_hardware_report

    modules = {"l.mlp.gate_proj": nn.Linear(6, 2), "l.mlp.up_proj": nn.Linear(6, 2),
               "l.self_attn.o_proj": nn.Linear(3, 3), "conv": nn.Conv1d(5, 2, 1)}
    scales = {"l.mlp.gate_proj": torch.ones(6), "l.mlp.up_proj": torch.ones(6),
              "l.self_attn.o_proj": torch.ones(3), "conv": torch.ones(5)}
    rep = smoothquant_hardware_report(modules, scales)
    rows = rep["modules"]
    assert rows["l.mlp.gate_proj"]["offline_fold_status"] == \
        "not_foldable_independently_shared_gate_up_input"
    assert rows["l.self_attn.o_proj"]["offline_fold_status"] == \
        "requires_producer_fanout_and_residual_proof"
    assert rows["conv"]["module_type"] == "Conv1d" and rows["conv"]["channels"] == 5
    assert rep["vector_count"] == 4 and rep["total_scale_values"] == 20
    assert rep["total_storage_bytes_fp16"] == 40
    assert all(r["storage_bytes_fp16"] == 2 * r["channels"] for r in rows.values())
    assert all(r["current_runtime_channelwise_divide"] for r in rows.values())
