#!/usr/bin/env python3
"""W8A8 linear-path benchmark on one MI355X.

Workload (one "step"): the W8A8 linear stack of one LLaMA-7B decode step at
M decode rows (default 8) plus the fp16 LM head, as the full-stack config
names it: 32 layers x {packed QKV [12288x4096], O [4096x4096], packed gate/up
[22016x4096] with fused SiLU*mul -> [M, 11008], down [4096x11008]}, then the
fp16 LM head [32003x4096] (not a W8A8 linear: the reference's F.linear of the
decode rows, here the hand-written dense GEMV of nanopointllm_amd.lm_head at
M <= 16, binary32 accumulation).  Every
layer has its own random-init weights (~N(0, 0.02), per-output int8, 6.48 GB
packed in HBM) so nothing is served from the 256 MB Infinity Cache; RMSNorm
and attention are stubbed by seeded fp16 activations, and the down projection
consumes the gate/up output.  The step is captured once in a HIP graph and
replayed.  Inputs are resident in HBM before timing.

`value` = algorithmic HBM bytes of the step / step time (GB/s), with bytes =
N*K + 2N + 2MK + 2M*N_out per W8A8 linear and 2*V*H + 2MH + 2MV for the LM
head.  The `roofline` object is for the dominant kernel (the packed gate/up
linear: per-token quantization, int8 GEMV and SiLU*mul in one kernel at
M <= 8), timed with HIP events on the stream it is launched on.
`cpu_baseline` times the torch-CPU restatement of the reference's integer
path on all host cores (rank 0, N=1 only), and `parity` reports the GPU
outputs' max-abs / max-relative error against it.  `extra` carries
per-projection decode GB/s at M=1,4,8, the prefill TOPS at M=560/768/1024
(the quantize + GEMM call, the int8-in call with its packing pass, and the
GEMM kernel alone), the stack without the LM head, the LM head alone (the
dense GEMV and torch's F.linear), and the whole-model step through the
runner.

    python bench.py [--steps K] [--warmup W] [--m 8] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "nano-pointllm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
# Per-launch HBM traffic of the gate/up GEMV, from rocprofv3 FETCH_SIZE /
# WRITE_SIZE runs of `bench.py --profile-gateup`, scaled by a copy kernel.
TRAFFIC_SUMMARY = ROOT / "profiles" / "gemv_fused_gateup_m8_traffic.json"
CALIBRATION_COPY_BYTES = 256 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=8, help="decode rows (tokens) per step")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-extra", action="store_true", help="skip the per-projection sweeps")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--profile-gateup", action="store_true",
                    help="only the counter-calibration copy and the gate/up linear loop "
                         "(the region rocprofv3 --pmc runs measure)")
    ap.add_argument("--profile-gemm", action="store_true",
                    help="only the prefill GEMM: packed gate/up (22016 x 4096, SiLU*mul) on "
                         "560 rows of int8 activations, 4 layers x 5 repetitions, after the "
                         "counter-calibration copy (the region rocprofv3 --pmc runs of the "
                         "GEMM measure)")
    ap.add_argument("--profile-proj", choices=["qkv", "o", "gateup", "down"],
                    help="only one projection's W8A8 linear (16-bit x, per-token quantization "
                         "inside the call, as in the decode step) at --profile-m rows, 4 layers "
                         "x 5 repetitions, after the counter-calibration copy (the region "
                         "rocprofv3 runs of that projection measure)")
    ap.add_argument("--profile-m", type=int, default=8)
    ap.add_argument("--profile-timeline", action="store_true",
                    help="only the start-up timeline of the fused gate/up decode kernel at --m "
                         "rows: 32 layers' launches in a graph on the timestamp build "
                         "(libw8a8_gfx950_timeline.so), per-workgroup phases of the last one")
    ap.add_argument("--profile-lm-head", action="store_true",
                    help="only the decode LM head (32003 x 4096 binary16, dense GEMV) at --m "
                         "rows: two weight copies alternating, 10 times each, after the "
                         "counter-calibration copy (the region rocprofv3 runs of the LM head "
                         "measure)")
    ap.add_argument("--profile-runner", action="store_true",
                    help="only the whole-model decode step through W8A8LlamaRunner at --m rows "
                         "(32 LLaMA-7B-shaped layers, LM head), captured and replayed (the "
                         "region rocprofv3 runs of the runner measure)")
    return ap.parse_args()


def profile_proj(device, name: str, m: int) -> dict:
    """One projection's linear over four layers' cold weights, five times,
    after a 256 MiB copy that calibrates the traffic counters."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    src = torch.empty(CALIBRATION_COPY_BYTES, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    del src, dst
    layers = [Layer(i, 8, device) for i in range(4)]
    spec = {p.name: p for p in W.PROJECTIONS}[name]
    x = (W.decode_activations(m, spec.k, seed=11) if m <= 16 else
         W.prefill_activations(m, spec.k, seed=11)).to(device)
    epi = _lib.EPI_SILU_MUL if spec.silu else _lib.EPI_DEQUANT
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        for layer in layers:
            p = layer.weights[name]
            w8a8.linear_dynamic(x, p.packed, p.scale, None, p.out_features, epilogue=epi)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / 20
    return {"projection": name, "m": m, "n": spec.n, "k": spec.k, "launches": 20,
            "host_ms_per_call": round(ms, 4),
            "algorithmic_bytes": W.algorithmic_bytes(m, spec.n, spec.k, silu=spec.silu)}


def profile_lm_head(device, m: int) -> dict:
    """The decode LM head on the dense GEMV: two copies of the weight
    alternating (cold, as in the decode step), 20 launches, after a 256 MiB
    copy that calibrates the traffic counters."""
    import torch

    from nanopointllm_amd.lm_head import dense_gemv

    src = torch.empty(CALIBRATION_COPY_BYTES, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    del src, dst
    lm, xh, nbytes = lm_head(m, device)
    lm2 = lm.clone()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        dense_gemv(xh, lm)
        dense_gemv(xh, lm2)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / 20
    return {"m": m, "shape": list(lm.shape), "launches": 20, "host_ms_per_call": round(ms, 4),
            "algorithmic_bytes": nbytes}


def profile_timeline(device, m: int) -> dict:
    """Per-workgroup start-up timeline of the fused gate/up decode kernel
    (22016 x 4096, binary16 x of m rows, SiLU*mul), from the timestamp build of
    the library: 32 layers' launches captured in a graph and replayed, then
    the stamps of the last launch (100 MHz real-time counter, microseconds
    from the earliest workgroup's entry; medians and ranges over the
    workgroups)."""
    import ctypes
    import statistics

    import torch

    from nanopointllm_amd import _lib, build as _build, w8a8
    import workloads as W
    from nanopointllm_amd.linear import PackedW8A8Weight

    spec = {p.name: p for p in W.PROJECTIONS}["gateup"]
    weights = [PackedW8A8Weight.from_float(
        W.linear_weight(spec.n, spec.k, seed=500 + i, device=device), None,
        layout=_lib.ROWS_INTERLEAVE_HALVES) for i in range(32)]
    x = W.decode_activations(m, spec.k, seed=5).to(device)

    def run():
        for p in weights:
            w8a8.linear_dynamic(x, p.packed, p.scale, None, p.out_features,
                                epilogue=_lib.EPI_SILU_MUL)

    # The same graph on the library proper, then on the timestamp build.
    plain_ms, g = time_graph(run, steps=20, warmup=3)
    del g
    lib = _lib.load(_build.TIMELINE_LIB_PATH)
    lib.w8a8_timeline_read.restype = ctypes.c_int
    lib.w8a8_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    _lib._lib = lib   # the wrappers now call into the timestamp build
    ms, g = time_graph(run, steps=20, warmup=3)
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    nb = -(-spec.n // 16)
    # The library's persistent grid (balanced_grid): every workgroup holds
    # ceil(nb / CUs) blocks or one less.
    groups = nb if nb <= cus else -(-nb // -(-nb // cus))
    buf = (ctypes.c_ulonglong * (groups * 16))()
    if lib.w8a8_timeline_read(ctypes.addressof(buf), groups) != 0:
        raise RuntimeError("w8a8_timeline_read failed")
    stamps = [[buf[wg * 16 + i] for i in range(16)] for wg in range(groups)]
    t0 = min(st[0] for st in stamps)
    us = lambda v: (v - t0) / 100.0  # noqa: E731

    def dist(vals):
        return {"median": round(statistics.median(vals), 2), "min": round(min(vals), 2),
                "max": round(max(vals), 2)}

    phases = {"entry": 0, "x_ready": 1, "prologue_done": 2, "first_weight_data": 3,
              "first_block_done": 4, "end": 15}
    out = {name: dist([us(st[i]) for st in stamps]) for name, i in phases.items()}
    # Blocks after the first: the workgroup's steady rate.
    intervals = []
    for wg, st in enumerate(stamps):
        n_mine = (nb - wg + groups - 1) // groups
        blocks = [st[4 + j] for j in range(min(n_mine, 11))]
        intervals += [(b - a) / 100.0 for a, b in zip(blocks[1:], blocks[2:])]
    block_bytes = 16 * spec.k
    per_block = statistics.median(intervals)
    return {"kernel": "gemv_fused_kernel (packed gate/up, SiLU*mul)", "m": m, "n": spec.n,
            "k": spec.k, "workgroups": groups,
            "us_per_launch_graph_plain": round(plain_ms * 1e3 / 32, 3),
            "us_per_launch_graph_timeline": round(ms * 1e3 / 32, 3),
            "phases_us": out, "steady_block_us": round(per_block, 3),
            "steady_GBps_per_cu": round(block_bytes / (per_block * 1e-6) / 1e9, 1),
            "steady_TBps_all_cus": round(block_bytes * groups / (per_block * 1e-6) / 1e12, 2)}


def profile_gemm(device) -> dict:
    """The packed gate/up GEMM at M = 560 (int8 in, SiLU*mul epilogue) over four
    layers' cold weights, after a 256 MiB copy that calibrates the counters."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    src = torch.empty(CALIBRATION_COPY_BYTES, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    del src, dst
    m, layers = 560, [Layer(i, 8, device) for i in range(4)]
    spec = {p.name: p for p in W.PROJECTIONS}["gateup"]
    xq, sx = w8a8.quant_rows(W.prefill_activations(m, spec.k, seed=11).to(device))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        for layer in layers:
            p = layer.weights["gateup"]
            w8a8.linear_i8in(xq, sx, p.packed, p.scale, None, p.out_features,
                             epilogue=_lib.EPI_SILU_MUL)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / 20
    return {"m": m, "n": spec.n, "k": spec.k, "launches": 20, "host_ms_per_call": round(ms, 4)}


class Layer:
    """One decoder layer's four packed W8A8 projections plus stub inputs."""

    def __init__(self, idx: int, m: int, device):
        import torch

        from nanopointllm_amd import _lib, w8a8
        import workloads as W
        from nanopointllm_amd.linear import PackedW8A8Weight

        self.weights = {}
        for j, spec in enumerate(W.PROJECTIONS):
            w16 = W.linear_weight(spec.n, spec.k, seed=1000 * idx + j, device=device)
            layout = _lib.ROWS_INTERLEAVE_HALVES if spec.silu else _lib.ROWS_AS_IS
            self.weights[spec.name] = PackedW8A8Weight.from_float(w16, None, layout=layout)
            del w16
        self.x = {name: W.decode_activations(m, W.HIDDEN, seed=100 * idx + j).to(device)
                  for j, name in enumerate(("qkv", "o", "gateup"))}
        self.m = m
        self.w8a8 = w8a8
        self.lib = _lib
        torch.cuda.synchronize()

    def step(self):
        w, x, f = self.weights, self.x, self.w8a8
        f.linear_dynamic(x["qkv"], w["qkv"].packed, w["qkv"].scale, None, w["qkv"].out_features)
        f.linear_dynamic(x["o"], w["o"].packed, w["o"].scale, None, w["o"].out_features)
        h = f.linear_dynamic(x["gateup"], w["gateup"].packed, w["gateup"].scale, None,
                             w["gateup"].out_features, epilogue=self.lib.EPI_SILU_MUL)
        f.linear_dynamic(h, w["down"].packed, w["down"].scale, None, w["down"].out_features)


def step_bytes(m: int, layers: int) -> int:
    import workloads as W

    return layers * sum(W.algorithmic_bytes(m, p.n, p.k, silu=p.silu) for p in W.PROJECTIONS)


def time_graph(fn, steps: int, warmup: int):
    """Capture fn in a HIP graph; return (ms per replay, graph)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                               # eager warm-up (allocator, code objects)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps, g


def event_time_ms(fn, reps: int) -> float:
    """Average ms of fn over reps, bracketed by HIP events on the current stream."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def gateup_kernel_roofline(layers, m: int, device) -> dict:
    """Average duration of the step's dominant launch, the packed gate/up
    linear (binary16 x, fused SiLU*mul), over 32 layers x 20 repetitions,
    bracketed by HIP events on the stream the kernels run on.  At decode sizes
    it is one kernel (quantization fused into the GEMV); otherwise the
    quantization and the GEMV launch are both counted."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    spec = {p.name: p for p in W.PROJECTIONS}["gateup"]
    x = layers[0].x["gateup"]
    outs = [torch.empty(m, spec.n // 2, dtype=torch.float16, device=device) for _ in layers]
    lib = _lib.load()
    stream = _lib.stream_handle(device)

    def call_args(layer, y, ws):
        p = layer.weights["gateup"]
        return (x.data_ptr(), _lib.F16, spec.k, p.packed.data_ptr(), p.scale.data_ptr(), None,
                _lib.EPI_SILU_MUL, y.data_ptr(), _lib.F16, spec.n // 2, 0.0, _lib.F16, m, spec.n,
                spec.k, None, None if ws is None else ws.data_ptr(),
                0 if ws is None else ws.numel(), stream)

    ws = None
    fused = lib.w8a8_linear(*call_args(layers[0], outs[0], None)) == _lib.OK
    if not fused:
        ws = torch.empty(w8a8.workspace_bytes(m, spec.k), dtype=torch.uint8, device=device)
    args = [call_args(layer, y, ws) for layer, y in zip(layers, outs)]

    def run_all():
        for a in args:
            rc = lib.w8a8_linear(*a)
            if rc:
                _lib.check(rc, "w8a8_linear")

    reps = 20
    ms = event_time_ms(run_all, reps) / len(args)
    nbytes = W.algorithmic_bytes(m, spec.n, spec.k, silu=True)
    achieved = nbytes / (ms * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_SUMMARY.exists():
        t = json.loads(TRAFFIC_SUMMARY.read_text())
        if t.get("m") == m and fused:
            traffic = t["hbm_bytes_per_launch"]
    kernel = ("gemv_fused_kernel (packed gate/up: per-token quantization + int8 GEMV + "
              "SiLU*mul, one launch)" if fused else
              "quant_rows_kernel + gemv_kernel (packed gate/up, SiLU*mul)")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kernel,
            "avg_launch_us": round(ms * 1e3, 3), "algorithmic_bytes_per_launch": nbytes}


def projection_sweep(layers, device, ms_list=(1, 4, 8)) -> dict:
    """Decode GB/s per projection (graph of 32 launches over distinct weights)."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    out = {}
    for m in ms_list:
        row = {}
        for spec in W.PROJECTIONS:
            if spec.silu:
                fn_args = dict(epilogue=_lib.EPI_SILU_MUL)
            else:
                fn_args = {}
            x16 = W.decode_activations(m, spec.k, seed=7).to(device)

            def run(spec=spec, x16=x16, fn_args=fn_args):
                for layer in layers:
                    p = layer.weights[spec.name]
                    w8a8.linear_dynamic(x16, p.packed, p.scale, None, p.out_features, **fn_args)

            ms, g = time_graph(run, steps=10, warmup=3)
            del g
            per = ms / len(layers)
            nbytes = W.algorithmic_bytes(m, spec.n, spec.k, silu=spec.silu)
            row[spec.name] = {"us": round(per * 1e3, 2),
                              "GBps": round(nbytes / (per * 1e-3) / 1e9, 1)}
        out[f"M{m}"] = row
    torch.cuda.synchronize()
    return out


def prefill_sweep(layers, device, m: int = 560) -> dict:
    """Prefill TOPS per projection, graphs over 8 layers' cold weights:
    * ``linear``: binary16 x in (per-token quantization launch + GEMM);
    * ``i8in_pack_gemm``: row-major int8 x in (``w8a8_linear_i8in``: the pass
      that packs the rows into 16x64 tiles, then the GEMM);
    * ``gemm_kernel``: the GEMM kernel alone on x already packed
      (``w8a8_linear_packed``), with the tile the library picks."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    lib = _lib.load()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    names = _lib.GEMM_TILE_NAMES
    out = {}
    for spec in W.PROJECTIONS:
        x16 = W.prefill_activations(m, spec.k, seed=11).to(device)
        xq, sx = w8a8.quant_rows(x16)
        xp = w8a8.pack_rows(xq)
        fn_args = dict(epilogue=_lib.EPI_SILU_MUL) if spec.silu else {}
        sub = layers[:8]

        def run_linear(spec=spec, x16=x16, fn_args=fn_args):
            for layer in sub:
                p = layer.weights[spec.name]
                w8a8.linear_dynamic(x16, p.packed, p.scale, None, p.out_features, **fn_args)

        def run_i8in(spec=spec, xq=xq, sx=sx, fn_args=fn_args):
            for layer in sub:
                p = layer.weights[spec.name]
                w8a8.linear_i8in(xq, sx, p.packed, p.scale, None, p.out_features,
                                 out_dtype=torch.float16, **fn_args)

        def run_kernel(spec=spec, xp=xp, sx=sx, fn_args=fn_args):
            for layer in sub:
                p = layer.weights[spec.name]
                w8a8.linear_packed(xp, sx, m, spec.k, p.packed, p.scale, None, p.out_features,
                                   out_dtype=torch.float16, **fn_args)

        timed = {}
        for key, fn in (("linear", run_linear), ("i8in_pack_gemm", run_i8in),
                        ("gemm_kernel", run_kernel)):
            ms, g = time_graph(fn, steps=10, warmup=3)
            del g
            timed[key] = ms / len(sub)
        ops = W.algorithmic_ops(m, spec.n, spec.k)
        row = {}
        for key, per in timed.items():
            row[f"{key}_us"] = round(per * 1e3, 2)
            row[f"{key}_TOPS"] = round(ops / (per * 1e-3) / 1e12, 1)
        row["gemm_kernel_frac_int8_peak"] = round(
            ops / (timed["gemm_kernel"] * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4)
        row["tile"] = names[lib.w8a8_gemm_tile_config(m, spec.n, cus)]
        out[spec.name] = row
    torch.cuda.synchronize()
    return out


def prefill_sweep_all(layers, device) -> dict:
    return {f"M{m}": prefill_sweep(layers, device, m) for m in (560, 768, 1024)}


def m_sweep(layers, device, proj: str, ms_list) -> dict:
    """Per-launch time of one projection's fused linear (fp16 in: quantize +
    product, or the fused decode kernel) across row counts: the GEMV / MFMA
    crossover and the 17..64-row regime of batched decode."""
    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    spec = {p.name: p for p in W.PROJECTIONS}[proj]
    epi = _lib.EPI_SILU_MUL if spec.silu else _lib.EPI_DEQUANT
    sub = layers[:8]
    out = {}
    for m in ms_list:
        x16 = (W.decode_activations(m, spec.k, seed=13) if m <= 16
               else W.prefill_activations(m, spec.k, seed=13)).to(device)

        def run(x16=x16):
            for layer in sub:
                p = layer.weights[proj]
                w8a8.linear_dynamic(x16, p.packed, p.scale, None, p.out_features, epilogue=epi)

        ms, g = time_graph(run, steps=10, warmup=3)
        del g
        per = ms / len(sub)
        nbytes = W.algorithmic_bytes(m, spec.n, spec.k, silu=spec.silu)
        out[f"M{m}"] = {"us": round(per * 1e3, 2),
                        "GBps": round(nbytes / (per * 1e-3) / 1e9, 1),
                        "TOPS": round(W.algorithmic_ops(m, spec.n, spec.k) / (per * 1e-3) / 1e12, 1)}
    return out


def mixed_chain(layers, device, h_scale_m: int = 567) -> dict:
    """7 decode rows + a 560-row prefill chunk (M=567): gate/up + SiLU*mul + int8
    requant (static scale) -> int8-in down projection."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W

    m = h_scale_m
    x = torch.cat([W.decode_activations(7, W.HIDDEN, seed=21),
                   W.prefill_activations(560, W.HIDDEN, seed=22)]).to(device)
    sub = layers[:8]
    gu0 = sub[0].weights["gateup"]
    h = w8a8.linear_dynamic(x, gu0.packed, gu0.scale, None, gu0.out_features,
                            epilogue=_lib.EPI_SILU_MUL)
    from nanopointllm_amd.w8a8 import static_activation_scale

    h_scale = float(static_activation_scale(h.abs().max(), device=device))
    s_rows = torch.full((m,), h_scale, dtype=torch.float32, device=device)

    def run():
        for layer in sub:
            gu, dn = layer.weights["gateup"], layer.weights["down"]
            hq = w8a8.linear_dynamic(x, gu.packed, gu.scale, None, gu.out_features,
                                     epilogue=_lib.EPI_SILU_MUL_Q8, y_scale=h_scale)
            w8a8.linear_i8in(hq, s_rows, dn.packed, dn.scale, None, dn.out_features,
                             out_dtype=torch.float16)

    ms, g = time_graph(run, steps=10, warmup=3)
    del g
    per = ms / len(sub)
    ops = W.algorithmic_ops(m, 2 * W.INTERMEDIATE, W.HIDDEN) + W.algorithmic_ops(m, W.HIDDEN, W.INTERMEDIATE)
    return {"M": m, "us_per_layer": round(per * 1e3, 2),
            "TOPS": round(ops / (per * 1e-3) / 1e12, 1), "h_scale": h_scale}


def decode_step_int8_mlp(layers, m: int, device) -> dict:
    """The decode step with the int8 MLP chain (static-A8 requant,
    lightweight_runner.py:362-379 with a calibrated h scale): gate/up's epilogue
    writes int8 h, and the down projection takes it without a quantization
    launch.  QKV and O are as in the default step."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W
    from nanopointllm_amd.w8a8 import static_activation_scale

    x0, gu0 = layers[0].x["gateup"], layers[0].weights["gateup"]
    h = w8a8.linear_dynamic(x0, gu0.packed, gu0.scale, None, gu0.out_features,
                            epilogue=_lib.EPI_SILU_MUL)
    h_scale = float(static_activation_scale(h.abs().max(), device=device))
    s_rows = torch.full((m,), h_scale, dtype=torch.float32, device=device)

    def step():
        for layer in layers:
            w, x = layer.weights, layer.x
            w8a8.linear_dynamic(x["qkv"], w["qkv"].packed, w["qkv"].scale, None,
                                w["qkv"].out_features)
            w8a8.linear_dynamic(x["o"], w["o"].packed, w["o"].scale, None, w["o"].out_features)
            hq = w8a8.linear_dynamic(x["gateup"], w["gateup"].packed, w["gateup"].scale, None,
                                     w["gateup"].out_features, epilogue=_lib.EPI_SILU_MUL_Q8,
                                     y_scale=h_scale)
            w8a8.linear_i8in(hq, s_rows, w["down"].packed, w["down"].scale, None,
                             w["down"].out_features, out_dtype=torch.float16)

    ms, g = time_graph(step, steps=10, warmup=3)
    del g
    spec = {p.name: p for p in W.PROJECTIONS}
    per_layer = (W.algorithmic_bytes(m, spec["qkv"].n, spec["qkv"].k)
                 + W.algorithmic_bytes(m, spec["o"].n, spec["o"].k)
                 + W.algorithmic_bytes(m, spec["gateup"].n, spec["gateup"].k, silu=True,
                                       int8_out=True)
                 + W.algorithmic_bytes(m, spec["down"].n, spec["down"].k, int8_in=True))
    nbytes = per_layer * len(layers)
    return {"ms": round(ms, 4), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes,
            "h_scale": h_scale}


def lm_head(m: int, device):
    """The fp16 LM head [32003 x 4096] of config 4 and its input rows (a
    plain 16-bit linear, not a W8A8 one), with its algorithmic bytes."""
    import torch

    import workloads as W

    g = torch.Generator(device=device)
    g.manual_seed(99)
    lm = (torch.randn(W.VOCAB, W.HIDDEN, generator=g, device=device) * 0.02).to(torch.float16)
    xh = W.decode_activations(m, W.HIDDEN, seed=98).to(device)
    nbytes = W.VOCAB * W.HIDDEN * 2 + 2 * m * W.HIDDEN + 2 * m * W.VOCAB
    return lm, xh, nbytes


def lm_head_alone(lm, xh, nbytes: int) -> dict:
    """The decode LM head by itself: the dense GEMV against torch's F.linear
    (the reference's op) on the same rows, in graphs that alternate the
    weight with a second copy so that neither is served from the 256 MB
    Infinity Cache (as in the decode step, where the layers' weights evict
    it)."""
    import torch

    from nanopointllm_amd.lm_head import dense_gemv

    lm2 = lm.clone()
    out = {}
    for name, fn in (("dense_gemv", dense_gemv), ("torch_F_linear", torch.nn.functional.linear)):
        if name == "dense_gemv" and xh.shape[0] > 16:
            continue
        ms, gr = time_graph(lambda: (fn(xh, lm), fn(xh, lm2)), steps=20, warmup=3)
        del gr
        ms /= 2
        out[name] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    del lm2
    return out


def stack_without_lm_head(layers, m: int, device) -> dict:
    """The 32-layer W8A8 stack alone (the headline step less the LM head)."""
    def step():
        for layer in layers:
            layer.step()

    ms, gr = time_graph(step, steps=10, warmup=3)
    del gr
    nbytes = step_bytes(m, len(layers))
    return {"ms": round(ms, 4), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes}


def runner_decode_step(m: int, device, steps: int = 20, warmup: int = 5) -> dict:
    """A whole decode step of a 32-layer LLaMA-7B-shaped model through
    ``W8A8LlamaRunner`` (lightweight_runner.py:421-737) at M = m rows: per
    layer the fused RMSNorm + packed QKV launch (with the previous layer's
    residual add), o_proj, the fused residual add + RMSNorm + gate/up SiLU*mul
    launch and down; then the final norm and the fp16 LM head.  Random weights
    (~N(0, 0.02)); the attention core is ``query_passthrough_core`` (no
    kernel).  Captured with ``DecodeGraphBucket`` (engine/cuda_graph.py:17-52)
    and replayed; the first replay is checked against the eager step.  Timed
    on the same model with per-token dynamic quantization of h, then as a
    560-row prefill step, then with the static int8 MLP chain (a calibrated h
    scale per layer, the maximum |h| of one eager step,
    lightweight_runner.py:362-379)."""
    import torch

    import workloads as W
    from nanopointllm_amd.runner import DecodeGraphBucket, W8A8LlamaRunner
    from nanopointllm_amd.w8a8 import static_activation_scale

    model = W.llama_model(device, layers=W.LAYERS, seed=7)
    runner = W8A8LlamaRunner(model, W.query_passthrough_core)
    ids = torch.randint(0, W.VOCAB, (m,), generator=torch.Generator().manual_seed(8)).to(device)
    nbytes = (step_bytes(m, W.LAYERS) + W.VOCAB * W.HIDDEN * 2 + 2 * m * W.HIDDEN
              + 2 * m * W.VOCAB)

    def timed(ids=ids) -> tuple[float, bool]:
        eager = runner(ids).clone()
        bucket = DecodeGraphBucket(device)
        bucket.capture(lambda: runner(ids))
        same = bool(torch.equal(bucket.replay(), eager))
        for _ in range(warmup):
            bucket.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            bucket.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        del bucket
        return ms, same

    ms, same = timed()
    # A prefill step of 560 rows (the size of 513 point tokens plus a prompt)
    # on the same model: every projection on the MFMA GEMM, the RMSNorm
    # prologue writing the GEMM's packed tiles.
    pm = 560
    pids = torch.randint(0, W.VOCAB, (pm,), generator=torch.Generator().manual_seed(9)).to(device)
    ms_pf, same_pf = timed(pids)
    ops_pf = W.LAYERS * sum(W.algorithmic_ops(pm, p.n, p.k) for p in W.PROJECTIONS)
    ops_pf += 2 * pm * W.VOCAB * W.HIDDEN
    # Calibrate: each layer's max |h| (the down projection's input) over one
    # eager step, then every MLP switches to the static int8 chain.  The step
    # runs layer by layer on the route whose down projection is a module call
    # (the same h as the decode route).
    h_max: dict[int, torch.Tensor] = {}
    hooks = [layer.mlp.down.register_forward_hook(
        lambda mod, args, out, i=i: h_max.__setitem__(i, args[0].detach().abs().max()))
        for i, layer in enumerate(runner.layers)]
    hidden, residual = runner.embed_tokens(ids), None
    for layer in runner.layers:
        hidden, residual = layer.forward_carry(hidden, residual)
    for h in hooks:
        h.remove()
    for i, layer in enumerate(runner.layers):
        layer.mlp.h_scale = float(static_activation_scale(h_max[i], device=device))
    ms_q8, same_q8 = timed()
    spec = {p.name: p for p in W.PROJECTIONS}
    h_bytes = (W.algorithmic_bytes(m, spec["gateup"].n, spec["gateup"].k, silu=True)
               + W.algorithmic_bytes(m, spec["down"].n, spec["down"].k))
    h_bytes_q8 = (W.algorithmic_bytes(m, spec["gateup"].n, spec["gateup"].k, silu=True,
                                      int8_out=True)
                  + W.algorithmic_bytes(m, spec["down"].n, spec["down"].k, int8_in=True))
    nbytes_q8 = nbytes - W.LAYERS * (h_bytes - h_bytes_q8)
    del runner, model
    torch.cuda.empty_cache()
    return {"ms": round(ms, 4), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes,
            "m": m, "layers": W.LAYERS, "replay_equals_eager": same,
            "int8_mlp_chain": {"ms": round(ms_q8, 4),
                               "GBps": round(nbytes_q8 / (ms_q8 * 1e-3) / 1e9, 1),
                               "bytes": nbytes_q8, "replay_equals_eager": same_q8},
            "prefill": {"m": pm, "ms": round(ms_pf, 4),
                        "TOPS": round(ops_pf / (ms_pf * 1e-3) / 1e12, 1),
                        "replay_equals_eager": same_pf},
            "attention_core": "query pass-through (no kernel)"}


def _median_s(fn, reps: int = 5) -> float:
    """Median wall time of fn over reps runs, after one untimed run."""
    fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def _host_weight(layer, name: str, n: int, k: int):
    """A layer's packed int8 weight back in row-major order on the host."""
    import torch

    p = layer.weights[name]
    return (torch.from_numpy(_unpack_rows(p.packed.cpu().numpy(), n, k)), p.scale.cpu())


def cpu_baseline(layers, m: int) -> dict:
    """The reference CPU integer path (the torch restatement of
    integer_linear_per_output_reference with per-token activation scales,
    w8a8.py:106-139, in oracle/torch_path.py) on all host cores, median of 5
    runs per configuration: config 1 ([16, 4096] x [4096, 4096]), the four
    decode projections at M = m on one layer's weights (gate/up with
    SiLU*mul), and O at M = 560.  `value` is the decode layer's rate in the
    headline's unit."""
    import torch

    import workloads as W
    from oracle import torch_path as T, w8a8_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    configs = {}

    def record(name, fn, nbytes, ops):
        t = _median_s(fn)
        configs[name] = {"ms": round(t * 1e3, 3), "GBps": round(nbytes / t / 1e9, 3),
                         "GOPS": round(ops / t / 1e9, 2)}
        return t

    x1, w1 = W.config1()
    _, q1, s1 = O.per_output_weight_qdq(w1.float().numpy())
    q1, s1 = torch.from_numpy(q1), torch.from_numpy(s1)
    record("config1_m16_n4096_k4096", lambda: T.per_token_linear(x1, q1, s1)[0].half(),
           W.algorithmic_bytes(16, 4096, 4096), W.algorithmic_ops(16, 4096, 4096))
    layer_bytes, layer_s = 0, 0.0
    for spec in W.PROJECTIONS:
        q, sc = _host_weight(layers[0], spec.name, spec.n, spec.k)
        x = W.decode_activations(m, spec.k, seed=5)
        if spec.silu:
            fn = (lambda x=x, q=q, sc=sc: T.silu_mul(T.per_token_linear(x, q, sc)[0].half()))
        else:
            fn = (lambda x=x, q=q, sc=sc: T.per_token_linear(x, q, sc)[0].half())
        nbytes = W.algorithmic_bytes(m, spec.n, spec.k, silu=spec.silu)
        layer_s += record(f"decode_m{m}_{spec.name}", fn, nbytes,
                          W.algorithmic_ops(m, spec.n, spec.k))
        layer_bytes += nbytes
    q, sc = _host_weight(layers[0], "o", W.HIDDEN, W.HIDDEN)
    xo = W.prefill_activations(560, W.HIDDEN, seed=11)
    record("prefill_m560_o", lambda: T.per_token_linear(xo, q, sc)[0].half(),
           W.algorithmic_bytes(560, W.HIDDEN, W.HIDDEN), W.algorithmic_ops(560, W.HIDDEN, W.HIDDEN))
    return {"value": round(layer_bytes / layer_s / 1e9, 4), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": (f"torch CPU int32 restatement of integer_linear_per_output_reference "
                       f"(per-token A8, w8a8.py:106-139), {cores} threads, median of 5 runs; "
                       f"value = one layer's 4 decode projections at M={m} "
                       f"({layer_bytes / 1e6:.1f} MB in {layer_s * 1e3:.1f} ms); per-config "
                       f"rates in 'configs'"),
            "configs": configs}


def _error_stats(got: "torch.Tensor", ref32: "torch.Tensor") -> dict:
    """max-abs and max-relative error (denominator clamped at 1e-8, as
    _tensor_error in w8a8.py:254-262) of a 16-bit output against binary32."""
    diff = (got.double() - ref32.double()).abs()
    rel = diff / ref32.double().abs().clamp_min(1e-8)
    return {"max_abs": float(diff.max()), "max_rel": float(rel.max()),
            "mean_abs": float(diff.mean())}


def parity_report(layers, m: int, device) -> dict:
    """The GPU's outputs against the CPU path (oracle/torch_path.py) on the
    same inputs: config 1 (dequant to fp16) and the packed gate/up with fused
    SiLU*mul at M = m (the dominant kernel).  int32 accumulators compared for
    equality; fp16 outputs with max-abs / max-relative error against the CPU
    path's binary32 values and the fraction bit-equal to its fp16 result."""
    import torch

    from nanopointllm_amd import _lib, w8a8
    import workloads as W
    from nanopointllm_amd.linear import PackedW8A8Weight
    from oracle import torch_path as T, w8a8_oracle as O

    out = {}
    x1, w1 = W.config1()
    _, q1, s1 = O.per_output_weight_qdq(w1.float().numpy())
    q1, s1 = torch.from_numpy(q1), torch.from_numpy(s1)
    p = PackedW8A8Weight.from_int8(q1.to(device), s1.to(device))
    y = w8a8.linear_dynamic(x1.to(device), p.packed, p.scale, None, 4096).cpu()
    acc = w8a8.linear_dynamic(x1.to(device), p.packed, p.scale, None, 4096,
                              epilogue=_lib.EPI_I32).cpu()
    ref, eacc = T.per_token_linear(x1, q1, s1)
    out["config1"] = {"int32_equal": bool(torch.equal(acc, eacc)),
                      "fp16_bit_equal_frac": float((y == ref.half()).float().mean()),
                      **_error_stats(y, ref)}
    q, sc = _host_weight(layers[0], "gateup", 2 * W.INTERMEDIATE, W.HIDDEN)
    x = layers[0].x["gateup"]
    p = layers[0].weights["gateup"]
    h = w8a8.linear_dynamic(x, p.packed, p.scale, None, p.out_features,
                            epilogue=_lib.EPI_SILU_MUL).cpu()
    acc = w8a8.linear_dynamic(x, p.packed, p.scale, None, p.out_features,
                              epilogue=_lib.EPI_I32).cpu()
    gu32, eacc = T.per_token_linear(x.cpu(), q, sc)
    pairs = gu32.half().view(m, -1, 2)
    ref32 = torch.nn.functional.silu(pairs[..., 0]).float() * pairs[..., 1].float()
    out[f"gateup_silu_m{m}"] = {"int32_equal": bool(torch.equal(acc, eacc)),
                                "fp16_bit_equal_frac": float(
                                    (h == T.silu_mul(gu32.half())).float().mean()),
                                **_error_stats(h, ref32)}
    return out


def _unpack_rows(packed, rows: int, k: int):
    import numpy as np

    rp, kp = -(-rows // 16) * 16, -(-k // 64) * 64
    t = packed.reshape(rp // 16, kp // 64, 4, 16, 16).transpose(0, 3, 1, 2, 4)
    return np.ascontiguousarray(t.reshape(rp, kp)[:rows, :k])


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: the W8A8 "
              "linear path runs on one GPU, and its throughput is the one GPU's.",
              file=sys.stderr)
        return 2
    import torch

    from nanopointllm_amd import _lib
    from nanopointllm_amd.lm_head import dense_gemv
    import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    _lib.load()
    device = torch.device("cuda:0")
    if args.profile_gemm:
        print(json.dumps({"profile_gemm": profile_gemm(device)}))
        return 0
    if args.profile_proj:
        print(json.dumps({"profile_proj": profile_proj(device, args.profile_proj,
                                                        args.profile_m)}))
        return 0
    m = args.m
    if args.profile_timeline:
        print(json.dumps({"profile_timeline": profile_timeline(device, m)}))
        return 0
    if args.profile_runner:
        print(json.dumps({"profile_runner": runner_decode_step(m, device)}))
        return 0
    if args.profile_lm_head:
        print(json.dumps({"profile_lm_head": profile_lm_head(device, m)}))
        return 0
    log(f"building {args.layers} layers of packed W8A8 weights (M={m})")
    layers = [Layer(i, m, device) for i in range(args.layers)]
    if args.profile_gateup:
        # Counter calibration: a plain device copy of known size, then the
        # gate/up GEMV loop timed by the roofline measurement.
        src = torch.empty(CALIBRATION_COPY_BYTES, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        roof = gateup_kernel_roofline(layers, m, device)
        print(json.dumps({"profile_gateup": roof, "calibration_copy_bytes": CALIBRATION_COPY_BYTES}))
        return 0

    lm, xh, lm_bytes = lm_head(m, device)
    # The decode LM head: the dense GEMV up to 16 rows, torch's GEMM beyond.
    head = dense_gemv if m <= 16 else torch.nn.functional.linear

    def step():
        for layer in layers:
            layer.step()
        head(xh, lm)

    log("capturing step graph")
    ms_per_step, graph = time_graph(step, args.steps, args.warmup)
    nbytes = step_bytes(m, args.layers) + lm_bytes
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    log(f"step {ms_per_step:.4f} ms, {value:.1f} GB/s")
    del graph

    log("timing gate/up GEMV kernel")
    roofline = gateup_kernel_roofline(layers, m, device)
    log(f"gate/up kernel {roofline['avg_launch_us']} us, {roofline['achieved']} GB/s")

    extra = {}
    if not args.no_extra:
        log("decode sweep M=1,4,8")
        extra["decode_per_projection"] = projection_sweep(layers, device)
        log("prefill sweep M=560,768,1024")
        extra["prefill"] = prefill_sweep_all(layers, device)
        log("QKV M sweep")
        extra["qkv_m_sweep"] = m_sweep(layers, device, "qkv",
                                       (1, 2, 4, 16, 17, 24, 32, 48, 64, 256, 2048))
        extra["gateup_m_sweep"] = m_sweep(layers, device, "gateup", (17, 24, 32, 48, 64))
        log("mixed M=567 int8 chain")
        extra["mixed_567_gateup_down_int8_chain"] = mixed_chain(layers, device)
        log("stack without the LM head")
        extra["stack_without_lm_head"] = stack_without_lm_head(layers, m, device)
        log("LM head alone")
        extra["lm_head"] = lm_head_alone(lm, xh, lm_bytes)
        log("decode step with the int8 MLP chain")
        extra["decode_step_int8_mlp_chain"] = decode_step_int8_mlp(layers, m, device)
        log("runner decode step (32 layers, fused norms, LM head)")
        extra["runner_decode_step"] = runner_decode_step(m, device)

    cpu = parity = None
    if not args.no_cpu:
        log("cpu baseline (torch int32 restatement, all host cores)")
        cpu = cpu_baseline(layers, m)
        log(f"cpu {cpu['value']} GB/s on {cpu['cores']} cores")
        log("parity against the CPU path")
        parity = parity_report(layers, m, device)
        log(f"parity {json.dumps(parity)}")

    result = {
        "metric": "W8A8 GEMV HBM GB/s & GEMM int8 TOPS (% roofline) at M=1,8,560, LLaMA-7B",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"llama7b_decode_w8a8_linear_stack_{args.layers}L_plus_fp16_lm_head",
                   "m": m, "layers": args.layers,
                   "projections": {p.name: [p.n, p.k] for p in W.PROJECTIONS},
                   "lm_head": {"shape": [W.VOCAB, W.HIDDEN], "dtype": "fp16",
                               "op": ("dense_gemv: HIP fp16 GEMV, binary32 accumulation "
                                      "(not a W8A8 linear)" if m <= 16 else
                                      "torch F.linear (not a W8A8 linear)")},
                   "weights": "random-init ~N(0,0.02), per-output int8, packed",
                   "bytes_per_step": nbytes, "graph": True},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": parity,
        "extra": extra,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
