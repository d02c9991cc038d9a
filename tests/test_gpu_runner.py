"""The W8A8 decoder stack (runner.py) in the shape of LightweightLlamaRunner
(nanopointllm/llama/lightweight_runner.py:421-737).

Bars:
* packed QKV on the prologue's int8 rows equals the three separate W8A8
  projections, bit for bit (prefill uses the packed product instead of
  paged_attention.py:1349-1352);
* the runner equals the chain of its primitives bit for bit, and the same
  rows give the same bits whether they run as one prefill batch (MFMA GEMM),
  in decode chunks of 8 (GEMV) or one by one (fused decode kernel) when the
  attention core is row-local, for binary16 and bfloat16 models; the
  carried residual gives the bits of the per-layer add in both dtypes;
* every replay of a captured decode step equals the eager step for the same
  input, with eager work and synchronizations between the replays;
* the final residual add + norm (one prologue launch) gives the oracle's
  rounded sum and its LightweightRMSNorm within 2 ulps, almost all bit-equal;
* end to end, the logits stay within the int8 quantization error of a dense
  binary32 model with the same weights and attention (relative Frobenius
  error below 5%, cosine above 0.998); a wiring mistake (missing residual,
  k and v swapped) is far outside that.
"""
from __future__ import annotations

import copy
import sys

import pytest
import torch
import torch.nn.functional as F

from nanopointllm_amd.lm_head import dense_gemv
from workloads import LlamaShaped

pytestmark = pytest.mark.gpu


def note(msg):
    sys.__stderr__.write(f"[gpu-case] {msg}\n")
    sys.__stderr__.flush()


def _model(cuda, *, hidden=256, heads=4, kv_heads=2, inter=384, vocab=512, layers=2, seed=0,
           dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    m = LlamaShaped(hidden=hidden, heads=heads, kv_heads=kv_heads, intermediate=inter,
                    vocab=vocab, layers=layers)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif "embed" in name:
                p.copy_(torch.randn(p.shape, generator=g))
            else:
                p.copy_(torch.randn(p.shape, generator=g) / p.shape[-1] ** 0.5)
    return m.to(device=cuda, dtype=dtype)


def _expand_kv(t, heads):
    return t.repeat_interleave(heads // t.shape[1], dim=1)


def causal_core(q, k, v, layer_index, state):
    """Dense causal attention over the T rows, in binary32 with contiguous
    2-D-per-head products, cast back to the activation dtype."""
    t, heads, d = q.shape
    qf = q.float().permute(1, 0, 2).contiguous()
    kf = _expand_kv(k.float(), heads).permute(1, 2, 0).contiguous()      # [H, D, T]
    vf = _expand_kv(v.float(), heads).permute(1, 0, 2).contiguous()
    scores = torch.matmul(qf, kf) / d ** 0.5
    mask = torch.ones(t, t, dtype=torch.bool, device=q.device).triu(1)
    probs = scores.masked_fill(mask, float("-inf")).softmax(-1)
    return torch.matmul(probs, vf).permute(1, 0, 2).reshape(t, heads * d).to(q.dtype)


def rowlocal_core(q, k, v, layer_index, state):
    """A row-local stand-in for attention: each row's context depends on its
    own q, k and v only (so rows can be split across launches)."""
    t, heads, d = q.shape
    return (q + 0.5 * _expand_kv(k, heads) - _expand_kv(v, heads)).reshape(t, heads * d)


def _dense_reference(weights, input_ids, core, heads):
    """The same decoder in binary32 with the unquantized weights."""
    W = {k: v.float() for k, v in weights.items()}

    def norm(x, w):
        return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6))

    x = W["model.embed_tokens.weight"][input_ids[0]]
    i = 0
    while f"model.layers.{i}.self_attn.q_proj.weight" in W:
        p = f"model.layers.{i}."
        h = norm(x, W[p + "input_layernorm.weight"])
        q = (h @ W[p + "self_attn.q_proj.weight"].t()).view(h.shape[0], heads, -1)
        k = (h @ W[p + "self_attn.k_proj.weight"].t()).view(h.shape[0], -1, q.shape[-1])
        v = (h @ W[p + "self_attn.v_proj.weight"].t()).view(h.shape[0], -1, q.shape[-1])
        x = x + core(q, k, v, i, None) @ W[p + "self_attn.o_proj.weight"].t()
        h = norm(x, W[p + "post_attention_layernorm.weight"])
        act = F.silu(h @ W[p + "mlp.gate_proj.weight"].t()) * (h @ W[p + "mlp.up_proj.weight"].t())
        x = x + act @ W[p + "mlp.down_proj.weight"].t()
        i += 1
    return norm(x, W["model.norm.weight"]) @ W["lm_head.weight"].t()


def _runner(model, core, **kw):
    from nanopointllm_amd.runner import W8A8LlamaRunner
    return W8A8LlamaRunner(model, core, **kw)


@pytest.mark.parametrize("tokens", [5, 96])
def test_packed_qkv_equals_three_projections(cuda, tokens):
    from nanopointllm_amd import w8a8
    from nanopointllm_amd.inject import inject_w8a8

    model = _model(cuda)
    inject_w8a8(model)
    attn = model.model.layers[0].self_attn
    x = torch.randn(tokens, 256, generator=torch.Generator().manual_seed(tokens)).half().to(cuda)
    note(f"packed QKV vs q/k/v projections, T={tokens}")
    xq, sx = w8a8.rmsnorm_quant(x, model.model.layers[0].input_layernorm.weight, 1e-6)
    q, k, v = attn.w8a8_qkv.project_i8(xq, sx, out_dtype=torch.float16)
    for packed, proj in ((q, attn.q_proj), (k, attn.k_proj), (v, attn.v_proj)):
        sep = proj.forward_i8(xq, sx, out_dtype=torch.float16)
        assert torch.equal(packed.reshape(tokens, -1), sep)


@pytest.mark.parametrize("tokens", [3, 96])
def test_runner_is_the_chain_of_its_primitives(cuda, tokens):
    from nanopointllm_amd import w8a8

    model = _model(cuda)
    runner = _runner(model, causal_core)
    ids = torch.randint(0, 512, (1, tokens), generator=torch.Generator().manual_seed(1)).to(cuda)
    note(f"runner vs primitive chain, T={tokens}")
    logits = runner(ids)
    x = model.model.embed_tokens(ids)[0]
    for i, layer in enumerate(model.model.layers):
        xq, sx = w8a8.rmsnorm_quant(x, layer.input_layernorm.weight, 1e-6)
        q, k, v = layer.self_attn.w8a8_qkv.project_i8(xq, sx, out_dtype=torch.float16)
        a = layer.self_attn.o_proj(causal_core(q, k, v, i, None))
        r, xq, sx = w8a8.rmsnorm_quant(a, layer.post_attention_layernorm.weight, 1e-6, residual=x)
        x = r + layer.mlp.w8a8_mlp.forward_i8(xq, sx, out_dtype=torch.float16)
    norm = model.model.norm
    rows = w8a8.prologue_quant(x, norm_weight=norm.weight, eps=norm.variance_epsilon,
                               return_rows=True).rows
    # The LM head: the module's weight, on the dense GEMV up to 16 rows and
    # F.linear beyond.
    assert runner.lm_head.linear is model.lm_head
    expect = dense_gemv(rows, model.lm_head.weight) if tokens <= 16 else model.lm_head(rows)
    assert logits.shape == (1, tokens, 512)
    assert torch.equal(logits[0], expect)


@pytest.mark.parametrize("h_scale", [None, 0.05])
def test_runner_within_quantization_error_of_dense_fp32(cuda, h_scale):
    model = _model(cuda)
    weights = {k: v.detach().clone() for k, v in model.state_dict().items()}
    h_scales = None if h_scale is None else {0: h_scale, 1: h_scale}
    runner = _runner(model, causal_core, h_scales=h_scales)
    ids = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(2)).to(cuda)
    note(f"runner vs dense fp32, h_scale={h_scale}")
    got = runner(ids)[0].float()
    ref = _dense_reference(weights, ids, causal_core, heads=4)
    rel = float((got - ref).norm() / ref.norm())
    cos = float(F.cosine_similarity(got.flatten(), ref.flatten(), dim=0))
    note(f"  rel {rel:.4f} cos {cos:.5f}")
    assert rel < 0.05 and cos > 0.998

    def swapped(q, k, v, i, s):
        return causal_core(q, v, k, i, s)
    bad = _dense_reference(weights, ids, swapped, heads=4)
    assert float((bad - ref).norm() / ref.norm()) > 0.2     # the bar separates wiring mistakes


@pytest.fixture(scope="module")
def llama7b_layer(cuda):
    """One decoder layer at LLaMA-7B sizes (hidden 4096, 32 heads, MLP
    11008), so decode rows take the GEMV and fused decode kernels."""
    return _model(cuda, hidden=4096, heads=32, kv_heads=32, inter=11008, vocab=256, layers=1,
                  seed=7)


def _check_rows_across_paths(runner, x, step: int, singles: int) -> None:
    """The final-norm rows of one batch, of chunks of `step` rows and of
    single rows are bit-equal (every W8A8 kernel path); the logits of chunks
    and single rows too (both on the dense GEMV), and the batch's (torch's
    GEMM past 16 rows) within two output ulps of them."""
    head = runner.lm_head
    runner.lm_head = torch.nn.Identity()
    try:
        whole = runner(inputs_embeds=x)
        chunks = torch.cat([runner(inputs_embeds=x[:, i:i + step])
                            for i in range(0, x.shape[1], step)], dim=1)
        assert torch.equal(whole, chunks)
        ones = torch.cat([runner(inputs_embeds=x[:, i:i + 1]) for i in range(singles)], dim=1)
        assert torch.equal(whole[:, :singles], ones)
    finally:
        runner.lm_head = head
    w = head.linear.weight
    logits = runner(inputs_embeds=x)
    assert torch.equal(logits, head.linear(whole))
    spans = range(0, x.shape[1], step)
    chunk_logits = torch.cat([runner(inputs_embeds=x[:, i:i + step]) for i in spans], dim=1)
    assert torch.equal(chunk_logits,
                       torch.cat([dense_gemv(whole[:, i:i + step], w) for i in spans], dim=1))
    one_logits = torch.cat([runner(inputs_embeds=x[:, i:i + 1]) for i in range(singles)], dim=1)
    assert torch.equal(one_logits, chunk_logits[:, :singles])
    # Two roundings of binary32 sums: within two output ulps plus the
    # accumulation bound K * 2^-24 * sum |x w| of each.
    ulp = 2.0 ** (torch.floor(torch.log2(logits.float().abs().clamp_min(2.0 ** -30)))
                  - (10 if x.dtype == torch.float16 else 7))
    mag = whole.float().abs() @ w.float().abs().t()
    tol = 2 * ulp + 2 * w.shape[1] * 2.0 ** -24 * mag
    assert ((chunk_logits.float() - logits.float()).abs() <= tol).all()


def test_rows_give_the_same_bits_on_every_kernel_path(cuda, llama7b_layer):
    model = copy.deepcopy(llama7b_layer)
    runner = _runner(model, rowlocal_core)
    x = torch.randn(1, 96, 4096, generator=torch.Generator().manual_seed(3)).half().to(cuda)
    note("runner rows: prefill GEMM vs decode chunks of 8 vs single rows")
    _check_rows_across_paths(runner, x, 8, 12)

def test_bf16_rows_give_the_same_bits_on_every_kernel_path(cuda):
    """As above for a bfloat16 model: one prefill batch (MFMA GEMM), decode
    chunks of 8 and single rows (fused decode kernels) give the same bits up to
    the LM head."""
    model = _model(cuda, hidden=4096, heads=32, kv_heads=32, inter=11008, vocab=256, layers=1,
                   seed=17, dtype=torch.bfloat16)
    runner = _runner(model, rowlocal_core)
    x = torch.randn(1, 80, 4096, generator=torch.Generator().manual_seed(4)).bfloat16().to(cuda)
    note("bf16 runner rows: prefill GEMM vs decode chunks of 8 vs single rows")
    assert runner(inputs_embeds=x[:, :2]).dtype == torch.bfloat16
    _check_rows_across_paths(runner, x, 8, 6)


@pytest.mark.parametrize("rows,dtype", [(1, torch.float16), (8, torch.float16),
                                        (40, torch.float16), (8, torch.bfloat16),
                                        (40, torch.bfloat16)])
def test_carried_residual_equals_the_per_layer_add(cuda, rows, dtype):
    """The runner leaves each layer's final residual add to the next layer's
    RMSNorm + QKV launch (forward_carry); two LLaMA-7B-size layers, so the
    second QKV takes the carried residual, on the fused decode kernel (rows 1
    and 8) and the activation prologue + 17-64-row GEMV route (40 rows).  Bits
    equal to a stack of
    the reference-form layer.forward calls (lightweight_runner.py:552)."""
    model = _model(cuda, hidden=4096, heads=32, kv_heads=32, inter=11008, vocab=256, layers=2,
                   seed=11, dtype=dtype)
    runner = _runner(model, rowlocal_core)
    x = torch.randn(1, rows, 4096, generator=torch.Generator().manual_seed(rows)).to(dtype).to(cuda)
    note(f"carried residual vs per-layer add, rows={rows}, {dtype}")
    got = runner(inputs_embeds=x)
    h = x
    for layer in runner.layers:
        h = layer(h)
    assert torch.equal(got, runner.lm_head(runner.final_norm(h[0], None).view(h.shape)))


@pytest.mark.parametrize("rows,dtype", [(1, torch.float16), (8, torch.float16),
                                        (8, torch.bfloat16), (560, torch.float16)])
def test_final_norm_is_lightweight_rmsnorm(cuda, rows, dtype):
    """The runner's final residual add + norm (one prologue launch) against
    the oracle's ``LightweightRMSNorm`` (lightweight_runner.py:239-257) of the
    rounded sum: the sum bit-exact, the normalized rows within 2 ulps and
    almost all bit-equal (binary32 sums of squares in another order); and
    within 2 ulps of the model's own torch module."""
    import numpy as np
    from oracle import w8a8_oracle as O

    model = _model(cuda, hidden=4096, heads=32, kv_heads=32, inter=256, vocab=64, layers=1,
                   seed=13)
    runner = _runner(model, rowlocal_core)
    norm = runner.norm
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(4096, generator=torch.Generator().manual_seed(5)))
        norm.weight.data = norm.weight.data.to(dtype)
    g = torch.Generator().manual_seed(rows)
    hid = (torch.randn(rows, 4096, generator=g) * 2).to(dtype)
    res = (torch.randn(rows, 4096, generator=g) * 0.5).to(dtype)
    note(f"final norm vs LightweightRMSNorm, rows={rows}, {dtype}")
    got = runner.final_norm(hid.to(cuda), res.to(cuda))
    assert got.dtype == dtype and got.shape == (rows, 4096)
    name = "f16" if dtype == torch.float16 else "bf16"
    summed = O.residual_add(hid.float().numpy(), res.float().numpy(), name)
    want = O.rmsnorm(summed, norm.weight.detach().float().cpu().numpy(), norm.variance_epsilon,
                     name)
    ulps = _ulps16(got.cpu(), torch.from_numpy(want).to(dtype))
    assert ulps.max() <= 2 and np.count_nonzero(ulps) <= max(2, ulps.size // 1000)
    with torch.no_grad():
        ref = norm((hid + res).to(cuda)).cpu()
    assert _ulps16(got.cpu(), ref).max() <= 2


def _ulps16(a: torch.Tensor, b: torch.Tensor):
    key = lambda t: (lambda i: torch.where(i < 0, -(i & 0x7FFF), i))(t.view(torch.int16).int())
    return (key(a) - key(b)).abs().numpy()


@pytest.mark.parametrize("rows", [1, 8, 96])
def test_decode_graph_replays_match_eager(cuda, llama7b_layer, rows):
    """Replays of a captured step equal the eager step: decode rows on the
    fused kernels (8 rows with the static int8 MLP chain), and 96 prefill
    rows on the prologue + GEMM route, whose workspaces come from torch's
    allocator during capture."""
    from nanopointllm_amd.runner import DecodeGraphBucket

    model = copy.deepcopy(llama7b_layer)
    runner = _runner(model, rowlocal_core, h_scales={0: 0.02} if rows == 8 else None)
    g = torch.Generator().manual_seed(rows)
    inputs = [torch.randn(1, rows, 4096, generator=g).half().to(cuda) for _ in range(3)]
    eager = [runner(inputs_embeds=x).clone() for x in inputs]
    static = torch.zeros_like(inputs[0])
    bucket = DecodeGraphBucket(cuda)
    note(f"capture decode step, rows={rows}")
    out = bucket.capture(lambda: runner(inputs_embeds=static))
    for rep in range(2):
        for x, e in zip(inputs, eager):
            static.copy_(x)
            got = bucket.replay()
            torch.cuda.synchronize()
            assert torch.equal(got, e), f"replay {rep} differs from eager"
            # eager work between replays
            runner(inputs_embeds=inputs[0])
    assert out is bucket.static_output


def test_layer_requires_injection(cuda):
    from nanopointllm_amd.runner import W8A8LlamaLayer

    model = _model(cuda)
    with pytest.raises(ValueError, match="inject_w8a8"):
        W8A8LlamaLayer(model.model.layers[0], 0, causal_core)
    with pytest.raises(ValueError, match="input_ids or inputs_embeds"):
        _runner(model, causal_core)()
