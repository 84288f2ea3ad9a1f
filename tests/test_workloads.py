"""CPU checks of the synthetic workloads against independent float32 restatements."""

from __future__ import annotations

import math

import torch

from flextensor_amd import workloads as W


def _ref_llama_logits(model: W.LlamaModel, tokens: torch.Tensor) -> torch.Tensor:
    """Plain float32 Llama forward (full causal attention, complex-number RoPE)."""
    s = model.shape
    f = {k: v.float() for k, v in model.state_dict().items()}
    x = f["embed.weight"][tokens]
    t = tokens.shape[1]
    inv = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2).float() / s.head_dim))
    ang = torch.outer(torch.arange(t).float(), inv)
    rot = torch.polar(torch.ones_like(ang), ang)  # e^{i * angle}

    def rope(v):  # v: [b, t, h, d]; pairs (j, j + d/2) form one complex number
        half = v.shape[-1] // 2
        c = torch.complex(v[..., :half], v[..., half:]) * rot.view(1, t, 1, half)
        return torch.cat([c.real, c.imag], -1)

    def norm(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + s.eps) * w

    for i in range(s.n_layers):
        p = f"layers.{i}."
        h = norm(x, f[p + "attn_norm.weight"])
        q = (h @ f[p + "attn.wq.weight"].T).view(1, t, s.n_heads, s.head_dim)
        k = (h @ f[p + "attn.wk.weight"].T).view(1, t, s.n_kv_heads, s.head_dim)
        v = (h @ f[p + "attn.wv.weight"].T).view(1, t, s.n_kv_heads, s.head_dim)
        q, k = rope(q), rope(k)
        att = torch.einsum("bqhd,bkhd->bhqk", q, k) / math.sqrt(s.head_dim)
        att = att.masked_fill(torch.ones(t, t).triu(1).bool(), float("-inf")).softmax(-1)
        o = torch.einsum("bhqk,bkhd->bqhd", att, v).reshape(1, t, -1)
        x = x + o @ f[p + "attn.wo.weight"].T
        h = norm(x, f[p + "mlp_norm.weight"])
        g = h @ f[p + "gate.weight"].T
        x = x + (torch.nn.functional.silu(g) * (h @ f[p + "up.weight"].T)) @ f[p + "down.weight"].T
    x = norm(x, f["norm.weight"])
    return (x[:, -1:] @ f["lm_head.weight"].T)


def test_tiny_llama_matches_float32_restatement():
    shape = W.LlamaShape(n_layers=2, hidden=64, n_heads=4, n_kv_heads=4, head_dim=16, inter=96, vocab=100, max_seq=32)
    model = W.build_llama(shape, seed=5)
    tokens = W.prompt_tokens(1, 12, shape.vocab, seed=5)
    model.init_cache(1, 32, torch.device("cpu"))
    got = model(tokens, 0)
    want = _ref_llama_logits(model, tokens)
    rel = (got - want).norm() / want.norm()
    assert rel < 2e-2, float(rel)  # bf16 model vs float32 restatement


def test_incremental_decode_matches_full_prefill():
    shape = W.LlamaShape(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, inter=96, vocab=100, max_seq=32)
    model = W.build_llama(shape, seed=6).float()
    tokens = W.prompt_tokens(1, 10, shape.vocab, seed=6)
    model.init_cache(1, 32, torch.device("cpu"))
    full = model(tokens, 0)
    model.init_cache(1, 32, torch.device("cpu"))
    model(tokens[:, :7], 0)
    for i in range(7, 10):
        step = model(tokens[:, i: i + 1], i)
    assert torch.allclose(step, full, atol=1e-4, rtol=1e-4)


def test_mlp_layer_sizes_and_packing():
    model = W.build_mlp_stack(2, 64, 176, seed=0)
    sizes = [p.numel() * 2 for p in model.layers[0].parameters()]
    assert sizes == [176 * 64 * 2, 176 * 2, 64 * 176 * 2, 64 * 2]
    assert W.LLAMA_7B.layer_bytes() == 404_766_720  # 7B-shape decoder layer in bf16


def test_scatter_set_shapes():
    sizes = W.scatter_sizes(2000, 4096, 64 << 20, seed=1)
    assert len(sizes) == 2000 and min(sizes) >= 4094 and max(sizes) <= 64 << 20
    assert all(n % 2 == 0 for n in sizes)
    for i, n in enumerate(sizes[:50]):
        shape = W.scatter_shape(n, i)
        assert math.prod(shape) * 2 == n and len(shape) == (1 if i % 2 == 0 else 2)
    assert 12e9 < sum(sizes) < 15e9
