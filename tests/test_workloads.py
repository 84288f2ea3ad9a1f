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


def _ref_dit_block(blk: W.DiTBlock, x, e, ctx):
    """Float32 restatement of one AdaLN DiT block (explicit softmax attention)."""
    s = blk.s
    f = {k: v.float() for k, v in blk.state_dict().items()}
    x, e, ctx = x.float(), e.float(), ctx.float()
    m = [(f["modulation"] + e)[:, i: i + 1] for i in range(6)]

    def ln(v, w=None, b=None):
        mu = v.mean(-1, keepdim=True)
        var = ((v - mu) ** 2).mean(-1, keepdim=True)
        y = (v - mu) / torch.sqrt(var + s.eps)
        return y * w + b if w is not None else y

    def rms(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + s.eps) * w

    def attn(p, xq, xkv):
        q = rms(xq @ f[p + "q.weight"].T + f[p + "q.bias"], f[p + "norm_q.weight"])
        k = rms(xkv @ f[p + "k.weight"].T + f[p + "k.bias"], f[p + "norm_k.weight"])
        v = xkv @ f[p + "v.weight"].T + f[p + "v.bias"]
        hd = s.head_dim
        q = q.view(1, -1, s.n_heads, hd).transpose(1, 2)
        k = k.view(1, -1, s.n_heads, hd).transpose(1, 2)
        v = v.view(1, -1, s.n_heads, hd).transpose(1, 2)
        a = torch.softmax(q @ k.transpose(-1, -2) / math.sqrt(hd), -1)
        o = (a @ v).transpose(1, 2).reshape(1, -1, s.dim)
        return o @ f[p + "o.weight"].T + f[p + "o.bias"]

    h = ln(x) * (1 + m[1]) + m[0]
    x = x + attn("self_attn.", h, h) * m[2]
    x = x + attn("cross_attn.", ln(x, f["norm3.weight"], f["norm3.bias"]), ctx)
    h = ln(x) * (1 + m[4]) + m[3]
    y = torch.nn.functional.gelu(h @ f["fc1.weight"].T + f["fc1.bias"], approximate="tanh") @ f["fc2.weight"].T
    return x + (y + f["fc2.bias"]) * m[5]


def test_dit_block_matches_float32_restatement():
    shape = W.DiTShape(n_blocks=2, dim=64, n_heads=4, ffn=160)
    model = W.build_dit(shape, seed=7)
    with torch.no_grad():
        for p in model.parameters():  # norm weights around 1 so the test exercises them
            if p.dim() == 1 and p.numel() == 64 and p.abs().max() < 0.2:
                p.add_(1.0)
    x, e, ctx = W.dit_inputs(shape, 24, 8, seed=7)
    got = model(x, e, ctx)
    want = x
    for blk in model.blocks:
        want = _ref_dit_block(blk, want, e, ctx)
    rel = (got.float() - want).norm() / want.norm()
    assert rel < 2e-2, float(rel)
    assert sum(p.numel() for p in model.blocks[0].parameters()) == shape.block_params()
    assert W.WAN_DIT.block_params() * 2 == 702_788_608


def _dequantized_twin(model: W.LlamaModel) -> W.LlamaModel:
    """Float32 copy of an fp8 model with every projection replaced by W_fp8 * scale."""
    s = model.shape
    twin = W.build_llama(W.LlamaShape(**{**s.__dict__, "fp8": False}), seed=0).float()
    mods = dict(model.named_modules())
    sd = {}
    for name, p in model.named_parameters():
        owner = name.rsplit(".", 1)[0]
        if isinstance(mods.get(owner), W.Fp8Linear):
            if name.endswith(".weight"):
                sd[name] = mods[owner].weight.float() * mods[owner].scale.float()[:, None]
        else:
            sd[name] = p.detach().float()
    twin.load_state_dict(sd, strict=False)
    return twin


def test_fp8_llama_matches_dequantized_float32():
    shape = W.LlamaShape(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, inter=96, vocab=100,
                         max_seq=32, fp8=True)
    model = W.build_llama(shape, seed=3)
    fp8_linears = [m for m in model.modules() if isinstance(m, W.Fp8Linear)]
    assert len(fp8_linears) == 14 and all(m.weight.dtype == torch.float8_e4m3fn for m in fp8_linears)
    # per-channel scales put every row's absmax at the top of the e4m3 range
    w = fp8_linears[0].weight.float()
    assert torch.allclose(w.abs().amax(1), torch.full((w.shape[0],), 448.0), rtol=0.07)
    tokens = W.prompt_tokens(2, 6, shape.vocab, seed=3)
    model.init_cache(2, 32, torch.device("cpu"))
    twin = _dequantized_twin(model)
    twin.init_cache(2, 32, torch.device("cpu"))
    with torch.no_grad():
        got = model(tokens, 0)
        want = twin(tokens, 0)
    assert float((got - want).norm() / want.norm()) < 1e-2
    assert W.LLAMA_70B_FP8.layer_bytes() == 855_838_720


class _FakeGpuInput:
    """Only what ``Fp8Linear.kernel_eligible`` reads of an input on the GPU."""

    def __init__(self, m: int, k: int) -> None:
        self.shape = (m, k)
        self.is_cuda = True
        self.dtype = torch.bfloat16

    def numel(self) -> int:
        return self.shape[0] * self.shape[1]


def test_fp8_kernel_needs_an_aligned_weight():
    """A weight packed without alignment (raw_block_transfer) takes the dequantize path instead of raising."""
    lin = W.Fp8Linear(64, 32)
    x = _FakeGpuInput(8, 64)
    assert lin.kernel_eligible(x)
    raw = torch.empty(32 * 64 + 16, dtype=torch.uint8)
    for shift in (1, 8):
        lin.weight.data = raw[shift: shift + 32 * 64].view(torch.float8_e4m3fn).view(32, 64)
        assert lin.weight.data_ptr() % 16 and not lin.kernel_eligible(x)
    lin.weight.data = raw[16: 16 + 32 * 64].view(torch.float8_e4m3fn).view(32, 64)
    assert lin.kernel_eligible(x)
    assert lin.kernel_eligible(_FakeGpuInput(512, 64))  # prefill rows take the tiled kernel
    assert not lin.kernel_eligible(_FakeGpuInput(8, 24)) and not lin.kernel_eligible(_FakeGpuInput(0, 64))


def test_fp8_group_falls_back_when_the_group_reaches_the_launch_limit(monkeypatch):
    """One grouped launch takes at most 2^31 output elements in all (the library refuses m * sum(n) above it):
    a long prefill through gate/up, each layer eligible alone, runs them one by one instead of raising."""
    class _Input(_FakeGpuInput):
        def reshape(self, *shape):
            return self

    calls = []
    monkeypatch.setattr(W.hip, "fp8_linear_group", lambda x, ws, ss: calls.append(len(ws)) or
                        [torch.empty(x.shape[0], w.shape[0], device="meta") for w in ws])
    gate, up = W.Fp8Linear(16, 28672), W.Fp8Linear(16, 28672)
    long_prefill = _Input(65536, 16)  # 65536 * 57344 >= 2^31, each layer alone is 65536 * 28672 < 2^31
    assert gate.kernel_eligible(long_prefill) and up.kernel_eligible(long_prefill)
    assert W.fp8_group(long_prefill, [gate, up]) is None and calls == []
    assert W.fp8_group(_Input(32768, 16), [gate, up]) is not None and calls == [2]  # 32768 * 57344 < 2^31


def test_grouped_and_fused_calls_only_for_modules_that_run_nothing_else(monkeypatch):
    """The decoder computes a projection from its weights directly (grouped q/k/v and gate/up, the fused
    SwiGLU and residual epilogues) only when calling the module would run its class's forward and nothing
    else. An offload unit's trap (a forward set on the instance) or a hook sends the call through the module,
    so a streamed projection is loaded before it is read and hooks see their calls."""
    class _Input(_FakeGpuInput):
        def reshape(self, *shape):
            return self

        def numel(self) -> int:
            return self.shape[0] * self.shape[1]

    calls = []
    monkeypatch.setattr(W.hip, "fp8_linear_group", lambda x, ws, ss: calls.append("group") or
                        [torch.empty(x.shape[0], w.shape[0], device="meta") for w in ws])
    monkeypatch.setattr(W.hip, "fp8_linear_swiglu", lambda x, wg, sg, wu, su: calls.append("swiglu") or
                        torch.empty(x.shape[0], wg.shape[0], device="meta"))
    gate, up, down = W.Fp8Linear(16, 32), W.Fp8Linear(16, 32), W.Fp8Linear(32, 16)
    x = _Input(8, 16)
    assert W.fp8_group(x, [gate, up]) is not None and W.fp8_swiglu(x, gate, up) is not None
    assert calls == ["group", "swiglu"]
    calls.clear()
    up.forward = lambda t: t  # what an offload manager's trap looks like: a forward on the instance
    assert W.fp8_group(x, [gate, up]) is None and W.fp8_swiglu(x, gate, up) is None
    del up.forward
    handle = gate.register_forward_pre_hook(lambda mod, args: None)
    assert W.fp8_group(x, [gate, up]) is None and W.fp8_swiglu(x, gate, up) is None
    handle.remove()
    handle = torch.nn.modules.module.register_module_forward_hook(lambda mod, args, out: None)
    assert W.fp8_group(x, [gate, up]) is None
    handle.remove()
    assert calls == []
    # prefill rows take no fused epilogue (the decode kernel's reduce applies them), and unequal gate/up
    # shapes take no SwiGLU epilogue
    assert W.fp8_swiglu(_Input(65, 16), gate, up) is None
    assert W.fp8_swiglu(x, gate, W.Fp8Linear(16, 48)) is None
    resid = torch.empty(8, 16, dtype=torch.bfloat16, device="meta")
    assert W.fp8_residual(_Input(65, 32), down, torch.empty(65, 16, dtype=torch.bfloat16, device="meta")) is None
    assert W.fp8_residual(_Input(8, 32), down, resid.float()) is None
    assert calls == []


def test_decoder_layer_keeps_its_numerics_on_the_cpu():
    """Moving the residual adds into the attention call and the MLP step changes no bit on the host path:
    x + o and residual + o are the same bf16 add."""
    s = W.LlamaShape(n_layers=1, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, inter=96, vocab=32, max_seq=8)
    model = W.build_llama(s, seed=0)
    model.init_cache(2, 8, torch.device("cpu"))
    layer = model.layers[0]
    x = torch.randn(2, 3, 64).to(torch.bfloat16)
    with torch.no_grad():
        got = layer(x, 0, model.rope_cos, model.rope_sin, model.cache_k[0], model.cache_v[0])
        model.init_cache(2, 8, torch.device("cpu"))
        h = x + layer.attn(layer.attn_norm(x), 0, model.rope_cos, model.rope_sin, model.cache_k[0], model.cache_v[0])
        n2 = layer.mlp_norm(h)
        want = h + layer.down(torch.nn.functional.silu(layer.gate(n2)) * layer.up(n2))
    assert torch.equal(got, want)
