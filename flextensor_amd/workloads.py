"""Synthetic, seeded workloads that exercise the streaming path.

* :func:`build_mlp_stack` - n x [Linear(h -> i, bias) -> SiLU -> Linear(i -> h, bias)]
  (8 layers at 4096 -> 11008 -> 4096 for the MLP-stack workload).
* :class:`LlamaModel` - Llama-style decoder: RMSNorm, rotary attention with a
  KV cache, SwiGLU MLP (32 layers, hidden 4096, 32 x 128 heads, 11008
  intermediate, vocab 32000 for the 7B shape).
* :func:`scatter_tensor_set` - the tensor set of the scatter microbenchmark:
  byte sizes log-uniform in [4 KiB, 64 MiB], bf16, 1-D or 2-D shapes.

Weights are drawn N(0, 0.02) in float32 from one ``torch.Generator`` seeded
with ``seed``, parameter by parameter in module registration order, then
cast to bfloat16. ``init_device="cuda"`` draws on the device generator (fast
for multi-GB models) and copies the result into CPU tensors; the two devices
give different (each deterministic) weights.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from . import hip


FP8_E4M3_MAX = 448.0


def init_normal_(model: nn.Module, seed: int, std: float = 0.02, init_device: str = "cpu") -> nn.Module:
    """Overwrite every parameter with N(0, std) draws (float32, then cast).

    An ``Fp8Linear`` draws its weight the same way, then stores it as
    float8_e4m3fn with a per-output-channel scale ``absmax / 448`` (bf16); the
    quantised weight is ``round_e4m3(w / scale)``.
    """
    gen = torch.Generator(device=init_device).manual_seed(seed)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, Fp8Linear):
                w = torch.empty(mod.weight.shape, dtype=torch.float32, device=init_device)
                w.normal_(0.0, std, generator=gen)
                scale = (w.abs().amax(dim=1) / FP8_E4M3_MAX).clamp_min(1e-12).to(torch.bfloat16)
                mod.weight.copy_((w / scale.float()[:, None]).to(torch.float8_e4m3fn))
                mod.scale.copy_(scale)
                continue
            for p in mod.parameters(recurse=False):
                w = torch.empty(p.shape, dtype=torch.float32, device=init_device)
                w.normal_(0.0, std, generator=gen)
                p.copy_(w.to(p.dtype))
    return model


class MLPBlock(nn.Module):
    def __init__(self, hidden: int, inter: int, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.fc1 = nn.Linear(hidden, inter, bias=True, dtype=dtype)
        self.fc2 = nn.Linear(inter, hidden, bias=True, dtype=dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.fc2(F.silu(self.fc1(x)))


class MLPStack(nn.Module):
    def __init__(self, n_layers: int, hidden: int, inter: int, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.layers = nn.ModuleList(MLPBlock(hidden, inter, dtype) for _ in range(n_layers))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x)
        return x


def build_mlp_stack(n_layers: int = 8, hidden: int = 4096, inter: int = 11008, seed: int = 0,
                    init_device: str = "cpu") -> MLPStack:
    with torch.device("meta"):
        model = MLPStack(n_layers, hidden, inter)
    model = model.to_empty(device="cpu")
    return init_normal_(model, seed, 0.02, init_device)


def mlp_input(batch: int = 16, hidden: int = 4096, seed: int = 0) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(batch, hidden, generator=gen, dtype=torch.float32).to(torch.bfloat16)


# ---- Llama-style decoder -----------------------------------------------------


@dataclass(frozen=True)
class LlamaShape:
    n_layers: int = 32
    hidden: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 32
    head_dim: int = 128
    inter: int = 11008
    vocab: int = 32000
    max_seq: int = 2048
    eps: float = 1e-5
    rope_theta: float = 10000.0
    fp8: bool = False  # projection weights in float8_e4m3fn with per-output-channel bf16 scales

    def layer_bytes(self, itemsize: int = 2) -> int:
        h, d = self.hidden, self.head_dim
        mats = h * self.n_heads * d + 2 * h * self.n_kv_heads * d + self.n_heads * d * h + 3 * h * self.inter
        if self.fp8:
            outs = self.n_heads * d + 2 * self.n_kv_heads * d + h + 2 * self.inter + h
            return mats + 2 * outs + 2 * 2 * h
        return itemsize * (mats + 2 * h)


LLAMA_7B = LlamaShape()
LLAMA_70B_FP8 = LlamaShape(n_layers=80, hidden=8192, n_heads=64, n_kv_heads=8, head_dim=128, inter=28672,
                           vocab=32000, max_seq=4096, fp8=True)


class Fp8Linear(nn.Module):
    """y = x @ (W_fp8 * scale[:, None])^T with W in float8_e4m3fn and a bf16 scale per output channel.

    On the GPU (K a multiple of 16) the library's fp8-weight MFMA kernels run:
    up to 64 rows (decode) a split-K kernel that reads each fp8 weight once,
    more rows (prefill) a tiled GEMM; both widen the weights to bf16 in
    registers. The decoder groups its q/k/v and gate/up projections into one
    launch each (:func:`fp8_group`). CPU inputs dequantise to bf16 and run a
    bf16 GEMM. Every e4m3 value is exactly
    representable in bf16, so both compute the same products; they differ in
    accumulation order and in rounding the product before the scale.
    """

    def __init__(self, in_features: int, out_features: int) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=torch.float8_e4m3fn),
                                   requires_grad=False)
        self.scale = nn.Parameter(torch.ones(out_features, dtype=torch.bfloat16), requires_grad=False)

    def kernel_eligible(self, x: torch.Tensor) -> bool:
        """Whether the library kernels take this call: a non-empty bf16 GPU input with K a multiple of
        16, and a contiguous, 16-byte aligned weight (``raw_block_transfer`` packs weights back to back
        without alignment; such a weight takes the dequantize path)."""
        k = x.shape[-1]
        m = x.numel() // k if k else 0
        w = self.weight
        return (x.is_cuda and x.dtype == torch.bfloat16 and m > 0 and k % 16 == 0 and m * w.shape[0] < 2**31
                and w.is_contiguous() and w.data_ptr() % 16 == 0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.kernel_eligible(x):
            k = x.shape[-1]
            y = hip.fp8_linear(x.reshape(x.numel() // k, k), self.weight, self.scale)
            return y.view(*x.shape[:-1], y.shape[-1])
        w = self.weight.to(torch.bfloat16)
        return F.linear(x, w) * self.scale


def _plain_call(module: nn.Module) -> bool:
    """Whether calling ``module`` would run its class's forward and nothing else: no forward set on the
    instance (an offload manager's enter/exit trap is one) and no forward hooks. Only then may a caller
    compute the module's output from its weights directly, in a grouped or fused launch."""
    from torch.nn.modules import module as torch_module

    return ("forward" not in module.__dict__ and not module._forward_hooks and not module._forward_pre_hooks
            and not torch_module._global_forward_hooks and not torch_module._global_forward_pre_hooks)


def fp8_group(x: torch.Tensor, layers: list[nn.Module]) -> list[torch.Tensor] | None:
    """The outputs of several ``Fp8Linear`` layers on one input in one grouped kernel launch, or None when
    any of them would not take the kernel, would run more than its own forward when called (an offload
    unit's trap, a hook), or the group's outputs together would reach 2^31 elements, the library's limit
    for one launch (the caller then runs them one by one)."""
    if not all(isinstance(lin, Fp8Linear) and lin.kernel_eligible(x) and _plain_call(lin) for lin in layers):
        return None
    k = x.shape[-1]
    if (x.numel() // k) * sum(lin.weight.shape[0] for lin in layers) >= 2**31:
        return None
    ys = hip.fp8_linear_group(x.reshape(x.numel() // k, k), [lin.weight for lin in layers],
                              [lin.scale for lin in layers])
    return [y.view(*x.shape[:-1], y.shape[-1]) for y in ys]


def _fusable(x: torch.Tensor, layers: list[nn.Module]) -> bool:
    """Whether a decode-batch call of these ``Fp8Linear`` layers on ``x`` can take a fused epilogue."""
    k = x.shape[-1]
    return (all(isinstance(lin, Fp8Linear) and lin.kernel_eligible(x) and _plain_call(lin) for lin in layers)
            and x.numel() // k <= hip.FP8_DECODE_MAX_ROWS)


def fp8_swiglu(x: torch.Tensor, gate: nn.Module, up: nn.Module) -> torch.Tensor | None:
    """``F.silu(gate(x)) * up(x)`` as one grouped launch whose reduce applies the activation, or None when
    the fused form does not apply (the caller then runs the layers and the activation as usual)."""
    if not _fusable(x, [gate, up]) or gate.weight.shape != up.weight.shape:
        return None
    k = x.shape[-1]
    y = hip.fp8_linear_swiglu(x.reshape(x.numel() // k, k), gate.weight, gate.scale, up.weight, up.scale)
    return y.view(*x.shape[:-1], y.shape[-1])


def fp8_residual(x: torch.Tensor, lin: nn.Module, residual: torch.Tensor) -> torch.Tensor | None:
    """``residual + lin(x)`` with the add folded into the linear's reduce, or None when the fused form
    does not apply (the caller then adds as usual)."""
    if not _fusable(x, [lin]) or residual.dtype != torch.bfloat16 or \
            residual.shape != (*x.shape[:-1], lin.weight.shape[0]):
        return None
    k = x.shape[-1]
    m = x.numel() // k
    y = hip.fp8_linear_residual(x.reshape(m, k), lin.weight, lin.scale, residual.reshape(m, -1))
    return y.view(residual.shape)


def _proj(s: LlamaShape, n_in: int, n_out: int, dtype: torch.dtype) -> nn.Module:
    return Fp8Linear(n_in, n_out) if s.fp8 else nn.Linear(n_in, n_out, bias=False, dtype=dtype)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float, dtype: torch.dtype) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotary embedding with full-width cos/sin tables (halves rotate against each other)."""
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rotated * sin


class Attention(nn.Module):
    def __init__(self, s: LlamaShape, dtype: torch.dtype) -> None:
        super().__init__()
        self.s = s
        self.wq = _proj(s, s.hidden, s.n_heads * s.head_dim, dtype)
        self.wk = _proj(s, s.hidden, s.n_kv_heads * s.head_dim, dtype)
        self.wv = _proj(s, s.hidden, s.n_kv_heads * s.head_dim, dtype)
        self.wo = _proj(s, s.n_heads * s.head_dim, s.hidden, dtype)

    def forward(self, x: torch.Tensor, pos: int, cos: torch.Tensor, sin: torch.Tensor,
                cache_k: torch.Tensor, cache_v: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """The attention block's output, plus ``residual`` when given (folded into the output projection's
        reduce for fp8 decode batches)."""
        s = self.s
        b, t, _ = x.shape
        qkv = fp8_group(x, [self.wq, self.wk, self.wv])
        q, k, v = qkv if qkv is not None else (self.wq(x), self.wk(x), self.wv(x))
        q = q.view(b, t, s.n_heads, s.head_dim)
        k = k.view(b, t, s.n_kv_heads, s.head_dim)
        v = v.view(b, t, s.n_kv_heads, s.head_dim)
        c = cos[pos: pos + t].view(1, t, 1, -1).to(q.dtype)
        sn = sin[pos: pos + t].view(1, t, 1, -1).to(q.dtype)
        q, k = _rotate(q, c, sn), _rotate(k, c, sn)
        cache_k[:b, pos: pos + t] = k
        cache_v[:b, pos: pos + t] = v
        keys = cache_k[:b, : pos + t]
        vals = cache_v[:b, : pos + t]
        rep = s.n_heads // s.n_kv_heads
        if rep > 1:
            keys = keys.repeat_interleave(rep, dim=2)
            vals = vals.repeat_interleave(rep, dim=2)
        qh = q.transpose(1, 2).contiguous()                    # [b, h, t, d]
        kt = keys.permute(0, 2, 3, 1).contiguous()             # [b, h, d, S]  (contiguous right operand)
        vh = vals.transpose(1, 2).contiguous()                 # [b, h, S, d]
        scores = torch.matmul(qh, kt).float() * (1.0 / math.sqrt(s.head_dim))
        if t > 1:
            n = pos + t
            mask = torch.ones(t, n, dtype=torch.bool, device=x.device).triu(diagonal=pos + 1)
            scores = scores.masked_fill(mask, float("-inf"))
        p = torch.softmax(scores, dim=-1).to(vh.dtype)
        o = torch.matmul(p, vh).transpose(1, 2).reshape(b, t, s.n_heads * s.head_dim)
        if residual is None:
            return self.wo(o)
        fused = fp8_residual(o, self.wo, residual)
        return fused if fused is not None else residual + self.wo(o)


class DecoderLayer(nn.Module):
    def __init__(self, s: LlamaShape, dtype: torch.dtype) -> None:
        super().__init__()
        self.attn_norm = RMSNorm(s.hidden, s.eps, dtype)
        self.attn = Attention(s, dtype)
        self.mlp_norm = RMSNorm(s.hidden, s.eps, dtype)
        self.gate = _proj(s, s.hidden, s.inter, dtype)
        self.up = _proj(s, s.hidden, s.inter, dtype)
        self.down = _proj(s, s.inter, s.hidden, dtype)

    def forward(self, x: torch.Tensor, pos: int, cos: torch.Tensor, sin: torch.Tensor,
                cache_k: torch.Tensor, cache_v: torch.Tensor) -> torch.Tensor:
        x = self.attn(self.attn_norm(x), pos, cos, sin, cache_k, cache_v, residual=x)
        h = self.mlp_norm(x)
        act = fp8_swiglu(h, self.gate, self.up)
        if act is None:
            gu = fp8_group(h, [self.gate, self.up])
            g, u = gu if gu is not None else (self.gate(h), self.up(h))
            act = F.silu(g) * u
        out = fp8_residual(act, self.down, x)
        return out if out is not None else x + self.down(act)


class LlamaModel(nn.Module):
    def __init__(self, s: LlamaShape = LLAMA_7B, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.shape = s
        self.embed = nn.Embedding(s.vocab, s.hidden, dtype=dtype)
        self.layers = nn.ModuleList(DecoderLayer(s, dtype) for _ in range(s.n_layers))
        self.norm = RMSNorm(s.hidden, s.eps, dtype)
        self.lm_head = nn.Linear(s.hidden, s.vocab, bias=False, dtype=dtype)
        inv = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, dtype=torch.float32) / s.head_dim))
        ang = torch.outer(torch.arange(s.max_seq, dtype=torch.float32), inv)
        self.register_buffer("rope_cos", torch.cat([ang.cos(), ang.cos()], -1), persistent=False)
        self.register_buffer("rope_sin", torch.cat([ang.sin(), ang.sin()], -1), persistent=False)
        self.cache_k: list[torch.Tensor] = []
        self.cache_v: list[torch.Tensor] = []

    def init_cache(self, batch: int, max_len: int, device: torch.device) -> None:
        s = self.shape
        shape = (batch, max_len, s.n_kv_heads, s.head_dim)
        dt = self.embed.weight.dtype
        self.cache_k = [torch.zeros(shape, dtype=dt, device=device) for _ in range(s.n_layers)]
        self.cache_v = [torch.zeros(shape, dtype=dt, device=device) for _ in range(s.n_layers)]

    def forward(self, tokens: torch.Tensor, pos: int = 0) -> torch.Tensor:
        """Logits of the last position, float32."""
        x = self.embed(tokens)
        for i, layer in enumerate(self.layers):
            x = layer(x, pos, self.rope_cos, self.rope_sin, self.cache_k[i], self.cache_v[i])
        return self.lm_head(self.norm(x[:, -1:])).float()


def build_llama(shape: LlamaShape = LLAMA_7B, seed: int = 0, init_device: str = "cpu") -> LlamaModel:
    with torch.device("meta"):
        model = LlamaModel(shape)
    model = model.to_empty(device="cpu")
    s = shape
    inv = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, dtype=torch.float32) / s.head_dim))
    ang = torch.outer(torch.arange(s.max_seq, dtype=torch.float32), inv)
    model.rope_cos.copy_(torch.cat([ang.cos(), ang.cos()], -1))
    model.rope_sin.copy_(torch.cat([ang.sin(), ang.sin()], -1))
    return init_normal_(model, seed, 0.02, init_device)


@torch.no_grad()
def generate(model: LlamaModel, prompt: torch.Tensor, steps: int) -> tuple[torch.Tensor, list[torch.Tensor]]:
    """Greedy decoding with no host synchronisation between steps.

    Returns the generated tokens ``[batch, steps]`` and the logits of every step.
    """
    logits = model(prompt, 0)
    out, all_logits = [], [logits]
    tok = logits.argmax(-1)
    pos = prompt.shape[1]
    for _ in range(steps - 1):
        out.append(tok)
        logits = model(tok, pos)
        all_logits.append(logits)
        tok = logits.argmax(-1)
        pos += 1
    out.append(tok)
    return torch.cat(out, dim=1), all_logits


def prompt_tokens(batch: int, length: int, vocab: int, seed: int = 0) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (batch, length), generator=gen)


# ---- Wan-style diffusion transformer -------------------------------------------


@dataclass(frozen=True)
class DiTShape:
    n_blocks: int = 40
    dim: int = 5120
    n_heads: int = 40
    ffn: int = 13824
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads

    def block_params(self) -> int:
        d, f = self.dim, self.ffn
        attn = 4 * (d * d + d) + 2 * d  # q, k, v, o with bias + q/k RMSNorm weights
        return 2 * attn + 2 * d + (d * f + f + f * d + d) + 6 * d  # + cross-attn norm, ffn, modulation

    def block_flops(self, tokens: int, text: int) -> float:
        d, f = self.dim, self.ffn
        lin = 2 * tokens * d * d * 4 + 2 * tokens * d * d * 2 + 2 * text * d * d * 2 + 2 * tokens * d * f * 2
        attn = 4 * tokens * tokens * d + 4 * tokens * text * d
        return float(lin + attn)


WAN_DIT = DiTShape()


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Attention over [batch, heads, seq, head_dim].

    On the GPU only the fused flash / memory-efficient kernels are allowed (a
    32760-token score matrix does not belong in HBM, and the unfused path runs
    batched products on transposed views); without a fused kernel this raises.
    """
    if q.device.type == "cuda":
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v)
    return F.scaled_dot_product_attention(q, k, v)


class _DiTAttention(nn.Module):
    def __init__(self, s: DiTShape, dtype: torch.dtype) -> None:
        super().__init__()
        self.s = s
        self.q = nn.Linear(s.dim, s.dim, dtype=dtype)
        self.k = nn.Linear(s.dim, s.dim, dtype=dtype)
        self.v = nn.Linear(s.dim, s.dim, dtype=dtype)
        self.o = nn.Linear(s.dim, s.dim, dtype=dtype)
        self.norm_q = RMSNorm(s.dim, s.eps, dtype)
        self.norm_k = RMSNorm(s.dim, s.eps, dtype)

    def forward(self, x: torch.Tensor, ctx: torch.Tensor, attn=None) -> torch.Tensor:
        b, n, _ = x.shape
        h, d = self.s.n_heads, self.s.head_dim
        q = self.norm_q(self.q(x)).view(b, n, h, d).transpose(1, 2)
        k = self.norm_k(self.k(ctx)).view(b, ctx.shape[1], h, d).transpose(1, 2)
        v = self.v(ctx).view(b, ctx.shape[1], h, d).transpose(1, 2)
        o = (attn or sdpa)(q, k, v)
        return self.o(o.transpose(1, 2).reshape(b, n, h * d))


class DiTBlock(nn.Module):
    """AdaLN-modulated block: self-attention, cross-attention to text, GELU FFN."""

    def __init__(self, s: DiTShape = WAN_DIT, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.s = s
        self.self_attn = _DiTAttention(s, dtype)
        self.cross_attn = _DiTAttention(s, dtype)
        self.norm3 = nn.LayerNorm(s.dim, eps=s.eps, dtype=dtype)
        self.fc1 = nn.Linear(s.dim, s.ffn, dtype=dtype)
        self.fc2 = nn.Linear(s.ffn, s.dim, dtype=dtype)
        self.modulation = nn.Parameter(torch.zeros(1, 6, s.dim, dtype=dtype))

    def _norm(self, x: torch.Tensor) -> torch.Tensor:
        return F.layer_norm(x.float(), (self.s.dim,), eps=self.s.eps).to(x.dtype)

    def forward(self, x: torch.Tensor, e: torch.Tensor, ctx: torch.Tensor, attn=None) -> torch.Tensor:
        m = (self.modulation.float() + e.float()).chunk(6, dim=1)
        h = (self._norm(x).float() * (1 + m[1]) + m[0]).to(x.dtype)
        x = (x.float() + self.self_attn(h, h, attn).float() * m[2]).to(x.dtype)
        x = x + self.cross_attn(self.norm3(x), ctx, attn)
        h = (self._norm(x).float() * (1 + m[4]) + m[3]).to(x.dtype)
        y = self.fc2(F.gelu(self.fc1(h), approximate="tanh"))
        return (x.float() + y.float() * m[5]).to(x.dtype)


class DiTModel(nn.Module):
    def __init__(self, s: DiTShape = WAN_DIT, dtype: torch.dtype = torch.bfloat16) -> None:
        super().__init__()
        self.shape = s
        self.blocks = nn.ModuleList(DiTBlock(s, dtype) for _ in range(s.n_blocks))
        self.attn = None  # attention override (callable on [b, h, s, d] tensors)

    def forward(self, x: torch.Tensor, e: torch.Tensor, ctx: torch.Tensor) -> torch.Tensor:
        for blk in self.blocks:
            x = blk(x, e, ctx, self.attn)
        return x


def build_dit(shape: DiTShape = WAN_DIT, seed: int = 0, init_device: str = "cpu") -> DiTModel:
    with torch.device("meta"):
        model = DiTModel(shape)
    model = model.to_empty(device="cpu")
    return init_normal_(model, seed, 0.02, init_device)


def dit_inputs(shape: DiTShape, tokens: int, text: int, seed: int = 0, device: str = "cpu"):
    """Latent tokens, timestep modulation and text context, all ~N(0, 1) in bf16."""
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(1, tokens, shape.dim, generator=gen, device=device).to(torch.bfloat16)
    e = torch.randn(1, 6, shape.dim, generator=gen, device=device).to(torch.bfloat16)
    ctx = torch.randn(1, text, shape.dim, generator=gen, device=device).to(torch.bfloat16)
    return x, e, ctx


# ---- scatter microbenchmark tensor set ------------------------------------------


def scatter_sizes(n: int = 2000, lo: int = 4096, hi: int = 64 << 20, seed: int = 1) -> list[int]:
    """Byte sizes log-uniform in [lo, hi], rounded down to whole bf16 elements."""
    rng = np.random.default_rng(seed)
    u = rng.uniform(math.log(lo), math.log(hi), size=n)
    return [int(math.exp(x)) // 2 * 2 for x in u]


def scatter_shape(nbytes: int, index: int) -> tuple[int, ...]:
    """1-D for even indices, 2-D [rows, cols] (cols = largest power of two <= 1024 dividing numel) for odd."""
    numel = nbytes // 2
    if index % 2 == 0 or numel == 0:
        return (numel,)
    cols = 1
    while cols < 1024 and numel % (cols * 2) == 0:
        cols *= 2
    return (numel // cols, cols)
