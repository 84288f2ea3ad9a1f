"""A model built from a saved profile and a safetensors checkpoint streams bitwise like the resident model.

The profile is made by offloading a model through discovery and profiling;
the checkpoint is that model's ``state_dict`` written by the ``safetensors``
package. ``load_model_from_profile`` then constructs the class on the meta
device, maps the checkpoint and packs the streamed weights straight from the
mapping; every forward must equal the resident forward bit for bit. The
DeepSeek-style ``weight.scale`` attribute must follow the streamed weight
(tests/unit/test_tensor_inner_fields.py:68-101 in the reference).
"""

from __future__ import annotations

import copy
import dataclasses

import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import save_file

from flextensor_amd import workloads as W
from flextensor_amd.config import OffloadConfig
from flextensor_amd.lazy_model_init import load_model_from_profile
from flextensor_amd.manager import OffloadManager, OffloadPhase
from tests.test_lazy_model_init import LinearWithScale

pytestmark = pytest.mark.gpu

SHAPE = W.LlamaShape(n_layers=6, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=704, vocab=512, max_seq=64)


def _cfg(budget: int, **kw) -> OffloadConfig:
    base = dict(include_patterns=["layers.*"], num_blocks=2, min_blocks=2, discovery_iters=1, profiling_iters=1,
                max_gpu_mem_bytes=budget)
    base.update(kw)
    return OffloadConfig(**base)


def _checkpoint(model: torch.nn.Module, path) -> str:
    save_file({k: v.detach().contiguous() for k, v in model.state_dict().items()}, str(path))
    return str(path)


def _logits(model: W.LlamaModel, tokens: torch.Tensor, gpu) -> torch.Tensor:
    model.init_cache(tokens.shape[0], SHAPE.max_seq, gpu)
    with torch.no_grad():
        return model(tokens)


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
@pytest.mark.parametrize("mode", ["allocation_block_transfer", "raw_block_transfer"])
def test_checkpoint_model_streams_bitwise(gpu, tmp_path, fp8, mode):
    shape = dataclasses.replace(SHAPE, fp8=fp8)
    model = W.build_llama(shape, seed=11)
    ckpt = _checkpoint(model, tmp_path / "model.safetensors")
    tokens = W.prompt_tokens(2, 8, shape.vocab, seed=11).to(gpu)
    want = _logits(copy.deepcopy(model).to(gpu), tokens, gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    rest = sum(p.numel() * p.element_size() for n, p in model.named_parameters() if not n.startswith("layers."))
    cfg = _cfg(rest + 4 * layer, transfer_mode=mode)
    src = OffloadManager(name=f"lazy-src-{mode}-{fp8}")
    src.offload(model, cfg)
    for _ in range(3):
        assert torch.equal(_logits(model, tokens, gpu), want)
    assert src.phase == OffloadPhase.INFERENCE and src.plan.streamed
    src.save_profile(str(tmp_path))
    streamed = list(src.plan.streamed)
    src.release()
    del model

    dst = OffloadManager(name=f"lazy-dst-{mode}-{fp8}")
    twin = load_model_from_profile(dst, str(tmp_path), W.LlamaModel, (shape,), safetensor_path=ckpt, config=cfg,
                                   strict=True)
    assert dst.phase == OffloadPhase.INFERENCE and dst.plan.streamed == streamed
    assert twin.rope_cos.is_cuda and not twin.training
    assert all(p.is_cuda for p in twin.parameters())
    for _ in range(3):
        assert torch.equal(_logits(twin, tokens, gpu), want)
    dst.release()


class InnerStack(torch.nn.Module):
    """Four layers of the DeepSeek-style ``weight.scale = scale`` pattern."""

    def __init__(self, n: int = 4, width: int = 64) -> None:
        super().__init__()
        self.layers = torch.nn.ModuleList(LinearWithScale(width, width) for _ in range(n))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = torch.relu(layer(x))
        return x


def test_inner_fields_follow_the_streamed_weight(gpu, tmp_path):
    torch.manual_seed(5)
    model = InnerStack()
    ckpt = _checkpoint(model, tmp_path / "inner.safetensors")
    x = torch.randn(4, 64, device=gpu)
    # The resident forward from the weights themselves: deepcopy of a Parameter drops its attributes.
    sd = {k: v.to(gpu) for k, v in model.state_dict().items()}
    want = x
    with torch.no_grad():
        for i in range(4):
            want = torch.relu(F.linear(want, sd[f"layers.{i}.weight"]) * sd[f"layers.{i}.scale"].mean())
    unit = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = _cfg(2 * unit + unit // 2)
    src = OffloadManager(name="inner-src")
    src.offload(model, cfg)
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(model(x), want)  # forward asserts weight.scale sits beside weight
    assert src.plan.streamed and model.layers[0].weight.scale is model.layers[0].scale
    src.save_profile(str(tmp_path))
    src.release()

    dst = OffloadManager(name="inner-dst")
    twin = load_model_from_profile(dst, str(tmp_path), InnerStack, safetensor_path=ckpt, config=cfg)
    assert dst.plan.streamed
    for layer in twin.layers:
        assert layer.weight.scale is layer.scale and layer.scale.is_cuda
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(twin(x), want)
    dst.release()


def test_missing_parameters_are_named_before_streaming(gpu, tmp_path):
    model = W.build_llama(SHAPE, seed=3)
    tokens = W.prompt_tokens(1, 4, SHAPE.vocab, seed=3).to(gpu)
    layer = sum(p.numel() * p.element_size() for p in model.layers[0].parameters())
    cfg = _cfg(10 * layer)
    src = OffloadManager(name="lazy-missing-src")
    src.offload(model, cfg)
    for _ in range(3):
        _logits(model, tokens, gpu)
    src.save_profile(str(tmp_path))
    src.release()
    sd = {k: v for k, v in model.state_dict().items() if k != "lm_head.weight"}
    ckpt = _checkpoint_dict(sd, tmp_path / "partial.safetensors")
    dst = OffloadManager(name="lazy-missing-dst")
    with pytest.raises(KeyError, match="lm_head.weight"):
        load_model_from_profile(dst, str(tmp_path), W.LlamaModel, (SHAPE,), safetensor_path=ckpt, config=cfg,
                                strict=True)
    with pytest.raises(RuntimeError, match="lm_head.weight"):
        load_model_from_profile(dst, str(tmp_path), W.LlamaModel, (SHAPE,), safetensor_path=ckpt, config=cfg)
    assert dst.model is None


def _checkpoint_dict(sd: dict[str, torch.Tensor], path) -> str:
    save_file({k: v.detach().contiguous() for k, v in sd.items()}, str(path))
    return str(path)
