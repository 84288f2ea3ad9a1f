"""Manual offload blocks on the GPU (offload_manager.py:2251-2298, 2990-2998 in the reference).

A model offloaded with no module units (``include_patterns=[]``) marks its
offload units with ``offload_block(label)``. Discovery finds each block's
parameters from the torch calls made inside it; parameters used outside
blocks, or by two blocks, stay on the GPU. Every pass must equal the
resident forward bit for bit, through discovery, profiling and streaming,
and a saved profile must restore the blocks. The direct-call pattern is the
reference's tests/unit/test_tensor_inner_fields.py:104-137.
"""

from __future__ import annotations

import contextlib

import pytest
import torch
from torch import nn

from flextensor_amd.config import OffloadConfig
from flextensor_amd.manager import (
    OffloadManager,
    OffloadPhase,
    get_offload_manager,
    offload_block,
    offload_from_profile,
    release,
)
from tests.test_gpu_lazy_init import InnerStack

pytestmark = pytest.mark.gpu


class BlockModel(nn.Module):
    """Embedding outside the blocks, one block per layer, one parameter shared by two blocks."""

    def __init__(self, n: int = 6, width: int = 128, vocab: int = 64) -> None:
        super().__init__()
        self.embed = nn.Embedding(vocab, width)
        self.layers = nn.ModuleList(nn.Linear(width, width) for _ in range(n))
        self.shared = nn.Parameter(torch.randn(width) * 0.01)
        self.manager: str | None = None  # the manager whose blocks wrap the layers

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        x = self.embed(tokens)
        for i, layer in enumerate(self.layers):
            block = offload_block(f"blk{i}", name=self.manager) if self.manager else contextlib.nullcontext()
            with block:
                x = torch.relu(layer(x))
                if i in (1, 4):
                    x = x + self.shared
        return x


def _bytes(module: nn.Module) -> int:
    return sum(p.numel() * p.element_size() for p in module.parameters())


def _cfg(budget: int, **kw) -> OffloadConfig:
    base = dict(include_patterns=[], num_blocks=2, min_blocks=2, discovery_iters=1, profiling_iters=1,
                max_gpu_mem_bytes=budget)
    base.update(kw)
    return OffloadConfig(**base)


def test_direct_calls_with_update_state(gpu):
    torch.manual_seed(1)
    model = InnerStack(6)
    torch.manual_seed(1)
    ref = InnerStack(6).to(gpu)
    x = torch.randn(4, 64, device=gpu)
    with torch.no_grad():
        want = ref(x)
    om = OffloadManager(name="manual-direct")
    om.offload(model, _cfg(3 * _bytes(model.layers[0])))
    assert all(p.device.type == "cpu" for p in model.parameters())
    phases = []
    with torch.no_grad():
        for _ in range(4):
            phases.append(om.phase)
            h = x
            for i, layer in enumerate(model.layers):
                with om.offload_block(f"blk{i}"):
                    h = torch.relu(layer(h))  # the layer asserts weight.scale sits beside weight
            om.update_state()  # no root forward ran: the caller ends the pass
            assert torch.equal(h, want)
    assert phases == [OffloadPhase.DISCOVERY, OffloadPhase.PROFILING, OffloadPhase.INFERENCE,
                      OffloadPhase.INFERENCE]
    assert [u.label for u in om.units] == [f"blk{i}" for i in range(6)]
    assert all(u.module is None for u in om.units) and om.plan.streamed
    for u, layer in zip(om.units, model.layers):
        assert sorted(u.names) == [f"layers.{u.label[3:]}.scale", f"layers.{u.label[3:]}.weight"]  # first-use order
        assert layer.weight.scale is layer.scale
    om.release()
    assert all(p.device.type == "cpu" for p in model.parameters())


def test_blocks_in_the_forward_and_a_saved_profile(gpu, tmp_path):
    torch.manual_seed(2)
    model = BlockModel()
    torch.manual_seed(2)
    ref = BlockModel().to(gpu)
    tokens = torch.randint(0, 64, (2, 8), device=gpu)
    with torch.no_grad():
        want = ref(tokens)
    layer = _bytes(model.layers[0])
    cfg = _cfg(_bytes(model.embed) + model.shared.numel() * 4 + 3 * layer)
    om = get_offload_manager("manual-fwd")  # the module-level offload_block looks managers up by name
    model.manager = om.name
    om.offload(model, cfg)
    with torch.no_grad():
        for _ in range(4):
            assert torch.equal(model(tokens), want)
    assert om.phase == OffloadPhase.INFERENCE and om.plan.streamed
    assert model.embed.weight.is_cuda and model.shared.is_cuda  # used outside blocks / by two blocks
    owned = {n for u in om.units for n in u.names}
    assert "embed.weight" not in owned and "shared" not in owned
    assert owned == {f"layers.{i}.{w}" for i in range(6) for w in ("weight", "bias")}
    om.save_profile(str(tmp_path))
    streamed = list(om.plan.streamed)
    om.release()

    torch.manual_seed(2)
    twin = BlockModel()
    twin.manager = "manual-fwd-dst"
    offload_from_profile(twin, str(tmp_path), cfg, name="manual-fwd-dst")
    dst = get_offload_manager("manual-fwd-dst")
    assert dst.phase == OffloadPhase.INFERENCE and all(u.module is None for u in dst.units)
    assert dst.plan.streamed == streamed
    with torch.no_grad():
        for _ in range(3):
            assert torch.equal(twin(tokens), want)
    release("manual-fwd-dst")


def test_block_errors(gpu):
    with pytest.raises(RuntimeError, match="Call offload"):
        OffloadManager(name="manual-none").offload_block("x")

    torch.manual_seed(3)
    model = InnerStack(4)
    om = OffloadManager(name="manual-nest")
    om.offload(model, _cfg(3 * _bytes(model.layers[0])))
    x = torch.randn(2, 64, device=gpu)
    with torch.no_grad():
        with om.offload_block("blk0"):
            h = model.layers[0](x)
            with pytest.raises(RuntimeError, match="do not nest"):
                with om.offload_block("blk1"):
                    pass
        assert model.layers[0].weight.device.type == "cpu"  # back on the host after the block
        for i in range(1, 4):
            with om.offload_block(f"blk{i}"):
                h = model.layers[i](h)
        om.update_state()
        with pytest.raises(RuntimeError, match="not seen during discovery"):
            with om.offload_block("never"):
                pass
    om.release()

    patched = InnerStack(4)
    om2 = OffloadManager(name="manual-mixed")
    om2.offload(patched, _cfg(3 * _bytes(patched.layers[0]), include_patterns=["layers.*"]))
    with pytest.raises(RuntimeError, match="no module units"):
        with om2.offload_block("blk0"):
            pass
    with torch.no_grad(), om2.offload_block("layers.0"):  # a patched module unit: the block does nothing
        patched.layers[0](x)
    om2.release()


def test_blocks_kept_encoded_in_hbm(gpu):
    """Manual blocks as units kept exponent-coded in HBM (encode_resident_blocks): bf16 layers of 2 MiB
    under a budget of 11 of 12 layers. Raw, 3 blocks would stream; with the option fewer do, the rest
    decode from HBM as their block opens, and every pass equals the resident forward bit for bit."""
    torch.manual_seed(4)
    model = BlockModel(n=12, width=1024).to(torch.bfloat16)
    torch.manual_seed(4)
    ref = BlockModel(n=12, width=1024).to(torch.bfloat16).to(gpu)
    tokens = torch.randint(0, 64, (2, 8), device=gpu)
    with torch.no_grad():
        want = ref(tokens)
    budget = _bytes(model.embed) + model.shared.numel() * 2 + 11 * _bytes(model.layers[0])
    om = get_offload_manager("manual-hbm")
    model.manager = om.name
    om.offload(model, _cfg(budget, encode_resident_blocks=True, link_benchmark=False))
    try:
        with torch.no_grad():
            for _ in range(4):
                assert torch.equal(model(tokens), want)
        assert om.phase == OffloadPhase.INFERENCE and om.plan.encoded_resident
        assert 0 < len(om.plan.streamed) < 3
        assert all(u.module is None for u in om.units)
        assert om.get_gpu_memory_usage().total_bytes <= budget
    finally:
        om.release()
    for p, q in zip(model.parameters(), ref.parameters()):
        assert p.device.type == "cpu" and torch.equal(p, q.cpu())
