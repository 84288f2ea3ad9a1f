"""Shared resident-tensor store materialized onto the GPU by stream-and-scatter.

The follower's device tensors must hold exactly the creator's bytes, with
the stored shapes and strides, whether the payloads cross in one chunk or in
many (staging buffers reused).
"""

from __future__ import annotations

import os

import pytest
import torch
from torch import nn

from flextensor_amd import workloads as W
from flextensor_amd.shm import SharedTensorStore, store_segment_name

pytestmark = pytest.mark.gpu


class _Model(nn.Module):
    def __init__(self, device: str = "cpu") -> None:
        super().__init__()
        self.body = W.build_mlp_stack(4, 256, 704, seed=11) if device == "cpu" else \
            W.build_mlp_stack(4, 256, 704, seed=11).to("meta")
        self.head = nn.Parameter(torch.arange(35, dtype=torch.float32, device=device).reshape(5, 7).t())  # Fortran
        self.register_buffer("steps", torch.tensor([1, 2, 3], dtype=torch.int64, device=device))
        self.register_buffer("odd", torch.arange(7, dtype=torch.uint8, device=device), persistent=False)


@pytest.fixture
def ns(request):
    name = f"ftxg_{os.getpid()}_{request.node.name}".replace("[", "_").replace("]", "").replace("-", "_")
    yield name
    try:
        os.unlink(os.path.join("/dev/shm", store_segment_name(name)))
    except FileNotFoundError:
        pass


@pytest.mark.parametrize("chunk_bytes", [None, 1 << 20, 64 << 10])
def test_store_materializes_on_gpu_bit_exact(gpu, ns, chunk_bytes):
    src = _Model()
    names = [n for n, _ in src.named_parameters()]
    creator = SharedTensorStore.create_from_model(ns, src, parameter_names=names)
    follower = SharedTensorStore.attach(ns)
    target = _Model(device="meta")
    try:
        follower.materialize_into(target, device=gpu, chunk_bytes=chunk_bytes)
    finally:
        follower.close()
        creator.close()
    want = dict(src.named_parameters())
    want.update(src.named_buffers())
    got = dict(target.named_parameters())
    got.update(target.named_buffers())
    assert set(got) == set(want)
    for name, t in want.items():
        g = got[name]
        assert g.device.type == "cuda" and g.dtype == t.dtype and g.shape == t.shape and g.stride() == t.stride()
        width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
        assert torch.equal(g.detach().cpu().view(width), t.detach().view(width)), name
    assert "odd" in target._non_persistent_buffers_set
    x = W.mlp_input(4, 256, seed=11)
    with torch.no_grad():
        assert torch.equal(target.body.to(gpu)(x.to(gpu)).cpu(), src.body.to(gpu)(x.to(gpu)).cpu())
