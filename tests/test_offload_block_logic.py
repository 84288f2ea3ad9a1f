"""Manual offload-block discovery on the CPU: which parameters each block owns.

The manager runs with the host as its device (no uploads happen), so the
bookkeeping of discovery is checked on its own: a parameter used inside one
block belongs to that block, one used outside blocks or by a second block is
placed for good, and the manager's own moves of a block's parameters at the
block's exit are not taken for uses.
"""

from __future__ import annotations

from unittest import mock

import pytest
import torch
from torch import nn

import flextensor_amd.manager as M
from flextensor_amd.config import OffloadConfig


class Blocks(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.embed = nn.Embedding(10, 8)
        self.layers = nn.ModuleList(nn.Linear(8, 8) for _ in range(3))
        self.shared = nn.Parameter(torch.ones(8))
        self.unused = nn.Parameter(torch.zeros(2))
        self.manager = ""

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        x = self.embed(tokens)
        for i, layer in enumerate(self.layers):
            with M.offload_block(f"blk{i}", name=self.manager):
                x = layer(x)
                if i != 1:
                    x = x + self.shared
        return x


@pytest.fixture
def host_manager():
    with mock.patch.object(M.nat, "load", lambda: None), \
            mock.patch.object(M.torch.cuda, "set_device", lambda d: None), \
            mock.patch.object(M.custom_ops, "register_manager", lambda *a: None), \
            mock.patch.object(M.OffloadManager, "_upload_into", lambda self, ts: 0):
        mgr = M.get_offload_manager("host-blocks")
        yield mgr
        mgr._reset_manual()
        mgr.model = None
        mgr.units, mgr._patched, mgr._hooks, mgr.order = [], [], [], []
        mgr.phase = M.OffloadPhase.NOT_INITIALIZED
        M._MANAGERS.pop("host-blocks", None)


def test_discovery_assigns_parameters_to_blocks(host_manager):
    model = Blocks()
    model.manager = "host-blocks"
    mgr = host_manager
    mgr.offload(model, OffloadConfig(include_patterns=[], discovery_iters=1, profiling_iters=1))
    mgr.device = torch.device("cpu")
    assert mgr._manual and len(mgr._pending) == sum(1 for _ in model.parameters())
    with torch.no_grad():
        model(torch.tensor([[1, 2, 3]]))
    assert mgr.phase == M.OffloadPhase.PROFILING  # the root forward's hook ended the discovery pass
    assert [u.label for u in mgr.units] == ["blk0", "blk1", "blk2"]
    assert [u.names for u in mgr.units] == [[f"layers.{i}.weight", f"layers.{i}.bias"] for i in range(3)]
    assert all(u.module is None for u in mgr.units)
    assert not mgr._pending  # embed (outside), shared (two blocks) and unused were placed for good


def test_a_block_exit_is_not_a_use(host_manager):
    model = Blocks()
    model.manager = "host-blocks"
    mgr = host_manager
    mgr.offload(model, OffloadConfig(include_patterns=[], discovery_iters=1, profiling_iters=1))
    mgr.device = torch.device("cpu")
    with torch.no_grad(), M.offload_block("blk0", name="host-blocks"):
        model.layers[0](torch.ones(1, 8))
    w = model.layers[0].weight
    assert mgr._block_owner[id(w)] == "blk0" and id(w) in mgr._pending
    assert mgr._mode is None and mgr._mode_depth == 0
    with pytest.raises(NotImplementedError, match="twice"):
        with M.offload_block("blk0", name="host-blocks"):
            pass
