"""HostPinner against the reference's host-pinning cases (tests/unit/test_host_pinning.py).

Restated for this build's pinner, which allocates ``torch``-mode blocks in a
page-locked arena and registers ``host_register``-mode storages through
``ftx_arena_register`` (mocked here: the CPU suite has no GPU). Cases:
tensors that are not pinned (non-CPU, meta, empty, already pinned) come back
unchanged (:820-853); in-place pins register each storage once, views
included (:96-122), and are released by ``release_all`` (:855-870);
``is_pinned`` follows torch's flag in ``torch`` mode and the registry in
``host_register`` mode, and reads a tensor without a storage pointer as not
pinned (:872-908); an unknown mode is refused (:1096-1108).
"""

from __future__ import annotations

import logging
from unittest.mock import MagicMock

import pytest
import torch

from flextensor_amd import _native as nat
from flextensor_amd.allocation_block import HostPinner


@pytest.fixture
def pins(monkeypatch):
    calls = {"register": [], "unregister": []}
    monkeypatch.setattr(nat, "arena_register", lambda ptr, n: calls["register"].append((ptr, n)))
    monkeypatch.setattr(nat, "arena_unregister", lambda ptr: calls["unregister"].append(ptr))
    return calls


def _fake(device: str = "cpu", *, pinned: bool = False, numel: int = 16) -> MagicMock:
    t = MagicMock(spec=torch.Tensor)
    t.device = torch.device(device)
    t.is_meta = False
    t.numel.return_value = numel
    t.is_pinned.return_value = pinned
    return t


@pytest.mark.parametrize("mode", ["torch", "host_register"])
def test_tensors_that_are_not_pinned_come_back_unchanged(pins, mode):
    pinner = HostPinner(mode)
    meta = torch.empty(8, dtype=torch.uint8, device="meta")
    empty = torch.empty(0, dtype=torch.uint8)
    on_gpu = _fake("cuda:0")
    pinned = _fake(pinned=True)
    for t in (meta, empty, on_gpu, pinned):
        assert pinner.pin(t) is t
    on_gpu.pin_memory.assert_not_called()
    pinned.pin_memory.assert_not_called()
    assert pins["register"] == []


def test_disabled_pinner_returns_every_tensor(pins):
    pinner = HostPinner("host_register", enabled=False)
    t = torch.arange(32, dtype=torch.uint8)
    assert pinner.pin(t) is t and pins["register"] == []
    block = pinner.new_block(64)  # pageable: a plain host tensor, nothing registered
    assert block.numel() == 64 and block.dtype == torch.uint8 and pins["register"] == []


def test_torch_mode_pin_returns_a_copy_in_a_pinner_block(monkeypatch):
    pinner = HostPinner("torch")
    blocks = []

    def new_block(nbytes):
        blocks.append(torch.zeros(nbytes, dtype=torch.uint8))
        return blocks[-1]

    monkeypatch.setattr(pinner, "new_block", new_block)
    t = torch.randn(3, 5, dtype=torch.float32)
    out = pinner.pin(t)
    assert out is not t and torch.equal(out, t) and out.dtype == t.dtype
    assert len(blocks) == 1 and out.untyped_storage().data_ptr() == blocks[0].data_ptr()


def test_torch_mode_pin_failure_raises(monkeypatch):
    pinner = HostPinner("torch")

    def fail(nbytes):
        raise RuntimeError("hipHostMalloc failed: out of memory")

    monkeypatch.setattr(pinner, "new_block", fail)
    with pytest.raises(RuntimeError, match="out of memory"):
        pinner.pin(torch.ones(4))


def test_host_register_pins_each_storage_once_views_included(pins):
    pinner = HostPinner("host_register")
    base = torch.zeros(256, dtype=torch.uint8)
    a, b = base[:128], base[128:]
    assert pinner.pin(a) is a and pinner.pin(b) is b and pinner.pin(base) is base
    storage = base.untyped_storage()
    assert pins["register"] == [(storage.data_ptr(), storage.nbytes())]
    assert pinner.pinned_bytes == 256


def test_host_register_pin_of_a_strided_view_registers_its_storage(pins):
    pinner = HostPinner("host_register")
    base = torch.zeros(8, 8, dtype=torch.float32)
    col = base[:, 3]  # not contiguous, offset into the storage
    assert pinner.pin(col) is col
    assert pins["register"] == [(base.untyped_storage().data_ptr(), base.untyped_storage().nbytes())]


def test_release_all_unregisters_every_pin_and_is_a_noop_in_torch_mode(pins):
    torch_pinner = HostPinner("torch")
    torch_pinner.release_all()
    assert pins["unregister"] == []
    pinner = HostPinner("host_register")
    ts = [torch.zeros(n, dtype=torch.uint8) for n in (16, 32)]
    for t in ts:
        pinner.pin(t)
    pinner.release_all()
    assert sorted(pins["unregister"]) == sorted(t.untyped_storage().data_ptr() for t in ts)
    assert pinner.pinned_bytes == 0


def test_is_pinned_follows_torch_in_torch_mode():
    pinner = HostPinner("torch")
    assert pinner.is_pinned(_fake(pinned=False)) is False
    assert pinner.is_pinned(_fake(pinned=True)) is True


def test_is_pinned_consults_the_registry_in_host_register_mode(pins):
    pinner = HostPinner("host_register")
    registered, other = torch.zeros(16, dtype=torch.uint8), torch.zeros(16, dtype=torch.uint8)
    pinner.pin(registered)
    assert pinner.is_pinned(registered) is True
    assert pinner.is_pinned(registered[4:]) is True  # a view of the registered storage
    assert pinner.is_pinned(other) is False
    assert not registered.is_pinned()  # registration does not set torch's flag


def test_is_pinned_reads_a_tensor_without_storage_pointer_as_not_pinned(caplog):
    pinner = HostPinner("host_register")
    broken = _fake()
    broken.untyped_storage.side_effect = RuntimeError("no storage")
    with caplog.at_level(logging.DEBUG, logger="flextensor_amd.allocation_block"):
        assert pinner.is_pinned(broken) is False
    assert "not pinned" in caplog.text


def test_unknown_mode_is_refused():
    with pytest.raises(ValueError, match="pinned_memory_mode"):
        HostPinner("cuda_register")
