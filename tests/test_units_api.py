"""``offload_units`` / ``resident_units`` on the CPU (tests/unit/test_offload_units_api.py:61-332 in the reference).

The manager is bound to a model and its selected units without a device:
the listings only walk the module tree.
"""

from __future__ import annotations

import pytest
from torch import nn

import flextensor_amd.manager as M


class _Block(nn.Module):
    def __init__(self, d: int = 4) -> None:
        super().__init__()
        self.lin = nn.Linear(d, d)

    def forward(self, x):
        return self.lin(x)


class _Stack(nn.Module):
    def __init__(self, n: int = 3) -> None:
        super().__init__()
        self.embed = nn.Linear(4, 4)
        self.blocks = nn.ModuleList(_Block() for _ in range(n))
        self.head = nn.Linear(4, 4)

    def forward(self, x):
        x = self.embed(x)
        for b in self.blocks:
            x = b(x)
        return self.head(x)


@pytest.fixture
def mgr():
    m = M.OffloadManager("units-api")
    yield m
    m.model, m.units = None, []


def _bind(mgr: M.OffloadManager, model: nn.Module, patterns: list[str]) -> nn.Module:
    mgr.model = model
    mgr.units = [M._Unit(label, model.get_submodule(label)) for label in M.select_offload_units(model, patterns, [])]
    return model


def test_empty_without_model_or_units(mgr):
    assert mgr.offload_units() == () and mgr.resident_units() == ()
    model = _bind(mgr, _Stack(), [])
    assert mgr.offload_units() == ()
    assert mgr.resident_units() == (("embed", model.embed), ("blocks.0", model.blocks[0]),
                                    ("blocks.1", model.blocks[1]), ("blocks.2", model.blocks[2]),
                                    ("head", model.head))


def test_units_in_order_with_live_modules(mgr):
    model = _bind(mgr, _Stack(), ["blocks.*"])
    assert mgr.offload_units() == tuple((f"blocks.{i}", model.blocks[i]) for i in range(3))
    replacement = nn.Identity()
    model.blocks[1] = replacement  # a compiled wrapper put in place of the unit
    assert mgr.offload_units()[1] == ("blocks.1", replacement)
    assert mgr.resident_units() == (("embed", model.embed), ("head", model.head))


def test_resident_units_are_outermost_islands(mgr):
    model = _bind(mgr, _Stack(), ["blocks.0", "blocks.2"])
    assert mgr.resident_units() == (("embed", model.embed), ("blocks.1", model.blocks[1]), ("head", model.head))
    _bind(mgr, _Stack(n=1), ["blocks.0"])
    assert [n for n, _ in mgr.resident_units()] == ["embed", "head"]


def test_a_shared_unit_hides_its_second_parent():
    class Inner(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.lin = nn.Linear(2, 2)

    class Outer(nn.Module):
        def __init__(self, inner: nn.Module) -> None:
            super().__init__()
            self.inner = inner
            self.gate = nn.Linear(2, 2)

        def forward(self, x):
            return self.inner(x) + self.gate(x)

    class Root(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.inner = Inner()
            self.outer = Outer(self.inner)

    m = M.OffloadManager("units-shared")
    model = _bind(m, Root(), ["inner"])
    assert m.offload_units() == (("inner", model.inner),)
    assert m.resident_units() == (("outer.gate", model.outer.gate),)


def test_containers_are_descended_but_sequential_is_an_island(mgr):
    class Root(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.blocks = nn.ModuleList([nn.Linear(4, 4), nn.Linear(4, 4)])
            self.tower = nn.Sequential(nn.Linear(4, 4), nn.Linear(4, 4))
            self.heads = nn.ModuleDict({"a": nn.Linear(4, 4), "b": nn.Linear(4, 4)})

    model = Root()
    mgr.model = model
    assert mgr.resident_units() == (("blocks.0", model.blocks[0]), ("blocks.1", model.blocks[1]),
                                    ("tower", model.tower), ("heads.a", model.heads["a"]),
                                    ("heads.b", model.heads["b"]))


def test_shared_module_listed_once(mgr):
    shared = nn.Linear(4, 4)
    model = nn.Module()
    model.add_module("a", shared)
    model.add_module("b", shared)
    mgr.model = model
    assert mgr.resident_units() == (("a", shared),)


def test_module_level_wrappers_match_the_manager():
    name = "units-pkg"
    try:
        om = M.get_offload_manager(name)
        model = _bind(om, _Stack(), ["blocks.1"])
        assert M.offload_units(name) == om.offload_units() == (("blocks.1", model.blocks[1]),)
        assert [n for n, _ in M.resident_units(name)] == ["embed", "blocks.0", "blocks.2", "head"]
    finally:
        M._MANAGERS.pop(name, None)
