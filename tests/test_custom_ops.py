"""Compute-boundary custom ops under torch.compile (CPU, no code generation).

The patched unit forwards of a manager call ``flextensor::pre_compute`` /
``post_compute`` while compiling; the compiled model must call enter/exit in
the eager order, once per unit per forward, and compute the same values.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from flextensor_amd import custom_ops
from flextensor_amd import workloads as W
from flextensor_amd.manager import OffloadManager, OffloadPhase, _Unit, select_offload_units


class _RecordingManager(OffloadManager):
    """A manager whose enter/exit only record (no device work)."""

    def __init__(self) -> None:
        super().__init__(name=f"rec-{id(self)}")
        self.calls: list[tuple[str, str]] = []
        self.phase = OffloadPhase.INFERENCE

    def _enter(self, label: str) -> None:
        self.calls.append(("enter", label))

    def _exit(self, label: str) -> None:
        self.calls.append(("exit", label))


def _patched(model: nn.Module) -> _RecordingManager:
    mgr = _RecordingManager()
    custom_ops.register_manager(id(mgr), mgr)
    for label in select_offload_units(model, ["layers.*"], []):
        mgr._patch(_Unit(label, model.get_submodule(label)))
    return mgr


def _expected(n: int) -> list[tuple[str, str]]:
    return [c for i in range(n) for c in (("enter", f"layers.{i}"), ("exit", f"layers.{i}"))]


@pytest.mark.parametrize("backend", ["eager", "aot_eager"])
def test_compiled_forward_keeps_enter_exit_order(backend):
    torch._dynamo.reset()
    model = W.build_mlp_stack(4, 32, 64, seed=1)
    x = W.mlp_input(3, 32, seed=1)
    with torch.no_grad():
        want = model(x)
    mgr = _patched(model)
    mgr.calls.clear()
    compiled = torch.compile(model, backend=backend, fullgraph=True)
    with torch.no_grad():
        for k in range(3):
            got = compiled(x)
            assert torch.equal(got, want)
            assert mgr.calls == _expected(4) * (k + 1)
    custom_ops.unregister_manager(id(mgr))


def test_eager_forward_calls_manager_directly():
    model = W.build_mlp_stack(3, 16, 32, seed=2)
    mgr = _patched(model)
    with torch.no_grad():
        model(W.mlp_input(2, 16, seed=2))
    assert mgr.calls == _expected(3)
    custom_ops.unregister_manager(id(mgr))


def test_released_manager_raises_and_unknown_id_is_a_no_op():
    x = torch.zeros(2)
    torch.ops.flextensor.pre_compute(x, "layers.0", 123456789)  # never registered: nothing to do
    mgr = _RecordingManager()
    custom_ops.register_manager(id(mgr), mgr)
    torch.ops.flextensor.pre_compute(x, "layers.0", id(mgr))
    assert mgr.calls == [("enter", "layers.0")]
    custom_ops.unregister_manager(id(mgr))
    with pytest.raises(RuntimeError, match="released"):
        torch.ops.flextensor.post_compute(x, "layers.0", id(mgr))


def test_op_schema_matches_the_reference():
    # custom_ops.py:313-328 of the reference
    schemas = {str(torch.ops.flextensor.pre_compute.default._schema),
               str(torch.ops.flextensor.post_compute.default._schema)}
    assert schemas == {
        "flextensor::pre_compute(Tensor(a!) input_tensor, str offload_unit_name, int manager_id) -> ()",
        "flextensor::post_compute(Tensor(a!) output_tensor, str offload_unit_name, int manager_id) -> ()",
    }


def test_compiling_before_inference_is_refused():
    torch._dynamo.reset()
    model = W.build_mlp_stack(2, 16, 32, seed=3)
    mgr = _patched(model)
    mgr.phase = OffloadPhase.PROFILING
    with pytest.raises(Exception, match="profiling"):
        torch.compile(model, backend="eager", fullgraph=True)(W.mlp_input(2, 16, seed=3))
    custom_ops.unregister_manager(id(mgr))


class _Recorder:
    def __init__(self) -> None:
        self.calls: list[tuple[str, str]] = []

    def _enter(self, label: str) -> None:
        self.calls.append(("enter", label))

    def _exit(self, label: str) -> None:
        self.calls.append(("exit", label))


def test_opcheck_accepts_the_compute_boundary_ops():
    """tests/unit/test_custom_ops.py:214-230: schema, autograd, fake and AOT dispatch checks."""
    for op in (torch.ops.flextensor.pre_compute.default, torch.ops.flextensor.post_compute.default):
        result = torch.library.opcheck(op, (torch.zeros(3), "unit", 987654321))
        assert set(result.values()) == {"SUCCESS"}, result


def test_fake_tensors_never_reach_the_manager():
    """tests/unit/test_custom_ops.py:54-96: tracing with fake tensors must not enter or exit units."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from flextensor_amd import custom_ops as C

    rec = _Recorder()
    C.register_manager(4242, rec)
    try:
        with FakeTensorMode() as mode:
            fake = mode.from_tensor(torch.zeros(2))
            torch.ops.flextensor.pre_compute(fake, "u", 4242)
            torch.ops.flextensor.post_compute(fake, "u", 4242)
        assert rec.calls == []
        carrier = torch.arange(4.0)
        torch.ops.flextensor.pre_compute(carrier, "u", 4242)
        torch.ops.flextensor.post_compute(carrier, "u", 4242)
        assert rec.calls == [("enter", "u"), ("exit", "u")]
        assert torch.equal(carrier, torch.arange(4.0))  # declared mutated, never written
    finally:
        C.unregister_manager(4242)


def test_managers_dispatch_independently():
    """tests/unit/test_custom_ops.py:151-200: each manager id reaches its own manager; releasing one leaves
    the other working."""
    from flextensor_amd import custom_ops as C

    a, b = _Recorder(), _Recorder()
    C.register_manager(1001, a)
    C.register_manager(1002, b)
    try:
        torch.ops.flextensor.pre_compute(torch.zeros(1), "x", 1001)
        torch.ops.flextensor.pre_compute(torch.zeros(1), "y", 1002)
        C.unregister_manager(1001)
        torch.ops.flextensor.post_compute(torch.zeros(1), "y", 1002)
        with pytest.raises(RuntimeError, match="released"):
            torch.ops.flextensor.post_compute(torch.zeros(1), "x", 1001)
        assert a.calls == [("enter", "x")] and b.calls == [("enter", "y"), ("exit", "y")]
        C.register_manager(1001, b)  # a new registration under the id replaces the old one
        torch.ops.flextensor.pre_compute(torch.zeros(1), "z", 1001)
        assert b.calls[-1] == ("enter", "z")
    finally:
        C.unregister_manager(1001)
        C.unregister_manager(1002)
