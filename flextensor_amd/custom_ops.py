"""Compute-boundary custom ops for compiled forwards.

``flextensor::pre_compute`` and ``flextensor::post_compute`` carry an offload
unit's ``enter`` / ``exit`` through ``torch.compile``, with the reference's
schema (custom_ops.py:313-328): each takes a tensor it declares as mutated
(``Tensor(a!)``) only so the compiler keeps the op ordered against the unit's
compute, the unit's name, and the manager id. Their values are never written.

The ops call the manager registered under the id; with none registered they
do nothing, and a manager that was registered and then released raises, as
the reference does (custom_ops.py:240-259), because skipping ``enter`` would
let the unit read a slot that holds another unit's weights.
"""

from __future__ import annotations

from typing import Any

import torch
from torch.library import Library

_MANAGERS: dict[int, Any] = {}
_RELEASED: set[int] = set()


def register_manager(manager_id: int, manager: Any) -> None:
    """Route the ops for ``manager_id`` to ``manager._enter`` / ``manager._exit``."""
    _MANAGERS[manager_id] = manager
    _RELEASED.discard(manager_id)


def unregister_manager(manager_id: int) -> None:
    if _MANAGERS.pop(manager_id, None) is not None:
        _RELEASED.add(manager_id)


def _lookup(manager_id: int) -> Any:
    mgr = _MANAGERS.get(manager_id)
    if mgr is None and manager_id in _RELEASED:
        raise RuntimeError(f"flextensor::pre_compute/post_compute called for manager_id={manager_id}, whose offload "
                           "manager was released: skipping enter/exit would leave the unit reading a slot that "
                           "holds other weights. Offload the model again before running it.")
    return mgr


def _pre_compute_impl(input_tensor: torch.Tensor, offload_unit_name: str, manager_id: int) -> None:
    mgr = _lookup(manager_id)
    if mgr is not None:
        mgr._enter(offload_unit_name)


def _post_compute_impl(output_tensor: torch.Tensor, offload_unit_name: str, manager_id: int) -> None:
    mgr = _lookup(manager_id)
    if mgr is not None:
        mgr._exit(offload_unit_name)


def _fake(tensor: torch.Tensor, offload_unit_name: str, manager_id: int) -> None:
    return None


_LIB = Library("flextensor", "FRAGMENT")
_LIB.define("pre_compute(Tensor(a!) input_tensor, str offload_unit_name, int manager_id) -> ()")
_LIB.define("post_compute(Tensor(a!) output_tensor, str offload_unit_name, int manager_id) -> ()")
_LIB.impl("pre_compute", _pre_compute_impl, "CompositeExplicitAutograd")
_LIB.impl("post_compute", _post_compute_impl, "CompositeExplicitAutograd")
torch.library.register_fake("flextensor::pre_compute", _fake, lib=_LIB)
torch.library.register_fake("flextensor::post_compute", _fake, lib=_LIB)


def first_tensor(obj: Any) -> torch.Tensor | None:
    """The first tensor in ``obj`` (a tensor, or nested tuples / lists / dicts of them)."""
    if isinstance(obj, torch.Tensor):
        return obj
    if isinstance(obj, (tuple, list)):
        for v in obj:
            t = first_tensor(v)
            if t is not None:
                return t
    if isinstance(obj, dict):
        for v in obj.values():
            t = first_tensor(v)
            if t is not None:
                return t
    return None
