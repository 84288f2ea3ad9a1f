"""Offload-unit selection by include/exclude patterns, on the CPU.

Cases of the reference's tests/unit/test_forward_patching.py:723-1560
(ancestor guard, parameter-level include patterns and their derivation,
unmatched-pattern warnings and aggregate errors, label uniqueness, the
DeepSeek-style ``*.scale`` alias) on models of the same shapes.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from flextensor_amd.selection import (module_patterns, parameter_filter, partition, path_matches, prefix_matches,
                                      select_offload_units)


class SimpleLayer(nn.Module):
    def __init__(self, dim: int = 10) -> None:
        super().__init__()
        self.linear = nn.Linear(dim, dim)


class ModelWithLayers(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layer1, self.layer2, self.layer3 = SimpleLayer(), SimpleLayer(), SimpleLayer()


class AttentionBlock(nn.Module):
    def __init__(self, dim: int = 10) -> None:
        super().__init__()
        self.q_proj = nn.Linear(dim, dim)
        self.k_proj = nn.Linear(dim, dim)


class TransformerLayer(nn.Module):
    def __init__(self, dim: int = 10) -> None:
        super().__init__()
        self.attn = AttentionBlock(dim)
        self.norm = nn.LayerNorm(dim)


class NestedModel(nn.Module):
    def __init__(self, n: int = 2, dim: int = 10) -> None:
        super().__init__()
        self.layers = nn.ModuleList(TransformerLayer(dim) for _ in range(n))
        self.head = nn.Linear(dim, dim)


class WrappedNestedModel(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.model = NestedModel()


class LayerWithDirectParam(nn.Module):
    def __init__(self, dim: int = 10) -> None:
        super().__init__()
        self.x = nn.Parameter(torch.randn(dim))
        self.linear = nn.Linear(dim, dim)


class ModelWithDirectParams(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layers = nn.ModuleList(LayerWithDirectParam() for _ in range(2))


class LinearWithScale(nn.Module):
    def __init__(self, dim: int = 10) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.randn(dim, dim))
        self.weight.scale = self.scale = nn.Parameter(torch.randn(dim))


class ModelWithInnerFieldLayers(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layers = nn.ModuleList(LinearWithScale() for _ in range(2))


def _paths(model: nn.Module) -> list[str]:
    return [p for p, _ in model.named_modules() if p]


@pytest.mark.parametrize("path, pattern, recursive, want", [
    ("layers.0", "layers.*", False, True),
    ("layers.0.attn", "layers.*", False, False),
    ("layers.0.attn", "layers.*", True, True),
    ("layers.0.attn", "*.attn", True, True),
    ("layers.0.attn", "*.attn", False, False),
    ("layers.10", "layers.1?", False, True),
    ("layers.1", "layers.1?", False, False),
    ("model.layers.3.mlp", "model.*.mlp", True, True),
    ("q_proj", "*proj", False, True),
])
def test_segment_glob(path, pattern, recursive, want):
    assert path_matches(path, pattern, recursive_star=recursive) is want


def test_partition_and_empty_bodies():
    assert partition(["layers.*", "name:embed", "class:MoELayer"]) == (["layers.*", "embed"], ["MoELayer"])
    for bad in ("class:", "name:  "):
        with pytest.raises(ValueError, match="empty body"):
            partition([bad])


def test_module_patterns_from_parameter_patterns():
    nested = NestedModel()
    assert "layers.*" in module_patterns(["layers.*"], _paths(nested), nested)
    assert "layers.*" in module_patterns(["layers.*.weight"], _paths(nested), nested)
    assert module_patterns(["layers.*.weight", "layers.*.bias"], _paths(nested), nested).count("layers.*") == 1
    flat = ModelWithLayers()
    assert set(module_patterns(["layer1.linear.weight"], _paths(flat), flat)) == {"layer1.linear"}
    assert set(module_patterns(["*.weight"], _paths(flat), flat)) == {"layer1.linear", "layer2.linear",
                                                                         "layer3.linear"}
    assert module_patterns(["*"], _paths(flat), flat) == ["*"]


def test_star_weight_on_a_wrapper_names_the_owners():
    m = WrappedNestedModel()
    got = set(module_patterns(["*.weight"], _paths(m), m))
    assert got == {"model.layers.0.attn.q_proj", "model.layers.0.attn.k_proj", "model.layers.0.norm",
                   "model.layers.1.attn.q_proj", "model.layers.1.attn.k_proj", "model.layers.1.norm", "model.head"}
    assert module_patterns(["*.weight"], _paths(m), None) == []  # no model: no per-parameter fallback
    mixed = set(module_patterns(["model.layers.*", "*.bias"], _paths(m), m))
    assert "model.layers.*" in mixed and "model.head" in mixed and "*" not in mixed


def test_unmatched_sibling_does_not_widen_to_the_ancestor():
    m = WrappedNestedModel()
    m.model.norm_f = nn.LayerNorm(10)
    got = set(module_patterns(["model.layers.*", "model.norm", "model.norm_f", "model.head"], _paths(m), m))
    assert {"model.layers.*", "model.norm_f", "model.head"} <= got and "model" not in got
    units = select_offload_units(m, ["model.layers.*", "model.norm", "model.head"], [])
    assert units == ["model.layers.0", "model.layers.1", "model.head"]


def test_parameter_patterns_select_owning_modules():
    assert select_offload_units(NestedModel(), ["layers.*.weight"], []) == ["layers.0", "layers.1"]
    assert select_offload_units(ModelWithLayers(), ["*"], []) == ["layer1", "layer2", "layer3"]
    units = select_offload_units(WrappedNestedModel(), ["*.weight"], [])
    assert len(units) > 1 and "model" not in units
    assert select_offload_units(ModelWithLayers(), ["*.weight"], []) == ["layer1.linear", "layer2.linear",
                                                                        "layer3.linear"]


def test_ancestor_guard_keeps_the_outermost_unit():
    m = NestedModel()
    assert select_offload_units(m, ["layers.*", "layers.*.attn"], []) == ["layers.0", "layers.1"]
    assert select_offload_units(m, ["layers.*", "*.weight"], []) == ["layers.0", "layers.1", "head"]
    assert select_offload_units(ModelWithDirectParams(), ["*.x", "*.weight"], []) == ["layers.0", "layers.1"]
    assert select_offload_units(ModelWithInnerFieldLayers(), ["*.scale"], []) == ["layers.0", "layers.1"]


def test_excludes_span_segments_and_classes():
    m = NestedModel(n=3)
    assert select_offload_units(m, ["layers.*"], ["layers.1"]) == ["layers.0", "layers.2"]
    assert select_offload_units(m, ["layers.*", "head"], ["*.2"]) == ["layers.0", "layers.1", "head"]
    assert select_offload_units(m, ["layers.*", "head"], ["class:Linear"]) == ["layers.0", "layers.1", "layers.2"]
    assert select_offload_units(m, ["class:torch.nn.modules.linear.*"], []) == ["layers.0.attn.q_proj",
                                                                               "layers.0.attn.k_proj",
                                                                               "layers.1.attn.q_proj",
                                                                               "layers.1.attn.k_proj",
                                                                               "layers.2.attn.q_proj",
                                                                               "layers.2.attn.k_proj", "head"]


def test_unmatched_patterns_warn_and_empty_selections_log_errors(caplog):
    m = NestedModel()
    with caplog.at_level("WARNING", logger="flextensor_amd.selection"):
        assert select_offload_units(m, ["layers.*", "bogus"], ["nothing.here"]) == ["layers.0", "layers.1"]
    assert "Include pattern 'bogus' did not match" in caplog.text
    assert "Exclude pattern 'nothing.here' did not match" in caplog.text
    assert "Include pattern 'layers.*'" not in caplog.text
    caplog.clear()
    with caplog.at_level("WARNING", logger="flextensor_amd.selection"):
        assert select_offload_units(m, ["bogus", "also_bogus"], []) == []
    assert "No modules matched any include pattern" in caplog.text
    caplog.clear()
    with caplog.at_level("WARNING", logger="flextensor_amd.selection"):
        assert select_offload_units(m, ["layers.*"], ["layers.*"]) == []
    assert "All 2 included modules were removed" in caplog.text
    caplog.clear()
    with caplog.at_level("WARNING", logger="flextensor_amd.selection"):
        assert select_offload_units(m, ["layers.*.weight", "*.bias"], ["*.norm.weight"]) == ["layers.0", "layers.1",
                                                                                             "head"]
    assert "did not match" not in caplog.text  # parameter patterns count as matched
    caplog.clear()
    with caplog.at_level("WARNING", logger="flextensor_amd.selection"):
        assert select_offload_units(m, [], []) == []
    assert "empty list" in caplog.text and "No modules matched" not in caplog.text


# ---- which parameters of a unit stream (tests/unit/test_tensor_discovery.py) ----------------------


@pytest.mark.parametrize("path,patterns,want", [
    ("layers.0.weight", ["*"], True), ("head.bias", ["*"], True),
    ("layers.0.weight", ["layers.*"], True), ("layers.0.bias", ["layers.*"], True), ("head.weight", ["layers.*"], False),
    ("layers.0.weight", ["*.weight"], True), ("layers.0.bias", ["*.weight"], False),
    ("layers.0.attn.weight", ["layers.*.attn.weight"], True), ("layers.0.attn.bias", ["layers.*.attn.weight"], False),
    ("layers.0.mlp.weight", ["layers.*.attn.weight"], False),
    ("layers.0.attn.q_proj.weight", ["layers.*"], True), ("layers.0.mlp.gate.weight", ["layers.*"], True),
    ("embed.weight", ["layers.*"], False),
    ("layers.0.attn.q_proj.weight", ["*.weight"], True), ("layers.0.attn.q_proj.bias", ["*.weight"], False),
    ("layers.0.attn.q_proj.weight", ["layers.*.attn"], True), ("layers.0.attn.k_proj.bias", ["layers.*.attn"], True),
    ("layers.0.mlp.gate.weight", ["layers.*.attn"], False),
    ("layer1.weight", ["*layer*"], True), ("my_layer.bias", ["*layer*"], True), ("layers.0.weight", ["*layer*"], True),
    ("head.weight", ["*layer*"], False), ("embed.bias", ["*layer*"], False),
])
def test_prefix_matching(path, patterns, want):
    """_any_prefix_matches cases, :1413-1470."""
    assert prefix_matches(path, patterns) is want


@pytest.mark.parametrize("path,include,exclude,want", [
    ("layers.0.weight", ["*"], [], True),
    ("layers.0.weight", ["*.bias"], [], False), ("layers.0.weight", ["*.bias"], ["*.weight"], False),
    ("layers.0.weight", ["*"], ["*.weight"], False),
    ("layers.0.bias", ["*.bias"], [], True),
    ("layers.0.attn.q.weight", ["layers.*"], [], True), ("embed.weight", ["layers.*"], [], False),
    ("layers.0.attn.q.weight", ["*"], ["layers.*"], False), ("embed.weight", ["*"], ["layers.*"], True),
    ("layers.0.mlp.weight", ["layers.*"], ["layers.*.attn"], True),
    ("layers.0.attn.q.weight", ["layers.*"], ["layers.*.attn"], False),
    ("layers.0.weight", ["*.weight"], ["layers.0.*"], False),
    ("my_layer.weight", ["*layer*"], [], True), ("my_layer.weight", ["*layer*"], ["*layer*"], False),
    ("my_layer.weight", ["*layer*"], ["*weight*"], True),  # a leaf segment is not a prefix of its own
])
def test_parameter_included_and_not_excluded(path, include, exclude, want):
    """_should_offload_param cases, :1475-1530."""
    assert parameter_filter(nn.Module(), include, exclude)(path) is want


class _Bar(nn.Module):
    def __init__(self):
        super().__init__()
        self.linear = nn.Linear(10, 10)


class _Inner(nn.Module):
    def __init__(self):
        super().__init__()
        self.bar = _Bar()
        self.norm = nn.LayerNorm(10)


def _nested():
    m = nn.Module()
    m.foo = nn.ModuleDict({"layers": nn.ModuleList([_Inner(), _Inner()])})
    return m


@pytest.mark.parametrize("exclude", [["foo.layers.0.bar"], ["foo.layers.*.bar"]])
def test_excluded_module_inside_a_unit_keeps_its_parameters_out(exclude):
    """:1139-1193: excluding a submodule of a unit drops all of its parameters and keeps the rest."""
    m = _nested()
    keep = parameter_filter(m, ["*"], exclude)
    names = [n for n, _ in m.foo["layers"][0].named_parameters()]
    streamed = {n for n in names if keep(f"foo.layers.0.{n}")}
    assert streamed == {"norm.weight", "norm.bias"}


def test_class_patterns_cover_the_parameters_below_the_class():
    m = _nested()
    keep = parameter_filter(m, ["class:_Inner"], ["class:LayerNorm"])
    assert keep("foo.layers.1.bar.linear.weight") and not keep("foo.layers.1.norm.bias")
    assert not parameter_filter(m, ["class:LayerNorm"], [])("foo.layers.0.bar.linear.bias")


def test_parameter_patterns_choose_units_and_their_parameters():
    """:79-116 with the parameter filter: the owning modules become units, and only the named parameters
    of them stream."""
    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.encoder = nn.Sequential(nn.Linear(4, 4), nn.ReLU(), nn.Linear(4, 4))
            self.head = nn.Linear(4, 2)

    m = Model()
    include, exclude = ["encoder.0.weight", "encoder.2.weight", "head"], ["encoder.2"]
    assert set(select_offload_units(m, include, exclude)) == {"encoder.0", "head"}
    keep = parameter_filter(m, include, exclude)
    assert [n for n, _ in m.named_parameters() if keep(n)] == ["encoder.0.weight", "head.weight", "head.bias"]
    assert set(select_offload_units(m, ["class:Linear"], ["head"])) == {"encoder.0", "encoder.2"}
    assert set(select_offload_units(m, ["encoder", "encoder.*"], [])) == {"encoder"}
    assert select_offload_units(m, ["encoder.9.weight"], []) == []
