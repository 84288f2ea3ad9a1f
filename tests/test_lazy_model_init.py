"""Checkpoint mapping and split-device construction on the CPU.

The safetensors parser is pinned byte for byte against the ``safetensors``
package's own reader on every dtype the format names, and against files with
broken headers. Construction keeps parameters on the meta device while
buffers keep their computed values, and object identity (tied weights,
``weight.scale`` attributes) survives both construction and loading: the
pattern of the reference's tests/unit/test_tensor_inner_fields.py:11-65.
"""

from __future__ import annotations

import gc
import json
import struct
import threading

import pytest
import torch
from safetensors.torch import load_file, save_file
from torch import nn

from flextensor_amd import lazy_model_init as L
from flextensor_amd import workloads as W
from flextensor_amd.profile import save_state
from tests.test_profile import _mock_state

SMALL = W.LlamaShape(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, inter=96, vocab=128, max_seq=32)


def _all_dtypes() -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(3)
    base = torch.randn(5, 7, generator=g)
    ints = torch.randint(-100, 100, (4, 6), generator=g)
    return {
        "f64": base.double(), "f32": base, "f16": base.half(), "bf16": base.bfloat16(),
        "e4m3": base.to(torch.float8_e4m3fn), "e5m2": base.to(torch.float8_e5m2),
        "i64": ints, "i32": ints.int(), "i16": ints.short(), "i8": ints.to(torch.int8),
        "u8": ints.abs().to(torch.uint8), "u16": ints.abs().to(torch.uint16), "u32": ints.abs().to(torch.uint32),
        "u64": ints.abs().to(torch.uint64), "bool": ints > 0,
        "scalar": torch.tensor(2.5), "empty": torch.zeros(0, 3), "odd": torch.arange(3, dtype=torch.int8),
    }


def _bytes(t: torch.Tensor) -> bytes:
    return t.contiguous().view(-1).view(torch.uint8).numpy().tobytes() if t.numel() else b""


def test_parser_matches_the_safetensors_reader(tmp_path):
    path = tmp_path / "all.safetensors"
    save_file(_all_dtypes(), str(path), metadata={"format": "pt", "note": "x"})
    want = load_file(str(path))
    f = L.SafetensorsFile(path)
    assert sorted(f.keys()) == sorted(want) and len(f) == len(want)
    assert f.metadata == {"format": "pt", "note": "x"}
    for name, w in want.items():
        got = f.get(name)
        assert got.dtype == w.dtype and got.shape == w.shape and got.is_contiguous(), name
        assert _bytes(got) == _bytes(w), name
        assert f.dtype(name) == w.dtype and f.shape(name) == tuple(w.shape)


def test_views_are_private_and_outlive_the_file_object(tmp_path):
    path = tmp_path / "a.safetensors"
    save_file({"a": torch.arange(1000, dtype=torch.float32)}, str(path))
    f = L.SafetensorsFile(path)
    t = f.get("a")
    del f
    gc.collect()
    t.add_(1)  # copy-on-write mapping: the file keeps its bytes
    assert torch.equal(t, torch.arange(1000, dtype=torch.float32) + 1)
    assert torch.equal(load_file(str(path))["a"], torch.arange(1000, dtype=torch.float32))


def _raw_file(path, header, data=b"", header_len=None):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h) if header_len is None else header_len) + h + data)
    return path


@pytest.mark.parametrize("case", ["short", "length", "json", "object", "dtype", "offsets", "nbytes", "shape"])
def test_broken_headers_are_rejected(tmp_path, case):
    p = tmp_path / "bad.safetensors"
    good = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "length":
        _raw_file(p, good, bytes(8), header_len=1 << 40)
    elif case == "json":
        p.write_bytes(struct.pack("<Q", 5) + b"{nope" + bytes(8))
    elif case == "object":
        _raw_file(p, [1, 2], bytes(8))
    elif case == "dtype":
        _raw_file(p, {"t": {"dtype": "F12", "shape": [2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "offsets":
        _raw_file(p, {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, bytes(4))
    elif case == "nbytes":
        _raw_file(p, {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, bytes(8))
    else:
        _raw_file(p, {"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}, bytes(8))
    with pytest.raises(ValueError):
        L.SafetensorsFile(p)


def test_load_specific_keys_strict_and_lenient(tmp_path):
    path = tmp_path / "k.safetensors"
    save_file({"a": torch.ones(3), "b": torch.zeros(2, dtype=torch.bfloat16)}, str(path))
    got = L.load_specific_keys(str(path), ["a", "missing"])
    assert list(got) == ["a"] and torch.equal(got["a"], torch.ones(3))
    with pytest.raises(KeyError, match="missing"):
        L.load_specific_keys(str(path), ["a", "missing"], strict=True)
    with pytest.raises(KeyError):
        L.SafetensorsFile(path).get("missing")


class LinearWithScale(nn.Module):
    """``self.weight.scale = self.scale = nn.Parameter(...)`` (tests/unit/test_tensor_inner_fields.py:11-45)."""

    def __init__(self, n_in: int, n_out: int, block: int = 16) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.randn(n_out, n_in))
        self.weight.scale = self.scale = nn.Parameter(torch.randn((n_out + block - 1) // block,
                                                                  (n_in + block - 1) // block))

    def forward(self, x):
        assert self.weight.scale.device == self.weight.device
        return nn.functional.linear(x, self.weight) * self.weight.scale.mean()


class InnerFields(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.layer1 = LinearWithScale(32, 48)
        self.layer2 = LinearWithScale(48, 32)

    def forward(self, x):
        return self.layer2(torch.relu(self.layer1(x)))


class Tied(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.embed = nn.Embedding(10, 8)
        self.head = nn.Linear(8, 10, bias=False)
        self.head.weight = self.embed.weight


def test_split_construction_keeps_buffers_and_restores_registration():
    orig = (nn.Module.register_parameter, nn.Module.register_buffer)
    model = L.create_split_device_model(W.LlamaModel, (SMALL,), None, "meta", "cpu")
    assert (nn.Module.register_parameter, nn.Module.register_buffer) == orig
    assert all(p.device.type == "meta" for p in model.parameters())
    ref = W.LlamaModel(SMALL)
    for name, b in model.named_buffers():
        assert b.device.type == "cpu" and torch.equal(b, dict(ref.named_buffers())[name]), name
    assert [n for n, _ in model.named_parameters()] == [n for n, _ in ref.named_parameters()]


def test_split_construction_acts_on_its_own_thread_only():
    inside, built = threading.Event(), threading.Event()
    other: dict[str, torch.device] = {}

    def build():
        inside.wait(10)
        other["device"] = nn.Linear(4, 4).weight.device
        built.set()

    t = threading.Thread(target=build)
    t.start()
    with L.split_device_init("meta", "cpu"):
        inside.set()
        assert built.wait(10)
        mine = nn.Linear(4, 4)
        with pytest.raises(RuntimeError, match="already active"):
            with L.split_device_init("meta", "cpu"):
                pass
    t.join()
    assert other["device"].type == "cpu" and mine.weight.device.type == "meta"


def test_inner_fields_survive_construction_and_loading():
    model = L.create_split_device_model(InnerFields, (), None, "meta", "cpu")
    for layer in (model.layer1, model.layer2):
        assert layer.weight.scale is layer.scale and layer.scale.device.type == "meta"
    src = InnerFields()
    left = L._assign(model, dict(src.state_dict()))
    assert left == []
    for name in ("layer1", "layer2"):
        layer, ref = getattr(model, name), getattr(src, name)
        assert layer.weight.scale is layer.scale
        assert torch.equal(layer.weight, ref.weight) and torch.equal(layer.weight.scale, ref.scale)
    x = torch.randn(3, 32)
    assert torch.equal(model(x), src(x))


def test_tied_weights_stay_tied_from_one_checkpoint_name():
    model = L.create_split_device_model(Tied, (), None, "meta", "cpu")
    assert model.head.weight is model.embed.weight
    w = torch.randn(10, 8)
    assert L._assign(model, {"embed.weight": w}) == []
    assert model.head.weight is model.embed.weight and torch.equal(model.head.weight, w)


def test_assign_checks_shapes_and_reports_what_stays_on_meta():
    model = L.create_split_device_model(InnerFields, (), None, "meta", "cpu")
    with pytest.raises(ValueError, match="shape"):
        L._assign(model, {"layer1.weight": torch.zeros(3, 3)})
    left = L._assign(model, {"layer1.weight": torch.zeros(48, 32)})
    assert sorted(left) == ["layer1.scale", "layer2.scale", "layer2.weight"]


def test_load_model_from_profile_argument_errors(tmp_path):
    with pytest.raises(ValueError, match="safetensor_path is required"):
        L.load_model_from_profile(None, str(tmp_path), InnerFields)
    save_state(_mock_state(["layer1.weight"]), tmp_path)  # a per-tensor strategy profile
    ckpt = tmp_path / "m.safetensors"
    save_file(InnerFields().state_dict(), str(ckpt))
    with pytest.raises(ValueError, match="transfer mode"):
        L.load_model_from_profile(None, str(tmp_path), InnerFields, safetensor_path=str(ckpt))
