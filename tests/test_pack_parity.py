"""The product's block pack (``layout.plan_block`` + ``pack_into``) against the oracle's C pack.

The product packs a label's tensors into one host block at 128-byte aligned
offsets (allocation_block.py:124-186); the oracle restates the same copy in C
(``oracle_pack``, pinned in ``test_oracle_golden.py``). Dense tensors must
land as their raw storage bytes (C-, Fortran- or permutation-contiguous);
tensors with gaps as their C-contiguous bytes. Padding stays zero.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flextensor_amd.layout import is_dense_layout, pack_into, plan_block
from oracle import layout as ol
from oracle import native as onat

DTYPES = [torch.float32, torch.bfloat16, torch.int32, torch.uint8, torch.float64, torch.float8_e4m3fn]


def _random_tensor(gen: torch.Generator, i: int) -> torch.Tensor:
    dtype = DTYPES[i % len(DTYPES)]
    shape = [int(x) for x in torch.randint(1, 9, (3,), generator=gen)]
    t = torch.randint(0, 120, shape, generator=gen, dtype=torch.int32).to(dtype)
    kind = i % 5
    if kind == 1:
        return t.permute(2, 0, 1)  # dense, permuted strides
    if kind == 2:
        return t.transpose(0, 2)  # dense, Fortran-like
    if kind == 3 and shape[2] > 1:
        return t[:, :, ::2]  # gaps: packed C-contiguous
    if kind == 4:
        return t.reshape(-1)[: max(1, t.numel() // 2)]  # a prefix view
    return t


def _oracle_bytes(t: torch.Tensor) -> np.ndarray:
    if is_dense_layout(t) and t.numel():
        lo = t.storage_offset() * t.element_size()
        n = t.numel() * t.element_size()
        return np.frombuffer(bytes(t.untyped_storage())[lo: lo + n], dtype=np.uint8)
    return t.contiguous().view(torch.uint8).reshape(-1).numpy()


@pytest.mark.parametrize("seed", range(12))
def test_pack_into_matches_the_oracle(seed):
    gen = torch.Generator().manual_seed(seed)
    tensors = [_random_tensor(gen, seed + i) for i in range(1 + seed % 7)]
    slots, total = plan_block(tensors)
    offsets, want_total = ol.packed_layout([t.numel() * t.element_size() for t in tensors])
    assert [s.offset for s in slots] == offsets and total == want_total
    block = torch.zeros(total, dtype=torch.uint8)
    views = pack_into(block, slots, tensors)
    want = np.zeros(total, np.uint8)
    onat.pack(want, offsets, [_oracle_bytes(t) for t in tensors])
    assert np.array_equal(block.numpy(), want)
    for v, t in zip(views, tensors):
        assert torch.equal(v.view(torch.uint8) if v.dtype == torch.float8_e4m3fn else v,
                           t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t)


def test_packed_layout_rule_matches_brute_force():
    """layout.is_packed_layout (utils.py:86-98) against enumerating every element offset: a layout is
    packed exactly when its offsets are 0..numel-1, each once. All ranks up to 3, sizes 0-3, strides 0-7."""
    import itertools

    from flextensor_amd.layout import is_packed_layout

    checked = 0
    for rank in range(4):
        for shape in itertools.product(range(4), repeat=rank):
            for stride in itertools.product(range(8), repeat=rank):
                n = 1
                for d in shape:
                    n *= d
                offsets = sorted(sum(i * s for i, s in zip(idx, stride))
                                 for idx in itertools.product(*(range(d) for d in shape)))
                want = n == 0 or offsets == list(range(n))
                assert is_packed_layout(shape, stride) == want, (shape, stride)
                checked += 1
    assert checked > 30000
