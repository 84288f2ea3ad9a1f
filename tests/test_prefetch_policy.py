"""The piecewise prefetch policy and the loaders' joins, on the CPU.

Cases of the reference's tests/unit/test_piecewise_prefetch_policy.py:24-163:
a prefetch still outstanding at a piece join is reported once (or raised in
strict mode); a wait clears it; at the end-of-forward join a prefetch for a
label already waited this pass is the next pass's and is not reported; and a
strict raise at a join still leaves the loader's transfer map cleared.
"""

from __future__ import annotations

import logging
from unittest.mock import MagicMock

import pytest

from flextensor_amd.loaders import PreallocatedBatchTransferTensorLoader, PreallocatedBatchTransferTensorLoaderReordered
from flextensor_amd.prefetch_policy import OutstandingPrefetch, PiecewisePrefetchPolicy, PiecewisePrefetchPolicyError


def test_disabled_is_noop(caplog):
    policy = PiecewisePrefetchPolicy(enabled=False)
    policy.on_schedule("L1", "L4")
    with caplog.at_level(logging.WARNING):
        assert policy.on_piece_join() == []
    assert "piecewise prefetch policy" not in caplog.text


def test_same_label_outstanding_at_join_warns(caplog):
    policy = PiecewisePrefetchPolicy(enabled=True)
    policy.on_schedule("layers.0", "layers.0")
    with caplog.at_level(logging.WARNING):
        assert policy.on_piece_join() == [OutstandingPrefetch("layers.0", "layers.0")]
    assert "layers.0" in caplog.text and "H2D prefetch" in caplog.text


def test_remapped_outstanding_warns_once(caplog):
    policy = PiecewisePrefetchPolicy(enabled=True)
    with caplog.at_level(logging.WARNING):
        policy.on_schedule("L1", "L4")
        assert policy.on_piece_join() == [OutstandingPrefetch("L1", "L4")]
        policy.on_schedule("L1", "L4")
        assert policy.on_piece_join() == [OutstandingPrefetch("L1", "L4")]
    assert "L1" in caplog.text and "L4" in caplog.text
    assert caplog.text.count("H2D prefetch") == 1


def test_wait_clears_outstanding(caplog):
    policy = PiecewisePrefetchPolicy(enabled=True)
    policy.on_schedule("L1", "L4")
    policy.on_wait("L4")
    with caplog.at_level(logging.WARNING):
        assert policy.on_piece_join() == []
    assert "piecewise prefetch policy" not in caplog.text


def test_strict_raises_and_reset_clears():
    policy = PiecewisePrefetchPolicy(enabled=True, strict=True)
    policy.on_schedule("L1", "L4")
    with pytest.raises(PiecewisePrefetchPolicyError, match=r"L1.*L4"):
        policy.on_piece_join()
    policy.on_schedule("L1", "L4")
    policy.reset()
    assert policy.on_piece_join() == []


def test_end_of_forward_skips_next_pass_prefetch(caplog):
    policy = PiecewisePrefetchPolicy(enabled=True, strict=True)
    policy.on_schedule("L2", "L0")
    policy.on_wait("L0")
    policy.on_schedule("L_last", "L0")  # the last layer prefetches L0 for the next pass
    with caplog.at_level(logging.WARNING):
        assert policy.on_piece_join(at_last_layer=True) == []
    assert "piecewise prefetch policy" not in caplog.text and policy._outstanding == {}


def test_end_of_forward_flags_a_never_waited_prefetch():
    policy = PiecewisePrefetchPolicy(enabled=True, strict=True)
    policy.on_schedule("L1", "L4")
    with pytest.raises(PiecewisePrefetchPolicyError, match="end-of-forward"):
        policy.on_piece_join(at_last_layer=True)


def test_mid_forward_join_has_no_next_pass_exemption():
    policy = PiecewisePrefetchPolicy(enabled=True, strict=True)
    policy.on_schedule("L2", "L0")
    policy.on_wait("L0")
    policy.on_schedule("L_last", "L0")
    with pytest.raises(PiecewisePrefetchPolicyError, match="PIECEWISE"):
        policy.on_piece_join(at_last_layer=False)


def _bare_loader(cls):
    loader = object.__new__(cls)
    loader.piecewise_prefetch_policy = PiecewisePrefetchPolicy(enabled=True, strict=True)
    loader.scheduled_transfers = {"keep": object()}
    loader._transfer_runtime = MagicMock()
    loader._transfer_runtime.is_active = False
    loader._compute_to_block_ids = {}
    loader.backend = MagicMock()
    loader.transfer_stream = MagicMock()
    loader.last_layer_label = "L_last"
    loader.offload_timing_collector = MagicMock()
    loader.link_bound = False
    return loader


def test_join_after_forward_clears_the_map_when_strict_raises():
    loader = _bare_loader(PreallocatedBatchTransferTensorLoader)
    loader.piecewise_prefetch_policy.on_schedule("L0", "L1")
    with pytest.raises(PiecewisePrefetchPolicyError):
        loader.join_after_forward()
    assert loader.scheduled_transfers == {}


def test_last_layer_exit_clears_the_map_when_strict_raises():
    loader = _bare_loader(PreallocatedBatchTransferTensorLoader)
    loader.piecewise_prefetch_policy.on_schedule("L0", "L1")
    with pytest.raises(PiecewisePrefetchPolicyError):
        loader.exit("L_last")
    assert loader.scheduled_transfers == {}


def test_reordered_last_layer_exit_allows_the_next_pass_prefetch():
    loader = _bare_loader(PreallocatedBatchTransferTensorLoaderReordered)
    pp = loader.piecewise_prefetch_policy
    pp.on_schedule("L1", "L0")
    pp.on_wait("L0")
    pp.on_schedule("L_last", "L0")
    loader.exit("L_last")  # must not raise
    assert loader.scheduled_transfers == {}
