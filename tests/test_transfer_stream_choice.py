"""Choice of the transfer stream, on the CPU with the probe replaced by recorded timings.

The transfer stream must not share the compute stream's hardware queue, or
every copy waits behind the forward's kernels. The first candidate whose tiny
fill finishes in the first half of the compute stream's queued work is kept;
when none does, the failure names every measurement instead of settling for a
stream that would serialize transfers behind compute.
"""

from __future__ import annotations

from unittest import mock

import pytest
import torch

from flextensor_amd import hip


class _FakeStream:
    def __init__(self, i: int) -> None:
        self.i = i


@pytest.fixture
def fake_device():
    made: list[_FakeStream] = []

    def new_stream(dev, name="transfer"):
        made.append(_FakeStream(len(made)))
        return made[-1]

    saved = (dict(hip._TRANSFER_STREAMS), list(hip._REJECTED_STREAMS), dict(hip._STREAM_PROBES))
    hip._TRANSFER_STREAMS.pop(7, None)
    hip._STREAM_PROBES.pop(7, None)
    with mock.patch.object(hip, "new_stream", new_stream), mock.patch.object(hip, "current_stream", lambda d: None):
        yield made
    hip._TRANSFER_STREAMS.clear(), hip._TRANSFER_STREAMS.update(saved[0])
    hip._REJECTED_STREAMS[:] = saved[1]
    hip._STREAM_PROBES.clear(), hip._STREAM_PROBES.update(saved[2])


def test_first_concurrent_candidate_is_kept_and_reported(fake_device):
    timings = iter([(2.0, 2.05), (2.0, 1.9), (2.0, 0.02), (2.0, 0.01)])
    with mock.patch.object(hip, "_probe_concurrency", lambda c, comp, d: next(timings)):
        s = hip.transfer_stream(torch.device("cuda", 7))
    assert s is fake_device[2]
    assert hip.transfer_stream(torch.device("cuda", 7)) is s  # cached, no second probe
    assert hip._REJECTED_STREAMS[-2:] == fake_device[:2]  # rejected candidates stay alive
    probe = hip.transfer_stream_probe(torch.device("cuda", 7))
    assert probe == {"chosen_candidate": 2, "rejected": 2, "attempts": 8, "compute_busy_ms": 2.0,
                     "transfer_fill_done_ms": 0.02}


def test_no_concurrent_candidate_is_an_error_naming_the_timings(fake_device):
    with mock.patch.object(hip, "_probe_concurrency", lambda c, comp, d: (2.0, 2.1)):
        with pytest.raises(hip.TransferStreamError, match=r"each of 3 new default-priority streams") as info:
            hip.transfer_stream(torch.device("cuda", 7), attempts=3)
    assert "(2.0, 2.1)" in str(info.value) and "GPU_MAX_HW_QUEUES" in str(info.value)
    assert 7 not in hip._TRANSFER_STREAMS and hip.transfer_stream_probe(torch.device("cuda", 7)) is None


def test_slowed_dispatch_still_counts_as_concurrent(fake_device):
    """Under a profiler every dispatch is slower and a concurrent fill lands near 60% of the compute time;
    only a fill that waits for (nearly) all of it marks a shared queue."""
    timings = iter([(1.5, 1.49), (1.5, 0.9)])
    with mock.patch.object(hip, "_probe_concurrency", lambda c, comp, d: next(timings)):
        s = hip.transfer_stream(torch.device("cuda", 7))
    assert s is fake_device[1] and hip.transfer_stream_probe(torch.device("cuda", 7))["rejected"] == 1
