"""The measured link curve's diagnostic table (link_model.format_memory_transfer_table).

Cases of the reference's tests/unit/test_memory_transfer_table.py:11-58,
restated: the empty message, a single row with its bandwidth, rows in
ascending size order, the ``=`` rules at top and bottom, binary size units.
"""

from __future__ import annotations

from flextensor_amd.link_model import LinkMeasurement, format_memory_transfer_table


def _rows(table: str) -> list[str]:
    return [ln for ln in table.split("\n")
            if ln.strip() and not ln.startswith(("=", "-")) and "Size" not in ln and "Memory" not in ln]


def test_empty_curve_has_a_message():
    assert format_memory_transfer_table({}) == "No memory transfer statistics available."


def test_one_row_with_its_bandwidth():
    table = format_memory_transfer_table({1 << 20: 1.0})  # 1 MiB in 1 ms = 1.049 GB/s
    (row,) = _rows(table)
    assert row.split() == ["1048576", "1.0", "MiB", "1.000", "1.049"]


def test_rows_ascend_by_size():
    rows = _rows(format_memory_transfer_table({4096: 0.01, 1024: 0.005, 1 << 20: 0.5}))
    assert [int(r.split()[0]) for r in rows] == [1024, 4096, 1 << 20]


def test_rules_at_top_and_bottom():
    lines = format_memory_transfer_table({1024: 0.01}).split("\n")
    assert lines[0] == lines[2] == lines[-1] == "=" * 110
    assert lines[1] == "Memory Transfer Statistics" and lines[4] == "-" * 110


def test_binary_size_units():
    table = format_memory_transfer_table({512: 0.01, 1024: 0.01, 1 << 20: 0.5, 1 << 30: 50.0})
    for text in ("512 B", "1.0 KiB", "1.0 MiB", "1.0 GiB"):
        assert text in table


def test_zero_time_reads_as_zero_bandwidth():
    (row,) = _rows(format_memory_transfer_table({4096: 0.0}))
    assert row.split()[-1] == "0.000"


def test_a_measurement_renders_its_sdma_curve():
    link = LinkMeasurement.from_dict({"kernel_max_bytes": 0, "split_min_bytes": 1 << 62, "n_copy_streams": 1,
                                      "sdma_ms": {"65536": 0.0125, "1048576": 0.03}, "kernel_ms": {}}, "test")
    rows = _rows(format_memory_transfer_table(link.memory_transfer_stats()))
    assert [r.split()[0] for r in rows] == ["65536", "1048576"]
    assert rows[0].split()[-1] == f"{65536 / 0.0125e-3 / 1e9:.3f}"
