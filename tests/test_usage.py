"""The `.colizig_usage` priors file on the host (expert_usage.zig:53-128)."""
from __future__ import annotations

import numpy as np

from colizig_amd.usage import ExpertUsage, MAGIC


def test_round_trip_and_layout(tmp_path):
    p = str(tmp_path / ".colizig_usage")
    u = ExpertUsage(3, 4, np.arange(12, dtype=np.uint64))
    u.save(p)
    raw = open(p, "rb").read()
    assert raw[:4] == MAGIC and int.from_bytes(raw[4:8], "little") == 3 and int.from_bytes(raw[8:12], "little") == 4
    assert len(raw) == 12 + 12 * 8 and int.from_bytes(raw[12 + 5 * 8:12 + 6 * 8], "little") == 5
    v = ExpertUsage.load(p, 3, 4)
    assert v is not None and np.array_equal(v.counts, u.counts)


def test_mismatch_and_missing_read_as_no_priors(tmp_path):
    p = str(tmp_path / ".colizig_usage")
    assert ExpertUsage.load(p, 3, 4) is None
    ExpertUsage(3, 4).save(p)
    assert ExpertUsage.load(p, 4, 3) is None and ExpertUsage.load(p, 3, 5) is None
    open(p, "ab").write(b"x")
    assert ExpertUsage.load(p, 3, 4) is None


def test_save_merges_and_saturates(tmp_path):
    p = str(tmp_path / ".colizig_usage")
    ExpertUsage(1, 3, np.array([1, 2, 2 ** 64 - 2], np.uint64)).save(p)
    ExpertUsage(1, 3, np.array([10, 0, 5], np.uint64)).save(p)
    assert ExpertUsage.load(p, 1, 3).counts.tolist() == [[11, 2, 2 ** 64 - 1]]


def test_top_ascending_order():
    u = ExpertUsage(1, 6, np.array([5, 0, 9, 5, 1, 0], np.uint64))
    assert u.top_ascending(0, 3) == [3, 0, 2]  # hottest 2, then 0 and 3 tied (lower id first), ascending heat
    assert u.top_ascending(0, 10) == [4, 3, 0, 2]  # zero counts never picked
