"""The streaming tier's policy objects through the C-ABI, on the CPU (host
code, no device): the bounded priority Scheduler (src/runtime/io.zig:58-140)
and the LastTokenPredictor (src/runtime/predict.zig:29-90).  The cases
restate the reference's own tests (io.zig:145-197, predict.zig:94-124) with
expert keys (the only resource kind this path schedules)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from colizig_amd import _lib

HIGH, MEDIUM, LOW = 0, 1, 2
STATS = ("submitted", "deduped", "upgraded", "rejected_full", "serviced_high", "serviced_medium", "serviced_low",
         "cancelled", "queue_peak", "queued")


@pytest.fixture()
def sched():
    hip = _lib.hip()
    made = []

    def make(cap):
        h = hip.colizig_hip_sched_create(cap)
        assert h > 0
        made.append(h)
        return h

    yield make
    for h in made:
        hip.colizig_hip_sched_destroy(h)


def _next(h):
    lay, eid = ctypes.c_uint32(), ctypes.c_uint32()
    rc = _lib.hip().colizig_hip_sched_next(h, ctypes.byref(lay), ctypes.byref(eid))
    assert rc in (0, 1)
    return (lay.value, eid.value) if rc == 1 else None


def _stats(h):
    v = (ctypes.c_uint64 * len(STATS))()
    assert _lib.hip().colizig_hip_sched_stats(h, v, len(STATS)) == 0
    return dict(zip(STATS, (int(x) for x in v)))


def test_priority_ordering(sched):
    """io.zig:147-161: HIGH drains before MEDIUM before LOW, FIFO within a
    priority."""
    hip = _lib.hip()
    h = sched(16)
    assert hip.colizig_hip_sched_submit(h, 0, 1, LOW) == 1
    assert hip.colizig_hip_sched_submit(h, 9, 100, MEDIUM) == 1
    assert hip.colizig_hip_sched_submit(h, 7, 3, HIGH) == 1
    assert hip.colizig_hip_sched_submit(h, 9, 101, HIGH) == 1
    assert [_next(h) for _ in range(5)] == [(7, 3), (9, 101), (9, 100), (0, 1), None]
    st = _stats(h)
    assert (st["serviced_high"], st["serviced_medium"], st["serviced_low"]) == (2, 1, 1)


def test_bounded_dedup_upgrade(sched):
    """io.zig:163-175: a full queue refuses; a re-submit dedups and upgrades
    (the upgraded key then comes out first)."""
    hip = _lib.hip()
    h = sched(2)
    assert hip.colizig_hip_sched_submit(h, 0, 1, LOW) == 1
    assert hip.colizig_hip_sched_submit(h, 0, 2, LOW) == 1
    assert hip.colizig_hip_sched_submit(h, 0, 3, LOW) == 0
    assert _stats(h)["rejected_full"] == 1
    assert hip.colizig_hip_sched_submit(h, 0, 1, HIGH) == 1
    st = _stats(h)
    assert st["upgraded"] == 1 and st["deduped"] == 1 and st["queued"] == 2
    assert _next(h) == (0, 1)


def test_mandatory_not_starved(sched):
    """io.zig:177-185: a HIGH key comes out first behind 50 LOW keys."""
    hip = _lib.hip()
    h = sched(64)
    for i in range(50):
        assert hip.colizig_hip_sched_submit(h, 1, i, LOW) == 1
    assert hip.colizig_hip_sched_submit(h, 2, 999, HIGH) == 1
    assert _next(h) == (2, 999)
    assert _stats(h)["queue_peak"] == 51


def test_cancel(sched):
    """io.zig:187-197: cancel removes a queued key; an absent one is 0."""
    hip = _lib.hip()
    h = sched(8)
    hip.colizig_hip_sched_submit(h, 2, 7, MEDIUM)
    assert hip.colizig_hip_sched_has(h, 2, 7) == 1
    assert hip.colizig_hip_sched_cancel(h, 2, 7) == 1
    assert hip.colizig_hip_sched_has(h, 2, 7) == 0
    assert hip.colizig_hip_sched_cancel(h, 0, 0) == 0
    assert _stats(h)["cancelled"] == 1


def test_bad_handle_and_priority(sched):
    hip = _lib.hip()
    h = sched(4)
    assert hip.colizig_hip_sched_submit(h, 0, 0, 3) == -1
    assert hip.colizig_hip_sched_submit(123456789, 0, 0, LOW) == -1
    assert hip.colizig_hip_sched_next(123456789, ctypes.byref(ctypes.c_uint32()), ctypes.byref(ctypes.c_uint32())) == -1


def _predict(h, layer, k=8):
    out = np.zeros(k, np.uint32)
    n = _lib.hip().colizig_hip_predictor_predict(h, layer, out.ctypes.data, k)
    assert n >= 0
    return out[:n].tolist()


def _record(h, layer, ids):
    a = np.asarray(ids, np.uint32)
    assert _lib.hip().colizig_hip_predictor_record(h, layer, a.ctypes.data, len(ids)) == 0


def test_last_token_predictor_tracks_pattern():
    """predict.zig:94-110: nothing predicted before the first record; the
    same routing twice scores 2/2, then a half change 1/2."""
    hip = _lib.hip()
    h = hip.colizig_hip_predictor_create(2)
    try:
        assert _predict(h, 0) == []
        _record(h, 0, [5, 9])
        assert _predict(h, 0) == [5, 9]
        _record(h, 0, [5, 9])
        _record(h, 0, [5, 3])
        p, c = ctypes.c_uint64(), ctypes.c_uint64()
        assert hip.colizig_hip_predictor_stats(h, ctypes.byref(p), ctypes.byref(c)) == 0
        assert (p.value, c.value) == (6, 3)
        assert 0.4 < c.value / p.value < 0.6
        assert _predict(h, 1) == []  # layers are independent
    finally:
        hip.colizig_hip_predictor_destroy(h)


def test_last_token_predictor_keeps_topk():
    """predict.zig:84-89: at most topk ids are kept per layer."""
    hip = _lib.hip()
    h = hip.colizig_hip_predictor_create(3)
    try:
        _record(h, 1, [1, 2, 3, 4, 5])
        assert _predict(h, 1) == [1, 2, 3]
    finally:
        hip.colizig_hip_predictor_destroy(h)


class PrefetchPrediction(ctypes.Structure):
    _fields_ = [("layer", ctypes.c_uint32), ("expert", ctypes.c_uint32), ("confidence", ctypes.c_float),
                ("expected_use_distance", ctypes.c_uint32)]


def _scored(h, layer, k):
    rows = (PrefetchPrediction * k)()
    n = _lib.hip().colizig_hip_predictor_predict_scored(h, layer, rows, k)
    assert n >= 0
    return [(r.layer, r.expert, r.confidence, r.expected_use_distance) for r in rows[:n]]


def test_predict_scored_rows():
    """predict.zig:112-124 restated: after recording [1, 2, 3] at layer 1
    with topk 3, predictScored gives three rows for layer 1, row 1 naming
    expert 2.  The confidence is the accuracy so far with a floor of 0.1
    (predict.zig:63), the expected use distance 1, and a short buffer takes
    the first rows only."""
    hip = _lib.hip()
    h = hip.colizig_hip_predictor_create(3)
    try:
        _record(h, 1, [1, 2, 3])
        rows = _scored(h, 1, 3)
        assert len(rows) == 3
        assert rows[0][0] == 1 and rows[1][1] == 2
        assert [r[1] for r in rows] == [1, 2, 3]
        # nothing scored yet (the first record had no prediction): accuracy 0 -> the 0.1 floor
        assert all(abs(r[2] - np.float32(0.1)) == 0 and r[3] == 1 for r in rows)
        assert _scored(h, 0, 3) == []  # no prediction for layer 0
        assert len(_scored(h, 1, 2)) == 2
        # every recorded id counts as predicted, the first record's three
        # included (predict.zig:79-88): 2 right of 6 -> accuracy 1/3
        _record(h, 1, [1, 2, 7])
        rows = _scored(h, 1, 3)
        assert [r[1] for r in rows] == [1, 2, 7]
        assert all(r[2] == np.float32(2.0 / 6.0) for r in rows)
        assert hip.colizig_hip_predictor_predict_scored(987654321, 1, None, 0) == -1
    finally:
        hip.colizig_hip_predictor_destroy(h)
