"""Host logic of the engine adapter: the condensed slot table."""

from __future__ import annotations

import random

import pytest

from suffixgpu_amd.adapter import SlotTable


def _apply(rows, moves, n_left):
    rows = list(rows)
    for src, dst in moves:
        rows[dst] = rows[src]
    return rows[:n_left]


def test_slots_condense_like_a_persistent_batch():
    t = SlotTable(8)
    for r in "abcde":
        t.add(r)
    moves = t.remove(["b", "d"])
    assert moves == [(4, 1)]
    assert t.req_at == ["a", "e", "c"]
    assert t.slot_of == {"a": 0, "e": 1, "c": 2}
    assert t.add("f") == 3
    moves = t.remove(["a", "f"])
    assert moves == [(2, 0)]
    assert t.req_at == ["c", "e"]
    assert t.remove(["c", "e"]) == []
    assert len(t) == 0


def test_slot_errors():
    t = SlotTable(2)
    t.add(1)
    with pytest.raises(KeyError):
        t.add(1)
    t.add(2)
    with pytest.raises(RuntimeError):
        t.add(3)
    with pytest.raises(KeyError):
        t.remove([3])


def test_slot_moves_replay_the_table_randomly():
    """Replaying the returned moves on a copy of the rows, in order, always
    gives the table's new order (the device copies the rows this way)."""
    rng = random.Random(5)
    t = SlotTable(16)
    rows = []
    nxt = 0
    for _ in range(400):
        if len(t) < 16 and rng.random() < 0.55:
            t.add(nxt)
            rows.append(nxt)
            nxt += 1
        elif len(t):
            k = rng.randint(1, len(t))
            gone = rng.sample(t.req_at, k)
            moves = t.remove(gone)
            rows = _apply(rows, moves, len(t))
        assert rows == t.req_at
        assert all(t.slot_of[r] == i for i, r in enumerate(t.req_at))
