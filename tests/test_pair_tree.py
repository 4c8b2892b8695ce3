"""A model of the dot2 kernel's split-K pair tree (pair_tree_sum in
se12_device.hpp) run on the CPU: the S partial sums of one output meet in a
fixed binary tree of 64-bit slots, each pair through one exchange whose first
arriver parks (1 << 32) | bits and whose second takes them back, adds and
clears the slot. Under any interleaving of the splits' exchanges exactly one
split ends with the total, its bits never depend on the order of arrival,
every slot a launch fills is clear again at its end, and the tree uses S - 1
slots (the handle allocates (S - 1) x batch rows x padded rows)."""

from __future__ import annotations

import random

import numpy as np
import pytest


def walk(s: int, S: int):
    """The slots split s exchanges in, level by level, with its side (0 =
    the pair's even member), as the device loop visits them; ends with the
    node count of the whole tree."""
    c, n, node = s, S, 0
    steps = []
    while n > 1:
        if (c ^ 1) < n:
            steps.append((node + (c >> 1), c & 1))
        node += n >> 1
        c >>= 1
        n = (n + 1) >> 1
    return steps, node


def run(partials: np.ndarray, rng: random.Random):
    """Every split walks the tree; each step of a random split is one
    exchange. Returns (holder, total bits, slots left non-zero)."""
    S = len(partials)
    slots: dict[int, int] = {}
    state = {s: (0, np.float32(partials[s])) for s in range(S)}  # split -> (next step, value)
    plans = {s: walk(s, S)[0] for s in range(S)}
    holders = []
    while state:
        s = rng.choice(sorted(state))
        i, v = state.pop(s)
        if i == len(plans[s]):
            holders.append((s, v))
            continue
        slot, odd = plans[s][i]
        old = slots.get(slot, 0)
        slots[slot] = (1 << 32) | int(v.view(np.uint32))
        if old == 0:
            continue  # parked: the sibling adds
        o = np.uint32(old & 0xFFFFFFFF).view(np.float32)
        v = np.float32(o + v) if odd else np.float32(v + o)
        slots[slot] = 0
        state[s] = (i + 1, v)
    assert len(holders) == 1
    return holders[0][0], int(holders[0][1].view(np.uint32)), [k for k, x in slots.items() if x]


@pytest.mark.parametrize("S", [2, 3, 4, 5, 6, 7, 8, 9, 13, 16, 36, 64])
def test_any_arrival_order_gives_the_same_bits_and_clears_every_slot(S):
    rng = random.Random(S)
    partials = (np.random.default_rng(S).standard_normal(S) * np.float32(1e3)).astype(np.float32)
    results = set()
    for _ in range(60):
        holder, bits, left = run(partials, rng)
        assert left == []
        results.add(bits)
    assert len(results) == 1
    total = np.uint32(results.pop()).view(np.float32)
    assert abs(float(total) - float(partials.astype(np.float64).sum())) <= 1e-4 * float(np.abs(partials).sum())


@pytest.mark.parametrize("S", range(1, 65))
def test_tree_has_s_minus_1_slots_reached_from_both_sides(S):
    uses: dict[tuple[int, int], int] = {}
    for s in range(S):
        steps, nodes = walk(s, S)
        assert nodes == S - 1
        for slot, odd in steps:
            assert 0 <= slot < S - 1
            uses[(slot, odd)] = uses.get((slot, odd), 0) + 1
    # every slot lies on some split's path, from both sides
    assert sorted({slot for slot, _ in uses}) == list(range(S - 1))
    assert all((slot, 0) in uses and (slot, 1) in uses for slot in range(S - 1))


def test_two_splits_sum_in_either_order():
    a, b = np.float32(0.1), np.float32(1e8)
    assert np.float32(a + b).view(np.uint32) == np.float32(b + a).view(np.uint32)
    for seed in range(10):
        _, bits, _ = run(np.array([a, b], dtype=np.float32), random.Random(seed))
        assert bits == int(np.float32(a + b).view(np.uint32))
