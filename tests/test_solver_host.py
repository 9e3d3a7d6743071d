"""CPU checks of the solver's host-side planning: the request-group split (cost-balanced, every
request exactly once) and the capacity buckets that let one captured solve graph serve many
layouts.  No kernel runs here."""

from __future__ import annotations

import itertools
import random

import pytest


def _cost(n: int) -> int:
    # the split's per-request cost, 378 MFLOP x L + 90 kFLOP x L^2, in units of 90 kFLOP
    return n * n + 4200 * n


def test_request_groups_cover_every_request_once(fcv):
    rng = random.Random(0)
    for trial in range(200):
        n = rng.randint(1, 40)
        lengths = [rng.randint(1, 3000) for _ in range(n)]
        for n_groups in (1, 2, 3, 4, 8):
            groups = fcv.solver.request_groups(lengths, n_groups)
            flat = [i for g in groups for i in g]
            assert sorted(flat) == list(range(n))
            assert all(g == sorted(g) and g for g in groups)
            assert len(groups) == min(n_groups, n)


def test_request_groups_balance_matches_brute_force_bound(fcv):
    # longest-first onto the least loaded group is within 4/3 of the best two-way split
    rng = random.Random(1)
    for trial in range(100):
        lengths = [rng.randint(50, 1500) for _ in range(rng.randint(2, 10))]
        groups = fcv.solver.request_groups(lengths, 2)
        worst = max(sum(_cost(lengths[i]) for i in g) for g in groups)
        best = min(
            max(sum(_cost(lengths[i]) for i in range(len(lengths)) if (mask >> i) & 1),
                sum(_cost(lengths[i]) for i in range(len(lengths)) if not (mask >> i) & 1))
            for mask in range(1 << len(lengths)))
        assert worst <= best * 4 / 3 + 1e-9


def test_request_groups_config3_split(fcv):
    # the bench workload's draw: the 1291-frame request with the four shortest (2307 rows per
    # CFG half), the next three together (2285)
    lengths = [1291, 992, 816, 477, 531, 157, 205, 123]
    assert fcv.solver.request_groups(lengths, 2) == [[0, 4, 5, 6, 7], [1, 2, 3]]


def test_default_concurrency(fcv):
    assert fcv.solver.default_concurrency(1) == 1
    assert all(fcv.solver.default_concurrency(n) == 2 for n in (2, 8, 64))


@pytest.mark.parametrize("rows", [1, 255, 256, 257, 300, 511, 512, 513, 1100, 4614, 9184, 123698])
def test_capacity_bucket_bounds(fcv, rows):
    cap, docs = fcv.solver.capacity_bucket(rows, 3)
    assert cap >= rows and cap >= 256
    # m * 2^e with m in 8..15: at most 12.5 % above the rows (past the 256-row floor)
    e = cap.bit_length() - 4
    assert cap % (1 << max(e, 0)) == 0 and 8 <= cap >> max(e, 0) <= 16
    if rows > 256:
        assert cap <= rows * 9 / 8 + 1
    assert docs == 4


def test_capacity_bucket_is_idempotent_and_monotonic(fcv):
    prev = 0
    for rows, nd in itertools.product(range(1, 6000, 37), (1, 2, 5, 16, 17)):
        cap, docs = fcv.solver.capacity_bucket(rows, nd)
        assert fcv.solver.capacity_bucket(cap, docs) == (cap, docs)
        assert docs >= max(nd, 2) and docs & (docs - 1) == 0 and docs < 2 * max(nd, 2)
        if nd == 1:
            assert cap >= prev
            prev = cap
