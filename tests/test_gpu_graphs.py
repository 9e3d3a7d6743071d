"""Capacity-bucketed solve graphs and the per-handle graph pool (fcv_dit_plan_capacity,
fcv_dit_solve; the reference's bucketed graph runners and plan pool, flashinfer_dit.py:143,
192-226,742-804).

A graph captured for a capacity replays for every other layout planned into it, with no new
capture, and gives bit for bit what an exact plan's eager solve gives; up to 4 captured
capacities alternate without re-capture."""

from __future__ import annotations

import pytest
import torch

from tests.gpu_helpers import make_estimator, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(scope="module")
def est2(fcv):
    sd = fcv.synthetic.random_state_dict(fcv.synthetic.DiTDims(depth=2), seed=91, gate_bias=0.5)
    return make_estimator(fcv, sd, depth=2)


def _solve(fcv, est, b, streaming, **kw):
    return fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, n_steps=3,
                                  streaming=streaming, concurrency=1, **kw).cpu()


@pytest.mark.parametrize("streaming", [False, True])
def test_one_graph_serves_every_layout_in_its_capacity(fcv, est2, streaming):
    mk = fcv.synthetic.make_batch
    batches = {
        "A": mk("A", [90, 61, 40], [30, 20, 10], seed=41),   # 382 CFG rows, 6 docs
        "B": mk("B", [70, 101, 11], [20, 40, 5], seed=42),   # 364 CFG rows, 6 docs
        "C": mk("C", [50, 50], [10, 20], seed=43),           # 200 CFG rows, 4 docs
    }
    cap = {k: fcv.solver.capacity_bucket(b.rows, 2 * b.n_requests) for k, b in batches.items()}
    assert cap["A"] == cap["B"] == (384, 8) and cap["C"] == (256, 4)
    say(f"[capacity] streaming={streaming}: exact-plan eager solves")
    exact = {k: _solve(fcv, est2, b, streaming, use_graph=False, bucketed=False)
             for k, b in batches.items()}
    _, c0 = est2.graph_stats()
    # (batch, captures expected after the solve): A's first solve runs eagerly, its second
    # captures the (384, 8) graph, which B then replays; C captures (256, 4) on its second solve
    sequence = [("A", 0), ("A", 1), ("B", 1), ("C", 1), ("C", 2), ("B", 2), ("A", 2), ("C", 2)]
    for name, captures in sequence:
        say(f"[capacity] streaming={streaming}: graph solve {name}")
        got = _solve(fcv, est2, batches[name], streaming, use_graph=True)
        assert torch.equal(got, exact[name]), name
        assert est2.graph_stats()[1] - c0 == captures, name


def test_graph_pool_keeps_four_capacities(fcv):
    """Five capacities, each captured on its second solve: the least recently used graph is
    dropped, the other four replay without re-capture, and every result equals the exact eager
    solve."""
    sd = fcv.synthetic.random_state_dict(fcv.synthetic.DiTDims(depth=2), seed=92, gate_bias=0.5)
    est2 = make_estimator(fcv, sd, depth=2)
    mk = fcv.synthetic.make_batch
    lens = [[20], [60, 60], [150, 30], [300, 120], [500, 200, 100]]
    batches = [mk(f"P{i}", n, [5] * len(n), seed=50 + i) for i, n in enumerate(lens)]
    caps = [fcv.solver.capacity_bucket(b.rows, 2 * b.n_requests) for b in batches]
    assert len(set(caps)) == 5
    exact = [_solve(fcv, est2, b, False, use_graph=False, bucketed=False) for b in batches]
    _, c0 = est2.graph_stats()
    for i, b in enumerate(batches):
        say(f"[pool] capacity {caps[i]}: first, second solve")
        assert torch.equal(_solve(fcv, est2, b, False, use_graph=True), exact[i])
        assert torch.equal(_solve(fcv, est2, b, False, use_graph=True), exact[i])
    pooled, c = est2.graph_stats()
    assert pooled == 4 and c - c0 == 5
    for i in (1, 2, 3, 4):  # still pooled: replays
        assert torch.equal(_solve(fcv, est2, batches[i], False, use_graph=True), exact[i])
    assert est2.graph_stats()[1] - c0 == 5
    # the first capacity was dropped: its next solve is its first sight again (eager)
    assert torch.equal(_solve(fcv, est2, batches[0], False, use_graph=True), exact[0])
    assert est2.graph_stats()[1] - c0 == 5
