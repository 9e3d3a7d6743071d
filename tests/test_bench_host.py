"""Host logic of bench.py (no GPU): the streaming leg's chunk plans follow the reference
planner's rules (streaming/chunker.py:20-56).  The expected chunks are the known answers of the
reference's own planner tests (tests/test_chunker.py), read as one session whose tokens all
arrive before token2wav asks for them."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_module", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_aligned_prompt_hops_double_to_the_cap(bench):
    """A 75-token prompt needs no pad: boundaries 18, 48, 108, 168 (tests/test_chunker.py:6-20),
    then the remainder past the last full hop is one final chunk."""
    plans = bench.chunk_plans(75, 168)
    assert plans[:4] == [(18, 0, False), (48, 15, False), (108, 45, False), (168, 105, False)]
    assert plans[4:] == [(168, 165, True)]


def test_pad_applies_to_the_first_chunk_only(bench):
    """A 71-token prompt adds 4 alignment tokens to the first hop only
    (tests/test_chunker.py:23-32)."""
    assert bench.chunk_plans(71, 52)[:2] == [(22, 0, False), (52, 19, False)]


def test_remainder_is_one_final_chunk(bench):
    """tests/test_chunker.py:35-40: after one 15-token chunk, 20 tokens in all flush as
    (20, 15, final)."""
    assert bench.chunk_plans(75, 20) == [(18, 0, False), (20, 15, True)]
    assert bench.chunk_plans(0, 17) == [(17, 0, True)]  # too short for a first hop
    assert bench.chunk_plans(0, 0) == []                 # nothing to emit


def test_uniform_hops(bench):
    """chunk 25, scale 1 and a 71-token prompt: a 29-token first hop, then 25-token hops
    (tests/test_chunker.py:56-77)."""
    plans = bench.chunk_plans(71, 29 + 3 * 25 + 7, chunk=25, scale=1)
    assert plans[0] == (32, 0, False)
    assert plans[1:4] == [(29 + 25 * i + 28, 29 + 25 * i, False) for i in range(3)]
    assert plans[-1] == (29 + 3 * 25 + 7, 29 + 3 * 25, True)


def test_every_token_is_consumed_once(bench):
    """Each chunk starts where the previous one ended, reads at most the tokens it has, and
    the last one is final and ends at the session's last token."""
    for prompt in (0, 1, 14, 15, 16, 71, 300):
        for total in (1, 18, 19, 47, 48, 200, 777):
            plans = bench.chunk_plans(prompt, total)
            assert plans[-1][2] and plans[-1][0] == total
            assert all(not f for _, _, f in plans[:-1])
            done = 0
            for prefix, offset, final in plans:
                assert offset == done and prefix <= total
                done = prefix if final else prefix - 3
            assert done == total
