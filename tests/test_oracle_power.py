"""The GPU parity tests can tell a wrong attention from a right one.

Each mistake is planted in the oracle, on the CPU, and run on exactly the weights and inputs a
GPU parity test uses (``tests/recipes.py``).  A test has power against a mistake when the
mistake moves the oracle's velocity by at least 5x the tolerance that test holds the GPU
kernels to (``VEL_TOL``), so a kernel with that mistake fails it by a wide margin:

* no RoPE, and RoPE with the rotation reversed (head 0's interleaved pairs);
* RoPE angles frozen past position max_pos/2 (a table indexing bug that only long documents
  would show);
* a uniform softmax (every visible key weighted equally);
* the chunk-causal boundary moved by one frame.

The 2-block recipe's long document is there for RoPE at high positions; its power is measured
on that document's rows, which its GPU test checks on their own.  Its chunk-boundary mutant
moves the velocity by only ~2x the tolerance, so the chunk rule is held to the 5x bar by the
22-block recipe, whose attention effects accumulate over 22 blocks.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import dit_oracle as O
from tests import recipes

POWER = 5.0


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


_rotary = O.apply_rotary
_freqs = O.rotary_freqs
_sdpa = F.scaled_dot_product_attention
_chunk_mask = O.subsequent_chunk_mask


def _plant(monkeypatch, mutant: str) -> None:
    if mutant == "no_rope":
        monkeypatch.setattr(O, "apply_rotary", lambda x, f: x)
    elif mutant == "reversed_rope":
        monkeypatch.setattr(O, "apply_rotary", lambda x, f: _rotary(x, -f))
    elif mutant == "rope_frozen_past_half":
        half = recipes.MAX_POS // 2
        monkeypatch.setattr(O, "rotary_freqs",
                            lambda pos, d=64: _freqs(pos.clamp(max=half - 1), d))
    elif mutant == "uniform_softmax":
        monkeypatch.setattr(O.F, "scaled_dot_product_attention",
                            lambda q, k, v, attn_mask=None, **kw: _sdpa(q * 0, k, v,
                                                                        attn_mask=attn_mask, **kw))
    elif mutant == "chunk_shift":
        monkeypatch.setattr(O, "subsequent_chunk_mask",
                            lambda size, c: _chunk_mask(size + 1, c)[1:, 1:])
    else:
        raise ValueError(mutant)


CASES = [
    ("sharp22", False, ["no_rope", "reversed_rope", "uniform_softmax"]),
    ("sharp22", True, ["no_rope", "reversed_rope", "uniform_softmax", "chunk_shift"]),
    ("sharp2_max_pos", False, ["no_rope", "reversed_rope", "rope_frozen_past_half",
                               "uniform_softmax"]),
    ("sharp2_max_pos", True, ["no_rope", "reversed_rope", "rope_frozen_past_half",
                              "uniform_softmax"]),
]


def _case(fcv, name):
    """(weights, inputs, rows the power is measured on)."""
    if name == "sharp22":
        inputs = recipes.cfg_pair_inputs(fcv)
        return recipes.state_dict(fcv, recipes.SHARP22), inputs, slice(None)
    inputs = recipes.max_pos_inputs()
    return recipes.state_dict(fcv, recipes.SHARP2), inputs, recipes.long_doc_rows(inputs[-1])


@pytest.mark.parametrize("name,streaming,mutants", CASES,
                         ids=[f"{c[0]}-{'stream' if c[1] else 'full'}" for c in CASES])
def test_gpu_recipes_detect_attention_mistakes(fcv, monkeypatch, name, streaming, mutants):
    sd, (x, mu, cond, spks, t, lengths), rows = _case(fcv, name)
    run = lambda: O.dit_forward_packed(sd, x, mu, cond, spks, t, lengths,
                                       streaming=streaming)[rows]
    base = run()
    moved = {}
    for m in mutants:
        with monkeypatch.context() as mp:
            _plant(mp, m)
            moved[m] = _rel(run(), base)
    print(f"{name} streaming={streaming}: " + ", ".join(f"{k} {v:.2e}" for k, v in moved.items()))
    for m, v in moved.items():
        assert v >= POWER * recipes.VEL_TOL, f"{m} moves the velocity by only {v:.2e}"


def test_mutants_are_planted(fcv, monkeypatch):
    """Each planted mistake changes what the oracle computes (on a tiny case), so a mutant
    that silently did nothing cannot make the power test pass vacuously."""
    x = torch.randn(1, 5, 64)
    f = O.rotary_freqs(torch.arange(5))
    with monkeypatch.context() as mp:
        _plant(mp, "no_rope")
        assert torch.equal(O.apply_rotary(x, f), x)
    with monkeypatch.context() as mp:
        _plant(mp, "reversed_rope")
        assert not torch.allclose(O.apply_rotary(x, f), _rotary(x, f))
    with monkeypatch.context() as mp:
        _plant(mp, "chunk_shift")
        assert not torch.equal(O.subsequent_chunk_mask(120, 50), _chunk_mask(120, 50))
    with monkeypatch.context() as mp:
        _plant(mp, "rope_frozen_past_half")
        pos = torch.arange(recipes.MAX_POS)
        assert torch.equal(O.rotary_freqs(pos)[:2048], _freqs(pos)[:2048])
        assert not torch.equal(O.rotary_freqs(pos)[2048:], _freqs(pos)[2048:])
