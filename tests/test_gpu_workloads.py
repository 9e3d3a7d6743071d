"""Parity at the full benchmark sizes, through properties that do not need a full-size oracle.

Workload 4 (32 streams, chunk-causal, 64 packed docs) and workload 5 (64 requests, full
attention, 128 packed docs, ~120 k rows) are too large for the fp32 CPU oracle, so each run is
checked by:
  * the hipGraph solve == the eager solve == a graph replay, bitwise (reference determinism
    gate, tests/gpu/test_stream_flashinfer.py:87-92);
  * batch invariance at full size: two requests solved on their own give bitwise the rows they
    get inside the full batch (tests/gpu/test_stream_batched.py:88-130);
  * the full-batch forward, restricted to the shortest request's CFG pair, against the fp32
    oracle run on that pair alone (velocity rel-L2 <= 1e-2).
"""

from __future__ import annotations

import pytest
import torch

from tests.gpu_helpers import oracle_packed, rel_l2, say

pytestmark = pytest.mark.gpu

VEL_TOL = 1e-2


def _rows(b, i):
    off = sum(b.lengths[:i])
    return slice(off, off + b.lengths[i])


@pytest.mark.parametrize("wl", [4, 5])
def test_full_size_workload(fcv, full22, wl):
    sd, est = full22
    b = fcv.synthetic.workload(wl)
    tag = f"[{b.name}]"
    say(f"{tag} {b.n_requests} requests, {len(b.doc_lengths)} docs, {b.rows} rows, "
        f"streaming={b.streaming}")

    solve = lambda graph, idx=None: fcv.solve_euler_packed(
        est,
        b.noise if idx is None else torch.cat([b.noise[_rows(b, i)] for i in idx]),
        b.mu if idx is None else torch.cat([b.mu[_rows(b, i)] for i in idx]),
        b.cond if idx is None else torch.cat([b.cond[_rows(b, i)] for i in idx]),
        b.spks if idx is None else b.spks[list(idx)],
        b.lengths if idx is None else [b.lengths[i] for i in idx],
        n_steps=b.n_steps, streaming=b.streaming, use_graph=graph).cpu()

    say(f"{tag} graph solve")
    graph = solve(True)
    say(f"{tag} eager solve")
    eager = solve(False)
    say(f"{tag} graph replay")
    replay = solve(True)
    assert torch.isfinite(graph).all()
    assert torch.equal(graph, eager) and torch.equal(graph, replay)

    # two requests on their own: the shortest and the longest
    i_short = min(range(b.n_requests), key=lambda i: b.lengths[i])
    i_long = max(range(b.n_requests), key=lambda i: b.lengths[i])
    say(f"{tag} batch invariance: requests {i_short} ({b.lengths[i_short]} frames) and "
        f"{i_long} ({b.lengths[i_long]} frames) alone")
    alone = solve(True, (i_short, i_long))
    n_s = b.lengths[i_short]
    assert torch.equal(alone[:n_s], graph[_rows(b, i_short)])
    assert torch.equal(alone[n_s:], graph[_rows(b, i_long)])

    # full-batch forward at the first step's t, shortest request's CFG pair vs the oracle
    say(f"{tag} full-batch forward")
    inp = b.cfg_inputs()
    t = torch.tensor([0.0])
    v = est.forward_packed(inp["x"], inp["mu"], inp["cond"], inp["spks"], t, b.doc_lengths,
                           streaming=b.streaming).cpu()
    rc = sum(b.lengths)
    r = _rows(b, i_short)
    v_pair = torch.cat([v[r], v[rc + r.start:rc + r.stop]])
    zeros = torch.zeros(n_s, 80)
    say(f"{tag} oracle forward of request {i_short} ({n_s} frames, CFG pair)")
    ref = oracle_packed(sd, torch.cat([b.noise[r], b.noise[r]]), torch.cat([b.mu[r], zeros]),
                        torch.cat([b.cond[r], zeros]),
                        torch.stack([b.spks[i_short], torch.zeros(80)]), t.expand(2),
                        [n_s, n_s], streaming=b.streaming)
    err = rel_l2(v_pair, ref)
    say(f"{tag} velocity rel_l2 vs fp32 oracle {err:.2e}")
    assert err <= VEL_TOL
