"""GPU parity of the HIP estimator against the fp32 CPU oracle and the reference golden vectors.

Tolerances: per-step velocity rel-L2 <= 1e-2 vs the fp32 path, mel rel-L2 <= 2e-2 after 10
Euler steps.  Where the oracle is given the same fp16-rounded
weights the GPU uses, the remaining error is activation rounding only and the bound is tighter.
"""

from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import dit_oracle as O
from tests import recipes
from tests.gpu_helpers import (f16_weights, make_estimator, oracle_packed, random_packed, rel_l2,
                               say)

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
VEL_TOL = 1e-2        # per-step velocity vs the fp32 reference path
F16_W_TOL = 5e-3      # vs the oracle running on the same fp16-rounded weights


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(scope="module")
def stress2(fcv):
    """Two blocks at full width with AdaLN gates pushed to ~0.5 so every block matters."""
    dims = fcv.synthetic.DiTDims(depth=2)
    sd = fcv.synthetic.random_state_dict(dims, seed=21, gate_bias=0.5)
    return sd, make_estimator(fcv, sd, depth=2)


@pytest.mark.parametrize("streaming", [False, True])
def test_one_block_300_frames(fcv, streaming):
    """Workload 1 shape (one block, 300 frames) with nonzero gates."""
    dims = fcv.synthetic.DiTDims(depth=1)
    sd = fcv.synthetic.random_state_dict(dims, seed=1, gate_bias=0.5)
    est = make_estimator(fcv, sd, depth=1)
    x, mu, cond, spks, t = random_packed([300], seed=1)
    say(f"[one_block] streaming={streaming}")
    v = est.forward_packed(x, mu, cond, spks, t, [300], streaming=streaming).cpu()
    ref32 = oracle_packed(sd, x, mu, cond, spks, t, [300], streaming)
    ref16 = oracle_packed(f16_weights(sd), x, mu, cond, spks, t, [300], streaming)
    e32, e16 = rel_l2(v, ref32), rel_l2(v, ref16)
    say(f"[one_block] rel_l2 vs fp32 {e32:.2e}, vs fp16-weight oracle {e16:.2e}")
    assert e32 <= VEL_TOL and e16 <= F16_W_TOL


@pytest.mark.parametrize("streaming", [False, True])
def test_reference_golden_block(fcv, streaming):
    """GPU forward on the reference DiT's own outputs (tests/golden/block1024.npz)."""
    g = dict(np.load(GOLDEN / "block1024.npz", allow_pickle=False))
    dims = fcv.synthetic.DiTDims(depth=1)
    sd = fcv.synthetic.random_state_dict(dims, seed=int(g["weight_seed"]),
                                         gate_bias=float(g["gate_bias"]))
    est = make_estimator(fcv, sd, depth=1, static_chunk_size=int(g["chunk"]))
    dev = "cuda:0"
    args = [torch.from_numpy(g[k]).to(dev) for k in ("x", "mask", "mu", "t", "spks", "cond")]
    out = est(*args, streaming=streaming).cpu()
    ref = torch.from_numpy(g["out_stream" if streaming else "out_full"])
    err = rel_l2(out, ref)
    say(f"[golden_block] streaming={streaming} rel_l2 {err:.2e}")
    assert err <= VEL_TOL


@pytest.mark.parametrize("shared_t", [False, True])
@pytest.mark.parametrize("streaming", [False, True])
def test_ragged_docs_two_blocks(fcv, stress2, streaming, shared_t):
    """Ragged packing edge cases: a 1-frame doc, a doc of exactly one 128-row tile, docs that
    straddle tiles, chunk boundaries not aligned to tiles; one t per document and one shared
    t."""
    sd, est = stress2
    lengths = [37, 128, 1, 200, 75]
    x, mu, cond, spks, t = random_packed(lengths, seed=2)
    if shared_t:
        t = t[:1]
    v = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming).cpu()
    ref = oracle_packed(f16_weights(sd), x, mu, cond, spks, t, lengths, streaming)
    off = 0
    for n in lengths:
        e = rel_l2(v[off:off + n], ref[off:off + n])
        say(f"[ragged] streaming={streaming} shared_t={shared_t} len={n} rel_l2 {e:.2e}")
        assert e <= F16_W_TOL
        off += n


@pytest.mark.parametrize("streaming", [False, True])
def test_long_document(fcv, stress2, streaming):
    """One 2500-frame document next to a short one: 40 key tiles per query tile, the long-sequence
    regime of the 128-document workload, checked against the oracle directly."""
    sd, est = stress2
    lengths = [2500, 37]
    x, mu, cond, spks, t = random_packed(lengths, seed=13)
    say(f"[long_doc] streaming={streaming} GPU forward")
    v = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming).cpu()
    say(f"[long_doc] streaming={streaming} oracle forward")
    ref = oracle_packed(f16_weights(sd), x, mu, cond, spks, t, lengths, streaming)
    e_long, e_short = rel_l2(v[:2500], ref[:2500]), rel_l2(v[2500:], ref[2500:])
    say(f"[long_doc] streaming={streaming} rel_l2 long {e_long:.2e} short {e_short:.2e}")
    assert e_long <= F16_W_TOL and e_short <= F16_W_TOL


@pytest.mark.parametrize("streaming", [False, True])
def test_max_pos_document_among_many_tiny_ones(fcv, stress2, streaming):
    """Size limits: one document exactly as long as the RoPE tables (max_pos rows, so its last
    query reads the tables' last row; 4096 as in the reference's finalize_weights,
    flashinfer_dit.py:262-273) packed with 150 documents of 1..40 frames (150 entries in every
    per-document table, many one-tile documents, most shorter than one 50-frame chunk)."""
    sd, _ = stress2
    est = make_estimator(fcv, sd, depth=2, max_pos=4096)
    g = torch.Generator().manual_seed(17)
    tiny = torch.randint(1, 41, (150,), generator=g).tolist()
    lengths = tiny[:75] + [est.max_pos] + tiny[75:]
    x, mu, cond, spks, t = random_packed(lengths, seed=19)
    t = t[:1]  # one t for every document, as in a solver step
    say(f"[limits] streaming={streaming} {len(lengths)} docs, {sum(lengths)} rows, GPU forward")
    v = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming).cpu()
    say(f"[limits] streaming={streaming} oracle forward")
    ref = oracle_packed(f16_weights(sd), x, mu, cond, spks, t, lengths, streaming)
    off, worst = 0, 0.0
    for n in lengths:
        e = rel_l2(v[off:off + n], ref[off:off + n])
        worst = max(worst, e)
        assert e <= F16_W_TOL, f"document of {n} rows at row {off}: rel_l2 {e:.2e}"
        off += n
    say(f"[limits] streaming={streaming} worst per-document rel_l2 {worst:.2e}")


def test_concurrent_request_groups_equal_one_batch(fcv, stress2):
    """The solve's request groups (each a packed CFG batch on its own handle and stream, all
    in flight together) give the same rows as one packed batch, bit for bit: eager, first
    graph capture and replay, for 1, 2, 3 and the default number of groups."""
    _, est = stress2
    lengths = [90, 300, 17, 150, 64, 33]
    g = torch.Generator().manual_seed(23)
    rc = sum(lengths)
    noise, mu, cond = (torch.randn(rc, 80, generator=g) for _ in range(3))
    spks = torch.randn(len(lengths), 80, generator=g)
    solve = lambda c, graph: fcv.solve_euler_packed(est, noise, mu, cond, spks, lengths,
                                                    n_steps=3, use_graph=graph,
                                                    concurrency=c).cpu()
    ref = solve(1, False)
    for c in (2, 3, None):
        for graph in (False, True, True, True):
            say(f"[groups] concurrency={c} graph={graph}")
            assert torch.equal(solve(c, graph), ref), f"concurrency {c}, graph {graph}"
    assert fcv.solver.request_groups(lengths, 2) == [[1, 2], [0, 3, 4, 5]]


def test_shared_t_equals_per_doc_t(fcv, stress2):
    """One shared t against the same t repeated per document, for 2, 16 and 20 documents, bit
    for bit: a document's modulation row is the same whichever way it is computed, and the
    LayerNorm passes and gated residuals apply it the same way.  Per-document t values are then
    checked against themselves: reversing the documents (and their t) moves documents between
    the first and the second launch of the 16-row skinny product that computes the modulation
    rows, and every document's rows stay identical, so the rows past the first launch are
    indexed right; each document alone at its own t equals its rows of the per-document call."""
    sd, est = stress2
    g = torch.Generator().manual_seed(3)
    for n_docs in (2, 16, 20):
        lengths = torch.randint(1, 80, (n_docs,), generator=g).tolist()
        x, mu, cond, spks, _ = random_packed(lengths, seed=n_docs)
        say(f"[shared_t] {n_docs} documents")
        a = est.forward_packed(x, mu, cond, spks, torch.tensor([0.3]), lengths)
        b = est.forward_packed(x, mu, cond, spks, torch.full((n_docs,), 0.3), lengths)
        assert torch.equal(a, b), n_docs
    t = torch.rand(n_docs, generator=g)
    full = est.forward_packed(x, mu, cond, spks, t, lengths)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    order = list(reversed(range(n_docs)))
    pick = lambda a: torch.cat([a[cu[d]:cu[d + 1]] for d in order])
    rev = est.forward_packed(pick(x), pick(mu), pick(cond), spks[order], t[order],
                             [lengths[d] for d in order])
    assert torch.equal(rev, pick(full))
    for d, n in enumerate(lengths):
        alone = est.forward_packed(x[cu[d]:cu[d + 1]], mu[cu[d]:cu[d + 1]], cond[cu[d]:cu[d + 1]],
                                   spks[d:d + 1], t[d:d + 1], [n])
        assert torch.equal(alone, full[cu[d]:cu[d + 1]]), d


def test_layernorm_with_large_residual_mean(fcv):
    """A residual stream whose row mean is at least 20 times its spread (+20 on every bias of
    the second position-embedding conv: Mish of a large argument is that argument, so every
    row of the residual gains ~20 while its spread stays ~0.4; the ratio is measured on the
    oracle's input embedding below).  Each
    LayerNorm takes its statistics in fp32 from the fp32 residual and writes the normalized,
    modulated fp16 row, the tensor the reference itself materializes, so the mean costs no
    precision: the forward keeps the velocity bar against the fp32 oracle and the tighter bar
    against the fp16-weight oracle."""
    dims = fcv.synthetic.DiTDims(depth=2)
    sd = fcv.synthetic.random_state_dict(dims, seed=21, gate_bias=0.5)
    key = "input_embed.conv_pos_embed.conv2.0.bias"
    sd[key] = sd[key] + 20.0
    est = make_estimator(fcv, sd, depth=2)
    lengths = [200, 75, 31]
    x, mu, cond, spks, t = random_packed(lengths, seed=29)
    t = t[:1]
    h = O.input_embedding(sd, x[None, :200], cond[None, :200], mu[None, :200], spks[:1])[0]
    ratio = float((h.mean(-1).abs() / h.std(-1)).min())
    say(f"[large_mean] residual |mean| / spread after the input embedding: min {ratio:.1f}")
    assert ratio >= 20.0
    ref32 = oracle_packed(sd, x, mu, cond, spks, t, lengths)
    ref16 = oracle_packed(f16_weights(sd), x, mu, cond, spks, t, lengths)
    v = est.forward_packed(x, mu, cond, spks, t, lengths).cpu()
    e32, e16 = rel_l2(v, ref32), rel_l2(v, ref16)
    say(f"[large_mean] rel_l2 vs fp32 oracle {e32:.2e}, vs fp16-weight oracle {e16:.2e}")
    assert e32 <= VEL_TOL and e16 <= F16_W_TOL


def test_padded_dropin_collapses_equal_t(fcv, stress2):
    """The padded drop-in gets t of length 2B, all equal, from the packed solver
    (flashinfer_flow.py:53-57); it computes one modulation row and gives the rows of the
    packed call with a shared t, bit for bit, for 2B = 24 documents."""
    sd, est = stress2
    g = torch.Generator().manual_seed(9)
    lengths = torch.randint(8, 60, (24,), generator=g).tolist()
    T = max(lengths)
    x, mu, cond, spks, _ = random_packed(lengths, seed=10)
    pad = lambda rows: O.unpack(rows, lengths, T)
    mask = torch.zeros(24, 1, T)
    for b, n in enumerate(lengths):
        mask[b, 0, :n] = 1
    dev = "cuda:0"
    out = est(pad(x).to(dev), mask.to(dev), pad(mu).to(dev), torch.full((24,), 0.55, device=dev),
              spks.to(dev), pad(cond).to(dev)).cpu()
    packed = est.forward_packed(x, mu, cond, spks, torch.tensor([0.55]), lengths).cpu()
    assert torch.equal(O.pack(out, lengths), packed)


def test_solve_twenty_steps_equals_stepwise(fcv, stress2):
    """A 20-step solve reads the estimator's 20-step schedule, whose modulation rows come from
    two passes of the skinny product (steps 0-15, then 16-19).  Eager, on its first capture and
    on a replay, it gives bit for bit the sample of 20 single forwards (each computing its own
    shared-t modulation row) each followed by the CFG Euler update of the C ABI, with the same
    cosine schedule."""
    _, est = stress2
    b = fcv.synthetic.make_batch("steps20", [70, 33, 41], [20, 10, 15], seed=61)
    ts, dts = fcv.euler_schedule(20)
    rc = sum(b.lengths)
    inp = b.cfg_inputs()
    dev = "cuda:0"
    x = inp["x"].to(dev)
    lib = fcv._lib.load()
    say("[steps20] stepwise forwards")
    for i in range(20):
        v = est.forward_packed(x, inp["mu"], inp["cond"], inp["spks"], torch.tensor([ts[i]]),
                               b.doc_lengths)
        fcv._lib.check(lib.fcv_euler_cfg_step(est._require(), x.data_ptr(), v.data_ptr(), dts[i],
                                              0.7, est._stream_ptr()))
    want = x[:rc].cpu()
    for graph in (False, True, True):
        say(f"[steps20] solve use_graph={graph}")
        got = fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, n_steps=20,
                                     use_graph=graph, concurrency=1).cpu()
        assert torch.equal(got, want), graph


def _solve_unscheduled(fcv, est, b, n_steps):
    """The sample of fcv_dit_solve, the C ABI's solve that computes its own modulation rows in
    the loop (kModGroup steps per pass), eager, on an exact plan of the CFG layout."""
    lib = fcv._lib.load()
    dev = "cuda:0"
    inp = b.cfg_inputs()
    est.plan(b.doc_lengths)
    x, mu, cond, spks = (inp[k].to(dev).contiguous() for k in ("x", "mu", "cond", "spks"))
    ts, dts = fcv.euler_schedule(n_steps)
    t_arr = (fcv._lib.c_float * n_steps)(*ts)
    dt_arr = (fcv._lib.c_float * n_steps)(*dts)
    fcv._lib.check(lib.fcv_dit_solve(est._require(), x.data_ptr(), mu.data_ptr(),
                                     cond.data_ptr(), spks.data_ptr(), t_arr, dt_arr, n_steps,
                                     0.7, 0, est._stream_ptr()))
    torch.cuda.synchronize()
    return x[:sum(b.lengths)].cpu()


def test_shared_schedule_twenty_steps(fcv, stress2):
    """The solve schedule (fcv_dit_schedule, then fcv_dit_solve_scheduled on each group's
    handle): 20 steps, so the schedule holds rows past one 16-row pass of the skinny product.
    It is computed once per estimator and step count and reused by every later solve.  One,
    two and three groups give bit for bit the sample of fcv_dit_solve, which computes its own
    modulation rows, eagerly, on the first capture and on a replay; a schedule buffer too
    small for the step count is refused."""
    _, est = stress2
    b = fcv.synthetic.make_batch("sched20", [70, 33, 41, 90], [20, 10, 15, 30], seed=62)
    solve = lambda c, graph: fcv.solve_euler_packed(
        est, b.noise, b.mu, b.cond, b.spks, b.lengths, n_steps=20, use_graph=graph,
        concurrency=c).cpu()
    say("[sched20] fcv_dit_solve (modulation rows computed in the loop)")
    ref = _solve_unscheduled(fcv, est, b, 20)
    first = None
    for c in (1, 2, 3):
        for graph in (False, True, True):
            say(f"[sched20] groups={c} graph={graph}")
            assert torch.equal(solve(c, graph), ref), (c, graph)
            buf, _ = est._schedules[20]
            first = first or buf.data_ptr()
            assert buf.data_ptr() == first  # one schedule, computed by the first solve
    lib = fcv._lib.load()
    handle = est._require()
    small = lib.fcv_dit_schedule_bytes(handle, 10)
    assert 0 < small < lib.fcv_dit_schedule_bytes(handle, 20)
    assert lib.fcv_dit_schedule_bytes(handle, 65) == 0
    buf = torch.empty(small, dtype=torch.uint8, device="cuda:0")
    ts, dts = fcv.euler_schedule(20)
    t_arr = (fcv._lib.c_float * 20)(*ts)
    rc_code = lib.fcv_dit_schedule(handle, t_arr, 20, buf.data_ptr(), buf.numel(),
                                   torch.cuda.current_stream().cuda_stream)
    assert rc_code == fcv._lib.FCV_ERR_INVALID


@pytest.mark.parametrize("streaming", [False, True])
def test_peaked_attention_depth22(fcv, sharp22, streaming):
    """22 blocks on the peaked-attention recipe (q/k weights of deviation 0.06, gates +0.2):
    the 550-frame CFG pair against the fp32 oracle.  On these weights and inputs dropping or
    reversing RoPE, a uniform softmax or a chunk boundary one frame off moves the oracle
    velocity by 5-50x the tolerance (tests/test_oracle_power.py), so this bar pins the RoPE
    epilogue, the softmax and the chunk-causal mask."""
    sd, est = sharp22
    x, mu, cond, spks, t, lengths = recipes.cfg_pair_inputs(fcv)
    say(f"[peaked22] streaming={streaming} GPU forward")
    v = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming).cpu()
    say(f"[peaked22] streaming={streaming} oracle forward")
    ref = oracle_packed(sd, x, mu, cond, spks, t, lengths, streaming)
    err = rel_l2(v, ref)
    say(f"[peaked22] streaming={streaming} velocity rel_l2 vs fp32 oracle {err:.2e}")
    assert err <= recipes.PEAKED_TOL


@pytest.mark.parametrize("streaming", [False, True])
def test_peaked_attention_max_pos_document(fcv, streaming):
    """A document as long as the RoPE tables (4096 rows) between 24 short ones, 2 blocks on the
    peaked-attention recipe, against the fp32 oracle: the long document on its own (RoPE up to
    the tables' last row; dropping, reversing or freezing RoPE past row 2048 moves it by
    5-8x the tolerance) and the short documents together."""
    sd = recipes.state_dict(fcv, recipes.SHARP2)
    est = make_estimator(fcv, sd, depth=2, max_pos=recipes.MAX_POS)
    x, mu, cond, spks, t, lengths = recipes.max_pos_inputs()
    say(f"[peaked_max_pos] streaming={streaming} {len(lengths)} docs, GPU forward")
    v = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming).cpu()
    say(f"[peaked_max_pos] streaming={streaming} oracle forward")
    ref = oracle_packed(sd, x, mu, cond, spks, t, lengths, streaming)
    long = recipes.long_doc_rows(lengths)
    rest = torch.ones(v.shape[0], dtype=torch.bool)
    rest[long] = False
    e_long, e_rest = rel_l2(v[long], ref[long]), rel_l2(v[rest], ref[rest])
    say(f"[peaked_max_pos] streaming={streaming} rel_l2 long {e_long:.2e} short docs {e_rest:.2e}")
    assert e_long <= recipes.PEAKED_TOL and e_rest <= recipes.PEAKED_TOL


def test_padded_dropin_matches_packed(fcv, stress2):
    sd, est = stress2
    lengths, T = [64, 33, 50], 64
    x, mu, cond, spks, t = random_packed(lengths, seed=4)
    pad = lambda rows: O.unpack(rows, lengths, T)
    mask = torch.zeros(3, 1, T)
    for b, n in enumerate(lengths):
        mask[b, 0, :n] = 1
    dev = "cuda:0"
    out = est(pad(x).to(dev), mask.to(dev), pad(mu).to(dev), t.to(dev), spks.to(dev),
              pad(cond).to(dev)).cpu()
    packed = est.forward_packed(x, mu, cond, spks, t, lengths).cpu()
    assert torch.equal(O.pack(out, lengths), packed)
    for b, n in enumerate(lengths):
        assert torch.all(out[b, :, n:] == 0)


def test_solve_euler_batched_dropin(fcv, stress2):
    """The padded drop-in solver (signature of flashinfer_flow.py:16-74) gives the packed
    solve's rows on valid frames and leaves padded frames at their noise, as the reference
    does (its estimator returns zeros there, so dt * dphi is zero)."""
    sd, est = stress2
    b = fcv.synthetic.make_batch("dropin", [40, 25, 33], [10, 5, 8], seed=12)
    pad = b.padded()
    dev = "cuda:0"
    decoder = SimpleNamespace(estimator=est, inference_cfg_rate=0.7)
    out = fcv.solve_euler_batched(decoder, pad["noise"].to(dev), pad["mu"].to(dev),
                                  pad["mask"].to(dev), pad["spks"].to(dev), pad["cond"].to(dev),
                                  num_timesteps=4).cpu()
    ref = fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, n_steps=4).cpu()
    assert torch.equal(O.pack(out, b.lengths), ref)
    for i, n in enumerate(b.lengths):
        assert torch.equal(out[i, :, n:], pad["noise"][i, :, n:])


def test_apply_mi355x_installs_estimator(fcv, stress2):
    """apply_mi355x (the apply_flashinfer counterpart, flashinfer_dit.py:951-988) reads the
    replaced estimator's shape and state dict under the reference's names and installs an
    estimator that computes exactly what one built directly from that state dict computes."""
    sd, est = stress2

    class _Attn(torch.nn.Module):
        heads = 16

    class _Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = _Attn()

    class _ReferenceDiT(torch.nn.Module):
        static_chunk_size = 50

        def __init__(self):
            super().__init__()
            self.transformer_blocks = torch.nn.ModuleList([_Block() for _ in range(2)])
            self.proj_out = torch.nn.Linear(1024, 80, device="meta")

        def state_dict(self, *args, **kwargs):
            return dict(sd)

    model = SimpleNamespace(flow=SimpleNamespace(decoder=SimpleNamespace(
        estimator=_ReferenceDiT())))
    new = fcv.apply_mi355x(model)
    assert model.flow.decoder.estimator is new
    lengths = [60, 45]
    x, mu, cond, spks, t = random_packed(lengths, seed=8)
    assert torch.equal(new.forward_packed(x, mu, cond, spks, t, lengths),
                       est.forward_packed(x, mu, cond, spks, t, lengths))


def test_missing_inputs_raise(fcv, stress2):
    _, est = stress2
    x = torch.zeros(1, 80, 8, device="cuda:0")
    with pytest.raises(ValueError, match="spks and cond are required"):
        est(x, torch.ones(1, 1, 8, device="cuda:0"), x, torch.zeros(1, device="cuda:0"), None, x)


def test_batch_invariance_and_determinism(fcv, stress2):
    """A document's velocity does not depend on its neighbours (no split-KV, per-row GEMMs),
    and repeated calls are bit-identical (reference tests/gpu/test_stream_batched.py,
    test_stream_flashinfer.py:87-92)."""
    sd, est = stress2
    lengths = [90, 300, 17, 150]
    x, mu, cond, spks, _ = random_packed(lengths, seed=5)
    t = torch.tensor([0.42])
    for streaming in (False, True):
        full = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming)
        again = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming)
        assert torch.equal(full, again)
        off = 0
        for d, n in enumerate(lengths):
            alone = est.forward_packed(x[off:off + n], mu[off:off + n], cond[off:off + n],
                                       spks[d:d + 1], t, [n], streaming=streaming)
            assert torch.equal(alone, full[off:off + n]), (streaming, d)
            off += n


def test_every_gemm_tile_shape_gives_the_same_bits(fcv, stress2, monkeypatch):
    """The GEMM tile shape only decides which rows and columns share a workgroup, never an
    element's K order.  Forcing each of the eleven shapes (FCV_GEMM_TILE, wherever it divides
    the output width) reproduces the default choice bit for bit, with the full and the
    chunk-causal mask and with one shared t and one t per document."""
    sd, est = stress2
    lengths = [90, 300, 17, 150]
    x, mu, cond, spks, t_doc = random_packed(lengths, seed=8)
    for streaming in (False, True):
        for t in (torch.tensor([0.42]), t_doc):
            monkeypatch.delenv("FCV_GEMM_TILE", raising=False)
            ref = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming)
            for shape in range(11):
                say(f"[tiles] streaming={streaming} n_t={t.numel()} shape {shape}")
                monkeypatch.setenv("FCV_GEMM_TILE", str(shape))
                got = est.forward_packed(x, mu, cond, spks, t, lengths, streaming=streaming)
                assert torch.equal(got, ref), (streaming, t.numel(), shape)
    monkeypatch.delenv("FCV_GEMM_TILE", raising=False)


def test_streaming_prefix_stability_gate_a(fcv, stress2):
    """Reference Gate A (tests/gpu/test_flashinfer_streaming_estimator.py:58-89): with the
    chunk-causal mask the first floor(160/50)*50 frames of T=160 and T=200 agree; with full
    attention they do not."""
    _, est = stress2
    x, mu, cond, spks, t = random_packed([200], seed=6)
    t = torch.tensor([0.6])

    def run(T, streaming):
        return est.forward_packed(x[:T], mu[:T], cond[:T], spks, t, [T], streaming=streaming).cpu()

    stable = 150
    d_stream = (run(160, True)[:stable] - run(200, True)[:stable]).abs().max().item()
    d_off = (run(160, False)[:stable] - run(200, False)[:stable]).abs().max().item()
    say(f"[gate_a] stream diff {d_stream:.2e} offline diff {d_off:.2e}")
    assert d_stream <= 1e-3
    assert d_off > 1e-3


def test_full_depth_single_request(fcv, full22):
    """Workload 2: 22 layers, one request of 550 frames (prompt 250) as its CFG pair."""
    sd, est = full22
    b = fcv.synthetic.workload(2)
    inp = b.cfg_inputs()
    t = torch.tensor([b.t])
    say("[dit22] GPU forward")
    v = est.forward_packed(inp["x"], inp["mu"], inp["cond"], inp["spks"], t, b.doc_lengths).cpu()
    say("[dit22] oracle forward")
    ref = oracle_packed(sd, inp["x"], inp["mu"], inp["cond"], inp["spks"], t, b.doc_lengths)
    err = rel_l2(v, ref)
    say(f"[dit22] velocity rel_l2 vs fp32 oracle {err:.2e}")
    assert err <= VEL_TOL


def test_euler_solve_small_batch(fcv, full22):
    """10-step CFG Euler: per-step velocity (GPU estimator fed the oracle's trajectory) and the
    final mel of the GPU solve (graph and eager) against the fp32 oracle solve."""
    sd, est = full22
    b = fcv.synthetic.make_batch("small", [90, 61], [30, 20], seed=9)
    pad = b.padded()
    steps = []

    def oracle_est(x, mask, mu, t, spks, cond, streaming):
        return O.dit_forward(sd, x, mask, mu, t, spks, cond, streaming=streaming)

    def observe(step, velocity, sample):
        steps.append((step, sample.clone(), velocity.clone()))

    say("[euler] oracle solve")
    ref = O.solve_euler_batched(oracle_est, pad["noise"], pad["mu"], pad["mask"], pad["spks"],
                                pad["cond"], n_steps=10, cfg_rate=0.7, on_step=observe)
    ts, _ = fcv.euler_schedule(10)
    lengths = b.doc_lengths
    worst = 0.0
    for step, sample, velocity in steps:
        x_rows = torch.cat([O.pack(sample, b.lengths)] * 2)
        zeros = torch.zeros_like(b.mu)
        v = est.forward_packed(x_rows, torch.cat([b.mu, zeros]), torch.cat([b.cond, zeros]),
                               torch.cat([b.spks, torch.zeros_like(b.spks)]),
                               torch.tensor([ts[step - 1]]), lengths).cpu()
        vref = torch.cat([O.pack(velocity[:2], b.lengths), O.pack(velocity[2:], b.lengths)])
        worst = max(worst, rel_l2(v, vref))
    say(f"[euler] worst per-step velocity rel_l2 {worst:.2e}")
    assert worst <= VEL_TOL
    ref_rows = O.pack(ref, b.lengths)
    graph = fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, use_graph=True).cpu()
    eager = fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, use_graph=False).cpu()
    replay = fcv.solve_euler_packed(est, b.noise, b.mu, b.cond, b.spks, b.lengths, use_graph=True).cpu()
    err = rel_l2(graph, ref_rows)
    say(f"[euler] mel rel_l2 after 10 steps {err:.2e}")
    assert err <= 2e-2
    assert torch.equal(graph, eager) and torch.equal(graph, replay)
