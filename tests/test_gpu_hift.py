"""GPU parity of the HiFT vocoder (include/fcv_hift.h) against the oracle, whose wiring is pinned
to the reference generator's own outputs.

Tolerances: the vocoder computes in fp32 (F0 predictor in fp64), so the waveform is within
rel-L2 1e-4 of the fp32 oracle and the harmonic source within 1e-5 absolute; a request's
waveform is bit-identical alone and packed with others.
"""

from __future__ import annotations

import pytest
import torch

from oracle import hift_oracle as H
from tests.gpu_helpers import rel_l2, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(scope="module")
def hift(fcv):
    """The CosyVoice3 HiFT shape with seeded weights and a seeded 64-frame noise table."""
    dims = fcv.synthetic.HiFTDims()
    sd = fcv.synthetic.random_hift_state_dict(dims, seed=71)
    buf = fcv.synthetic.random_hift_buffers(dims, max_samples=480 * 64, seed=72)
    v = fcv.HiFTVocoder(dims, device="cuda:0", buffers=buf)
    v.load_reference_state_dict(sd)
    v.finalize_weights()
    return dims, H.fold_weight_norm(sd), buf, v


@pytest.mark.parametrize("finalize", [True, False])
def test_vocoder_matches_oracle(hift, finalize):
    dims, sd, buf, v = hift
    mel = torch.randn(1, 80, 40, generator=torch.Generator().manual_seed(73))
    say(f"[hift] 40 frames, finalize={finalize}")
    speech, s = v.inference(mel.cuda(), finalize=finalize)
    ref, ref_s = H.inference(sd, mel, buf, dims, finalize)
    assert speech.shape == ref.shape and s.shape == ref_s.shape
    es = float((s.cpu() - ref_s).abs().max())
    ew = rel_l2(speech.cpu(), ref)
    say(f"[hift] source max abs {es:.2e}, waveform rel_l2 {ew:.2e}")
    assert es <= 1e-5
    assert ew <= 1e-4


def test_long_requests_packed_match_oracle(fcv):
    """Three requests of 600-700 frames (12-14 s of audio each) in one packed call against the
    oracle run on each alone: the harmonic source phase reaches ~1e6 rad over such a request and
    is accumulated sequentially in the reference's fp32 order, so the source stays within 1e-5
    absolute and the waveform within rel-L2 1e-4 over the whole length."""
    dims = fcv.synthetic.HiFTDims()
    sd = fcv.synthetic.random_hift_state_dict(dims, seed=75)
    frames = (640, 700, 613)
    buf = fcv.synthetic.random_hift_buffers(dims, max_samples=480 * max(frames), seed=76)
    v = fcv.HiFTVocoder(dims, device="cuda:0", buffers=buf)
    v.load_reference_state_dict(sd)
    v.finalize_weights()
    folded = H.fold_weight_norm(sd)
    g = torch.Generator().manual_seed(77)
    mels = [torch.randn(80, n, generator=g) for n in frames]
    fin = [True, False, True]
    say(f"[hift long] packed call, {sum(frames)} frames")
    speech, source = v.inference_batched([m.cuda() for m in mels], fin, return_source=True)
    for i, (m, f) in enumerate(zip(mels, fin)):
        say(f"[hift long] oracle, request {i} ({m.shape[1]} frames, finalize={f})")
        ref, ref_s = H.inference(folded, m[None], buf, dims, f)
        assert speech[i].shape == ref.shape and source[i].shape == ref_s.shape
        es = float((source[i].cpu() - ref_s).abs().max())
        ew = rel_l2(speech[i].cpu(), ref)
        say(f"[hift long] request {i}: source max abs {es:.2e}, waveform rel_l2 {ew:.2e}")
        assert es <= 1e-5
        assert ew <= 1e-4


def test_packed_requests_equal_requests_alone(hift):
    """Three requests of different lengths, final and not: one packed call or one call each
    gives bit-identical waveforms."""
    _, _, _, v = hift
    g = torch.Generator().manual_seed(74)
    mels = [torch.randn(80, n, generator=g).cuda() for n in (9, 33, 21)]
    fin = [False, True, True]
    say("[hift] packed 3 requests")
    packed = v.inference_batched(mels, fin)
    for m, f, p in zip(mels, fin, packed):
        alone = v.inference_batched([m], [f])[0]
        assert p.shape == alone.shape == (1, v.output_samples(m.shape[1], f))
        assert torch.equal(p, alone)


def test_tile_size_does_not_change_the_waveform(hift, monkeypatch):
    """The conv kernel's 64x64 and 32x32 tiles (the second for launches too small to fill the
    CUs) sum every output in the same order: forcing either size (FCV_HIFT_TILE) reproduces
    the default call bit for bit, for a short streaming chunk and a packed pair (the fixture's
    noise table holds 64 frames of source per request)."""
    dims, sd, buf, v = hift
    g = torch.Generator().manual_seed(23)
    for frames, fin in (([60], [False]), ([40, 55], [True, False])):
        mels = [torch.randn(80, n, generator=g).to("cuda:0") for n in frames]
        monkeypatch.delenv("FCV_HIFT_TILE", raising=False)
        ref = v.inference_batched(mels, fin, graph=False)
        for size in ("32", "64"):
            say(f"[hift tiles] {frames} forced {size}")
            monkeypatch.setenv("FCV_HIFT_TILE", size)
            got = v.inference_batched(mels, fin, graph=False)
            assert all(torch.equal(a, b) for a, b in zip(got, ref)), (frames, size)
    monkeypatch.delenv("FCV_HIFT_TILE", raising=False)


def test_short_non_final_chunk_is_rejected(hift):
    _, _, _, v = hift
    with pytest.raises(ValueError):
        v.inference_batched([torch.zeros(80, 7, device="cuda")], [False])


def test_vocoder_graph_replays_new_layouts(fcv, hift):
    """Calls in one capacity bucket share one captured graph: a layout never seen before
    replays it with no new capture and gives bit for bit the eager call's waveforms and
    sources; a call in another bucket captures its own graph (the reference's per-bucket
    streaming vocoder graphs, hift_graph.py:65-169)."""
    _, _, _, v = hift
    g = torch.Generator().manual_seed(78)
    calls = {"A": ([40, 20], [False, True]), "B": ([30, 33], [True, False]),
             "C": ([9, 12, 20], [False, True, True])}
    mels = {k: [torch.randn(80, n, generator=g).cuda() for n in f] for k, (f, _) in calls.items()}
    cap = {k: fcv.hift.capacity_bucket(sum(f), len(f)) for k, (f, _) in calls.items()}
    assert cap["A"] == cap["B"] == (64, 2) and cap["C"] == (64, 4)
    run = lambda k, graph: v.inference_batched(mels[k], calls[k][1], return_source=True,
                                               concurrency=1, graph=graph)
    eager = {k: run(k, False) for k in calls}
    _, c0 = v.graph_stats()
    for name, captures in [("A", 0), ("A", 1), ("B", 1), ("C", 1), ("C", 2), ("B", 2), ("A", 2)]:
        say(f"[hift graph] call {name}")
        speech, source = run(name, True)
        assert all(torch.equal(a, b) for a, b in zip(speech, eager[name][0])), name
        assert all(torch.equal(a, b) for a, b in zip(source, eager[name][1])), name
        assert v.graph_stats()[1] - c0 == captures, name
