"""GPU checks of the packed streaming Flow step (token2wav.py:154-226 over
flashinfer_flow.py:207-281): B = 1 vs B = N invariance end to end (front-end, chunk-causal
packed solve from the fixed noise prefix, Mel-cache bookkeeping) and a multi-chunk session
against the fp32 oracle pipeline (Mel rel-L2 <= 2e-2 after 10 Euler steps)."""

from __future__ import annotations

import copy
from types import SimpleNamespace

import pytest
import torch

from oracle import dit_oracle as O
from oracle import frontend_oracle as F
from tests.gpu_helpers import make_estimator, rel_l2, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.fixture(scope="module")
def flow2(fcv):
    """Front-end at full shape + a 2-block full-width DiT with nonzero gates + fixed noise."""
    fdims = fcv.synthetic.FlowDims()
    fsd = fcv.synthetic.random_flow_state_dict(fdims, seed=41)
    fe = fcv.FlowFrontEnd(device="cuda:0")
    fe.load_reference_state_dict(fsd)
    fe.finalize_weights()
    dsd = fcv.synthetic.random_state_dict(fcv.synthetic.DiTDims(depth=2), seed=42, gate_bias=0.5)
    fe.decoder = fcv.CFMDecoder(make_estimator(fcv, dsd, depth=2), noise_seed=43)
    return fsd, dsd, fe


def _session(g, prompt_tokens: int, tokens: int):
    cond = SimpleNamespace(
        prompt_tokens_flow=torch.randint(0, 6561, (prompt_tokens,), generator=g).tolist(),
        prompt_feat=torch.randn(1, 2 * prompt_tokens, 80, generator=g),
        spk_embedding=torch.randn(192, generator=g))
    return SimpleNamespace(cond=cond, tokens=torch.randint(0, 6561, (tokens,), generator=g).tolist(),
                           mel_cache=None, speech_offset=0, chunk_index=0)


def test_stream_step_batched_equals_sessions_alone(fcv, flow2):
    """Five sessions at different prefixes (first hop with prompt padding, later hops, a final
    chunk): packed together or one at a time, every session's new Mel frames and cache are
    bit-identical."""
    _, _, fe = flow2
    g = torch.Generator().manual_seed(44)
    sessions = [_session(g, p, n) for p, n in ((0, 40), (13, 60), (25, 90), (7, 33), (40, 120))]
    plans = [SimpleNamespace(prefix_len=18, token_offset=0, finalize=False),
             SimpleNamespace(prefix_len=35, token_offset=2, finalize=False),
             SimpleNamespace(prefix_len=63, token_offset=30, finalize=False),
             SimpleNamespace(prefix_len=33, token_offset=20, finalize=True),
             SimpleNamespace(prefix_len=120, token_offset=75, finalize=True)]
    alone_sessions = copy.deepcopy(sessions)
    sf = fcv.StreamingFlow(fe)
    say("[stream] packed step, 5 sessions")
    packed = sf.stream_step_batched(sessions, plans)
    for i, (s, p) in enumerate(zip(alone_sessions, plans)):
        say(f"[stream] session {i} alone")
        alone = sf.stream_step(s, p)
        lookahead = 0 if p.finalize else 3
        want = 2 * (p.prefix_len - lookahead - p.token_offset)
        assert packed[i].shape == (1, 80, want)
        assert torch.equal(packed[i], alone), f"session {i} differs between B=1 and B=5"
        assert torch.equal(sessions[i].mel_cache, s.mel_cache)


def test_stream_chunks_match_oracle(fcv, flow2):
    """Three consecutive chunks of one session (15+pad, 30, then the final remainder); each
    step's full-prefix Mel against the oracle pipeline: per-stream token features, prompt
    condition, fixed-noise prefix, chunk-causal fp32 DiT, CFG Euler."""
    fsd, dsd, fe = flow2
    g = torch.Generator().manual_seed(45)
    s = _session(g, 11, 80)
    sf = fcv.StreamingFlow(fe)
    plans = [SimpleNamespace(prefix_len=19 + 3, token_offset=0, finalize=False),
             SimpleNamespace(prefix_len=49 + 3, token_offset=19, finalize=False),
             SimpleNamespace(prefix_len=80, token_offset=49, finalize=True)]
    spk = F.speaker_projection(s.cond.spk_embedding[None], fsd["spk_embed_affine_layer.weight"],
                               fsd["spk_embed_affine_layer.bias"])

    def oracle_est(x, mask, mu, t, spks, cond, streaming):
        return O.dit_forward(dsd, x, mask, mu, t, spks, cond, streaming=streaming)

    for k, p in enumerate(plans):
        say(f"[stream] chunk {k}: prefix {p.prefix_len}, finalize {p.finalize}")
        new = sf.stream_step(s, p)
        toks = s.cond.prompt_tokens_flow + s.tokens[:p.prefix_len]
        mu = F.streaming_token_features(fsd, toks, p.finalize)  # [1, Tm, 80]
        tm = mu.shape[1]
        plen = s.cond.prompt_feat.shape[1]
        cond = torch.zeros(1, tm, 80)
        cond[0, :plen] = s.cond.prompt_feat[0]
        noise = fe.decoder.rand_noise[:, :, :tm].float()
        ref = O.solve_euler_batched(oracle_est, noise, mu.transpose(1, 2), torch.ones(1, 1, tm),
                                    spk, cond.transpose(1, 2), n_steps=10, cfg_rate=0.7,
                                    streaming=True)
        want = ref[:, :, plen + 2 * p.token_offset:]
        assert new.shape == want.shape
        err = rel_l2(new.cpu(), want)
        say(f"[stream] chunk {k} new Mel rel_l2 {err:.2e}")
        assert err <= 2e-2
    assert s.mel_cache.shape == (1, 80, 2 * 80) and s.chunk_index == 3


def test_stream_step_vocodes_sessions_in_one_packed_call(fcv, flow2):
    """With HiFTVocoder.inference as the vocoder, a packed step vocodes every session's Mel
    cache in one call; the PCM equals vocoding each session on its own (a plain callable), bit
    for bit, over two consecutive chunks."""
    _, _, fe = flow2
    dims = fcv.synthetic.HiFTDims()
    voc = fcv.HiFTVocoder(dims, device="cuda:0",
                          buffers=fcv.synthetic.random_hift_buffers(dims, max_samples=480 * 400,
                                                                    seed=46))
    voc.load_reference_state_dict(fcv.synthetic.random_hift_state_dict(dims, seed=47))
    voc.finalize_weights()
    g = torch.Generator().manual_seed(48)
    sessions = [_session(g, p, n) for p, n in ((0, 60), (12, 80), (30, 50))]
    alone = copy.deepcopy(sessions)
    packed_sf = fcv.StreamingFlow(fe, vocoder=voc.inference)
    plain_sf = fcv.StreamingFlow(fe, vocoder=lambda speech_feat, finalize:
                                 voc.inference(speech_feat, finalize))
    steps = [[SimpleNamespace(prefix_len=21, token_offset=0, finalize=False)] * 3,
             [SimpleNamespace(prefix_len=51, token_offset=18, finalize=False),
              SimpleNamespace(prefix_len=80, token_offset=18, finalize=True),
              SimpleNamespace(prefix_len=50, token_offset=18, finalize=True)]]
    for k, plans in enumerate(steps):
        say(f"[stream+hift] step {k}")
        pcm = packed_sf.stream_step_batched(sessions, plans)
        for i, (s, p) in enumerate(zip(alone, plans)):
            ref = plain_sf.stream_step(s, p)
            assert pcm[i].shape == ref.shape and pcm[i].shape[1] > 0
            assert torch.equal(pcm[i], ref), f"session {i} step {k}"
            assert sessions[i].speech_offset == s.speech_offset
