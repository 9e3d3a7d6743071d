"""CPU checks of the streaming host logic (token2wav.py:188-226): chunk bookkeeping of the Mel
cache and PCM offsets, and argument validation.  No kernel runs here."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch


def _session():
    cond = SimpleNamespace(prompt_tokens_flow=[1, 2], prompt_feat=torch.zeros(1, 4, 80),
                           spk_embedding=torch.ones(192))
    return SimpleNamespace(cond=cond, tokens=list(range(40)), mel_cache=None, speech_offset=0,
                           chunk_index=0)


def _vocoder(speech_feat, finalize):
    # 4 samples per Mel frame, value = channel-0 Mel value: enough to check offsets
    return (speech_feat[:, 0, :].repeat_interleave(4, dim=1), None)


def test_finish_chunk_appends_new_frames_and_returns_new_pcm(fcv):
    fe = fcv.FlowFrontEnd(vocab_size=8, channels=128, device="cpu")
    sf = fcv.StreamingFlow(fe, vocoder=_vocoder)
    s = _session()
    full1 = torch.arange(10.0).view(1, 1, 10).expand(1, 80, 10)
    out1 = sf._finish_chunk(s, SimpleNamespace(token_offset=0, finalize=False), full1)
    assert s.mel_cache.shape == (1, 80, 10) and out1.shape == (1, 40) and s.speech_offset == 40
    # the next chunk recomputes the prefix; only frames past token_offset * 2 are appended
    full2 = 100 + torch.arange(30.0).view(1, 1, 30).expand(1, 80, 30)
    out2 = sf._finish_chunk(s, SimpleNamespace(token_offset=5, finalize=True), full2)
    assert s.mel_cache.shape == (1, 80, 30) and s.chunk_index == 2
    assert torch.equal(s.mel_cache[0, 0, :10], torch.arange(10.0))
    assert torch.equal(s.mel_cache[0, 0, 10:], 110 + torch.arange(20.0))
    assert out2.shape == (1, 80) and s.speech_offset == 120
    assert torch.equal(out2[0, :4], torch.full((4,), 110.0))


def test_finish_chunk_without_vocoder_returns_new_mel(fcv):
    fe = fcv.FlowFrontEnd(vocab_size=8, channels=128, device="cpu")
    sf = fcv.StreamingFlow(fe)
    s = _session()
    full = torch.randn(1, 80, 12)
    new = sf._finish_chunk(s, SimpleNamespace(token_offset=2, finalize=False), full)
    assert torch.equal(new, full[:, :, 4:]) and torch.equal(s.mel_cache, full[:, :, 4:])


def test_stream_step_batched_validates_arguments(fcv):
    fe = fcv.FlowFrontEnd(vocab_size=8, channels=128, device="cpu")
    sf = fcv.StreamingFlow(fe)
    with pytest.raises(ValueError):
        sf.stream_step_batched([_session()], [])
    with pytest.raises(ValueError):
        sf.stream_step_batched([], [])


def test_cfm_decoder_fixed_noise_is_seeded(fcv):
    a, b = fcv.CFMDecoder(None), fcv.CFMDecoder(None)
    assert a.rand_noise.shape == (1, 80, 15000) and torch.equal(a.rand_noise, b.rand_noise)
    assert not torch.equal(a.rand_noise, fcv.CFMDecoder(None, noise_seed=1).rand_noise)
