"""Packed streaming Flow steps on the MI355X path: the Flow half of
``CosyVoice3Token2Wav.stream_step`` / ``stream_step_batched`` / ``_finish_chunk``
(faster_cosyvoice/token2wav/token2wav.py:154-200, 203-226).

Sessions and plans are the reference's own objects, used by duck typing: a session has
``cond.prompt_tokens_flow``, ``cond.prompt_feat`` ``(1, P, 80)``, ``cond.spk_embedding``
``(192,)``, ``tokens``, ``mel_cache``, ``speech_offset``, ``chunk_index``
(streaming/session.py:18-27); a plan has ``prefix_len``, ``token_offset``, ``finalize``
(streaming/chunker.py:14-17).  Vocoding (HiFT) is not part of this path: pass the vocoder as a
callable with ``hift.inference``'s signature, or leave it out and receive each chunk's new Mel
frames instead of PCM.  When the vocoder is ``HiFTVocoder.inference``, a packed step vocodes
all of its sessions in one packed call.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from typing import Any

import torch

from .frontend import flow_inference_batched_streaming, frontend_for

NOISE_FRAMES = 50 * 300


class CFMDecoder:
    """The inference attributes of ``CausalConditionalCFM`` that the packed flow reads
    (flow_matching.py:199-200 and builders.py:22-28): the estimator, the CFG rate and the
    fixed noise prefix that keeps repeated full-prefix streaming deterministic."""

    def __init__(self, estimator: Any, inference_cfg_rate: float = 0.7,
                 rand_noise: torch.Tensor | None = None, noise_seed: int = 0):
        self.estimator = estimator
        self.inference_cfg_rate = inference_cfg_rate
        if rand_noise is None:
            g = torch.Generator().manual_seed(noise_seed)
            rand_noise = torch.randn([1, 80, NOISE_FRAMES], generator=g)
        self.rand_noise = rand_noise


class StreamingFlow:
    """``stream_step`` / ``stream_step_batched`` over the packed MI355X flow.

    ``flow``: a ``FlowFrontEnd`` with a ``decoder`` (``CFMDecoder``), or a reference flow whose
    decoder estimator was replaced by ``apply_mi355x``.  ``vocoder``: optional
    ``vocoder(speech_feat=mel, finalize=bool) -> (speech, ...)``."""

    def __init__(self, flow: Any, vocoder: Callable[..., Any] | None = None):
        self.flow = flow
        self.vocoder = vocoder
        self.token_mel_ratio = frontend_for(flow).token_mel_ratio

    def stream_step(self, session: Any, plan: Any) -> torch.Tensor:
        """One chunk of one session (token2wav.py:154-186): the packed path with B = 1."""
        return self.stream_step_batched([session], [plan])[0]

    @torch.no_grad()
    def stream_step_batched(self, sessions: Sequence[Any], plans: Sequence[Any]) -> list:
        """One packed Flow step across independent sessions (token2wav.py:203-226): each
        session's full token prefix, chunk-causal attention, then every session finishes its
        chunk in input order."""
        if len(sessions) != len(plans) or not sessions:
            raise ValueError("need one plan per session and at least one session")
        token_list = [list(s.cond.prompt_tokens_flow) + list(s.tokens[:p.prefix_len])
                      for s, p in zip(sessions, plans)]
        prompt_feat_list = [s.cond.prompt_feat for s in sessions]
        emb = torch.stack([torch.as_tensor(s.cond.spk_embedding).float() for s in sessions])
        finalize_list = [bool(p.finalize) for p in plans]
        mels = flow_inference_batched_streaming(self.flow, token_list, prompt_feat_list, emb,
                                                finalize_list)
        batched = getattr(self.vocoder, "__self__", None)
        if batched is not None and hasattr(batched, "inference_batched"):
            # a packed vocoder: every session's Mel cache in one call (same PCM as one call per
            # session, the vocoder being batch-invariant)
            for s, p, m in zip(sessions, plans, mels):
                self._append_mel(s, p, m)
            speech = batched.inference_batched([s.mel_cache for s in sessions], finalize_list)
            return [self._emit(s, sp) for s, sp in zip(sessions, speech)]
        return [self._finish_chunk(s, p, m) for s, p, m in zip(sessions, plans, mels)]

    def _append_mel(self, session: Any, plan: Any, mel_full: torch.Tensor) -> torch.Tensor:
        new_mel = mel_full[:, :, plan.token_offset * self.token_mel_ratio:]
        session.mel_cache = (new_mel if session.mel_cache is None
                             else torch.cat([session.mel_cache, new_mel], dim=2))
        session.chunk_index += 1
        return new_mel

    @staticmethod
    def _emit(session: Any, speech: torch.Tensor) -> torch.Tensor:
        new = speech[:, session.speech_offset:]
        session.speech_offset += new.shape[1]
        return new.cpu()

    def _finish_chunk(self, session: Any, plan: Any, mel_full: torch.Tensor) -> torch.Tensor:
        """Append the chunk's new Mel frames to the session cache (token2wav.py:188-200); with a
        vocoder, vocode the cache and return only the new PCM on the CPU, else return the new
        Mel frames ``(1, 80, n)``."""
        new_mel = self._append_mel(session, plan, mel_full)
        if self.vocoder is None:
            return new_mel
        speech = self.vocoder(speech_feat=session.mel_cache, finalize=plan.finalize)[0]
        return self._emit(session, speech)
